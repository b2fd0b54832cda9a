"""A chain of linears in one launch: the round's linears back to back, where a linear may read an
earlier one's output (``plm_gemm_chain_packed`` / ``plm_gemm_chain`` in ``include/plm_amd.h``).

The reference replays a round as a CUDA graph of separate ``fast_gemm`` launches, 4L+1 of them
(plm/decoder.py:312-324, plm/fast_gemm.py:82-97). On MI355X every launch pays a few microseconds
of start-up and tail in which HBM idles; a chain keeps one persistent grid streaming weights
across the linears. With packed weights (the default) the workgroups meet at a grid barrier after
each linear another one reads, with the next linear's first weights already requested; the
streaming kernel on row-major weights (``packed=False``) starts each tile of a linear as soon as
the producer tiles it reads are written.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .fast_gemm import (Config, HALF_DTYPES, _tile, packed_gate_up, packed_weight, reset_counters, row_major_weight,
                        workspace)


@dataclass
class Link:
    """One linear of a chain: ``y = x @ w.T``. ``dep`` is the index of the earlier link whose ``y``
    this ``x`` is (its leading ``K`` columns), or -1 when ``x`` comes from outside the chain.
    ``act`` (packed chains): ``w`` is a fused gate/up weight ``[2I, K]`` and ``y`` ``[M, I]`` gets
    ``silu(gate) * up`` (``fast_gemm.gate_up_silu``'s result); the chain's tile needs an even
    ``wave_frags``."""

    x: torch.Tensor
    w: torch.Tensor
    y: torch.Tensor
    dep: int = -1
    split_k: int = 1
    act: bool = False


class LinearChain:
    """Validated, prepared chain; ``run()`` launches it on the current stream (graph-capturable
    once constructed: the descriptor upload and workspace sizing happen here)."""

    def __init__(self, links: list[Link], cfg: Config, packed: bool = True):
        if not links:
            raise ValueError("a chain needs at least one linear")
        self.links = links
        self.cfg = dict(cfg)
        self.packed = packed
        x0 = links[0].x
        self.device = x0.device
        self.dtype = x0.dtype
        self.M = x0.shape[0]
        if self.dtype not in HALF_DTYPES:
            raise TypeError(f"chain operands must be bf16 or fp16, got {self.dtype}")
        arr = (_lib.ChainGemm * len(links))()
        for i, ln in enumerate(links):
            for name, t in (("x", ln.x), ("w", ln.w)):
                if t.dtype != self.dtype or t.device != self.device or t.dim() != 2 or t.stride(1) != 1:
                    raise ValueError(f"link {i}: {name} must be a row-major {self.dtype} matrix on {self.device}")
            if ln.x.shape[0] != self.M or ln.y.shape[0] != self.M or ln.x.shape[1] != ln.w.shape[1]:
                raise ValueError(f"link {i}: shapes x{tuple(ln.x.shape)} w{tuple(ln.w.shape)} y{tuple(ln.y.shape)}")
            cols = ln.w.shape[0] // 2 if ln.act else ln.w.shape[0]
            if ln.y.shape[1] != cols or ln.y.stride(1) != 1 or ln.y.device != self.device:
                raise ValueError(f"link {i}: y must be a row-major [{self.M},{cols}] matrix")
            if ln.y.dtype not in ((self.dtype,) if ln.act else (self.dtype, torch.float32)):
                raise TypeError(f"link {i}: y must be {self.dtype}" + ("" if ln.act else " or float32"))
            if ln.act and not packed:
                raise ValueError(f"link {i}: the SiLU-and-multiply epilogue needs a packed chain")
            g = arr[i]
            wp = packed_gate_up(ln.w) if ln.act else (packed_weight(ln.w) if packed else row_major_weight(ln.w))
            g.x, g.w, g.y = ln.x.data_ptr(), wp.data_ptr(), ln.y.data_ptr()
            g.ldx, g.ldw, g.ldy = ln.x.stride(0), ln.w.stride(0), ln.y.stride(0)
            g.N, g.K = ln.w.shape[0], ln.w.shape[1]
            g.split_k, g.dep = ln.split_k, ln.dep
            g.out_f32 = _lib.PLM_OUT_SILU_MUL if ln.act else int(ln.y.dtype == torch.float32)
        self._tile = _tile(self.cfg)
        lib = _lib.lib()
        prepare = lib.plm_gemm_chain_packed_prepare if packed else lib.plm_gemm_chain_prepare
        need = int(prepare(arr, len(links), self.M, self._tile))
        if need < 0:
            _lib.check(need, "plm_gemm_chain_prepare")
        self.host = arr
        raw = bytes(memoryview(arr).cast("B"))
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        self.workspace_bytes = need
        self.ws = workspace(self.device, need)

    def run(self) -> None:
        lib = _lib.lib()
        entry = lib.plm_gemm_chain_packed if self.packed else lib.plm_gemm_chain
        status = entry(_lib.DTYPE_CODES[self.dtype], self.host, self.table.data_ptr(), len(self.links), self.M,
                       self._tile, self.ws.data_ptr(), self.ws.numel(), _lib.stream_handle(self.device))
        _lib.check(status, f"plm_gemm_chain({len(self.links)} linears, M={self.M}, cfg={self.cfg})")

    @property
    def sync_mode(self) -> int:
        """How the launch makes linears wait for the ones they read (packed chains): 0 none, 1 grid
        barriers, 2 tile-done flags (``plm_gemm_chain_packed_sync_mode``)."""
        if not self.packed:
            raise ValueError("sync_mode describes packed chains")
        mode = int(_lib.lib().plm_gemm_chain_packed_sync_mode(self.host, len(self.links), self._tile))
        if mode < 0:
            _lib.check(mode, "plm_gemm_chain_packed_sync_mode")
        return mode

    def error_flag(self) -> int:
        """The counter area's error flag (1 if a wait for another workgroup gave up); syncs."""
        torch.cuda.synchronize(self.device)
        return int(self.ws[: 4 * (_lib.ERROR_INDEX + 1)].view(torch.int32)[_lib.ERROR_INDEX].item())

    def check(self) -> None:
        """Raises if a launch since the last check had a wait give up (its outputs, and those of
        every launch after it until this check, are invalid), and resets the workspace's whole
        counter area (the error int, split arrival counters, flags and epochs: the workspace is
        shared with the other entry points, whose counters a failed launch can leave off zero) so
        later launches are judged on their own. Synchronises the device; call it outside graph
        capture, after the launches (or graph replays) it vouches for."""
        if self.error_flag():
            reset_counters(self.ws)
            torch.cuda.synchronize(self.device)
            raise RuntimeError(f"a chained launch of {len(self.links)} linears had a wait for another workgroup give "
                               "up (another process on the device, or the grid was not resident): outputs invalid")
