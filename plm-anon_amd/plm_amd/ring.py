"""The round's linears in one launch with the weight stream on a wavefront of its own
(``plm_ring_chain`` in ``include/plm_amd.h``).

The reference replays a round as a CUDA graph of 4L+1 separate ``fast_gemm`` launches
(plm/decoder.py:312-324, plm/fast_gemm.py:82-97). ``RingChain`` runs such a sequence of linears,
each reading an earlier one's output, as one persistent launch in which every compute unit keeps
one wavefront streaming the packed weights into LDS ahead of the four that multiply: the weights
of the next linear arrive while its input is still being produced. Each linear's result depends
only on its own tile geometry (``tile_rows``, ``split_k``), so a one-link chain reproduces any
link bit for bit.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .chain import Link
from .fast_gemm import HALF_DTYPES, packed_weight

MAX_ROWS = 64  # the ring chain's widest round (M <= 64)


@dataclass(frozen=True)
class Geometry:
    """A link's tile: ``tile_rows`` 16-row weight fragments per tile, K split over ``split_k``
    workgroups."""

    tile_rows: int
    split_k: int


class RingChain:
    """Validated, prepared ring chain; ``run()`` launches it on the current stream (graph-capturable
    once constructed). ``geometry`` overrides a link's tile (index -> ``Geometry``); otherwise the
    library picks one for the device's compute units. The chain owns its workspace (zeroed here):
    it keeps tile flags and arrival counters between launches."""

    def __init__(self, links: list[Link], geometry: dict[int, Geometry] | None = None,
                 workgroups: int | None = None):
        if not links:
            raise ValueError("a chain needs at least one linear")
        x0 = links[0].x
        self.links = links
        self.device = x0.device
        self.dtype = x0.dtype
        self.M = x0.shape[0]
        if self.dtype not in HALF_DTYPES:
            raise TypeError(f"chain operands must be bf16 or fp16, got {self.dtype}")
        if not 1 <= self.M <= MAX_ROWS:
            raise ValueError(f"a ring chain takes 1..{MAX_ROWS} rows, got {self.M}")
        geometry = geometry or {}
        arr = (_lib.RingLink * len(links))()
        self._packed = []
        for i, ln in enumerate(links):
            if ln.act:
                raise ValueError(f"link {i}: the ring chain has no SiLU-and-multiply epilogue")
            for name, t in (("x", ln.x), ("w", ln.w)):
                if t.dtype != self.dtype or t.device != self.device or t.dim() != 2 or t.stride(1) != 1:
                    raise ValueError(f"link {i}: {name} must be a row-major {self.dtype} matrix on {self.device}")
            if ln.x.shape[0] != self.M or ln.y.shape[0] != self.M or ln.x.shape[1] != ln.w.shape[1]:
                raise ValueError(f"link {i}: shapes x{tuple(ln.x.shape)} w{tuple(ln.w.shape)} y{tuple(ln.y.shape)}")
            if ln.y.shape[1] != ln.w.shape[0] or ln.y.stride(1) != 1 or ln.y.device != self.device:
                raise ValueError(f"link {i}: y must be a row-major [{self.M},{ln.w.shape[0]}] matrix")
            if ln.y.dtype not in (self.dtype, torch.float32):
                raise TypeError(f"link {i}: y must be {self.dtype} or float32")
            wp = packed_weight(ln.w)
            self._packed.append(wp)
            g = arr[i]
            g.x, g.w, g.y = ln.x.data_ptr(), wp.data_ptr(), ln.y.data_ptr()
            g.ldx, g.ldy = ln.x.stride(0), ln.y.stride(0)
            g.N, g.K = ln.w.shape[0], ln.w.shape[1]
            g.dep = ln.dep
            g.out_f32 = int(ln.y.dtype == torch.float32)
            geo = geometry.get(i)
            g.tile_rows, g.split_k = (geo.tile_rows, geo.split_k) if geo is not None else (0, 0)
        lib = _lib.lib()
        need = int(lib.plm_ring_chain_prepare(arr, len(links), self.M, int(workgroups or 0)))
        if need < 0:
            _lib.check(need, "plm_ring_chain_prepare")
        self.host = arr
        self.table = torch.frombuffer(bytearray(bytes(memoryview(arr).cast("B"))), dtype=torch.uint8).to(self.device)
        self.ws = torch.zeros(need, dtype=torch.uint8, device=self.device)

    @property
    def geometry(self) -> list[Geometry]:
        """Each link's tile as prepared."""
        return [Geometry(int(g.tile_rows), int(g.split_k)) for g in self.host]

    def run(self) -> None:
        status = _lib.lib().plm_ring_chain(_lib.DTYPE_CODES[self.dtype], self.host, self.table.data_ptr(),
                                           len(self.links), self.M, self.ws.data_ptr(), self.ws.numel(),
                                           _lib.stream_handle(self.device))
        _lib.check(status, f"plm_ring_chain({len(self.links)} linears, M={self.M})")

    def error_flag(self) -> int:
        """The workspace's error flag (1 if a wait for another workgroup gave up); syncs."""
        torch.cuda.synchronize(self.device)
        return int(self.ws[: 4 * (_lib.ERROR_INDEX + 1)].view(torch.int32)[_lib.ERROR_INDEX].item())

    def check(self) -> None:
        """Raises if a launch since the last check had a wait give up (its outputs, and those of later
        launches until this check, are invalid); the workspace is then zeroed whole (flags, arrival
        counters and the launch epoch start again together). Synchronises; call it outside graph
        capture."""
        if self.error_flag():
            self.ws.zero_()
            torch.cuda.synchronize(self.device)
            raise RuntimeError(f"a ring chain of {len(self.links)} linears had a wait for another workgroup give up "
                               "(another process on the device, or the grid was not resident): outputs invalid")
