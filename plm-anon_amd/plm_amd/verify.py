"""Fused LM-head verify step on the HIP kernel: the LM-head GEMM with the round's acceptance
epilogue folded in, so the ``[R, V]`` logits are never written to memory.

Per row ``r`` it returns the nucleus decision for ``pending[r]`` (``nucleus_acceptance``,
plm/decoder.py:71-75) and the row argmax with lowest-index ties (``logits.argmax(-1)``,
plm/decoder.py:362). ``round_to`` fixes which logits the decision reads: ``"fp32"`` is the fp32
accumulator; ``"bf16"``/``"fp16"`` round it to the model dtype first, which is what the reference's
decoder sees (the GEMM output cast at plm/fast_gemm.py:46, upcast again at plm/decoder.py:73).
"""

from __future__ import annotations

import torch

from . import _lib
from .fast_gemm import HALF_DTYPES, Config, packed_weight, workspace

ROUND_MODES = {"fp32": _lib.PLM_ROUND_F32, "bf16": _lib.PLM_ROUND_BF16, "fp16": _lib.PLM_ROUND_F16}

# Verify tile over packed weights (plm_lm_head_verify_packed): the row-split layout, 128-row tiles.
VERIFY_CONFIG: Config = {"wave_frags": 2, "k_waves": 1, "split_k": 1, "unroll": 2}

# A GEMM tile with the packed verify's accumulation order (every logit one MFMA chain over the K
# steps in order): ``hip_linear_f32`` with it (or any row-split tile with split_k 1) returns, bit for
# bit, the logits the packed verify decides on.
LOGITS_CONFIG: Config = {"wave_frags": 2, "k_waves": 1, "split_k": 1, "unroll": 2}

# The same pair for the verify kernel over row-major weights (``packed=False``): its workgroup's
# four wavefronts each take a quarter of K, summed in wavefront order, as the packed GEMM's
# 4-wavefront K split does.
ROWMAJOR_VERIFY_CONFIG: Config = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}
ROWMAJOR_LOGITS_CONFIG: Config = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2}


def verify_workspace_bytes(R: int, V: int, K: int, cfg: Config = VERIFY_CONFIG) -> int:
    return int(_lib.lib().plm_lm_head_verify_workspace_bytes(R, V, K, _lib.Tile.from_config(cfg)))


def lm_head_verify(x: torch.Tensor, w: torch.Tensor, pending: torch.Tensor, p: float, round_to: str = "fp32",
                   cfg: Config | None = None, accept: torch.Tensor | None = None,
                   argmax: torch.Tensor | None = None, packed: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """``(accept[R] bool, argmax[R] int64)`` for ``logits = x[R,K] @ w[V,K]^T``.

    ``pending[R]`` (int64, on the GPU) are the proposed ids; an id outside ``[0, V)`` is never
    accepted. ``p <= 0`` accepts nothing (exact matching, plm/decoder.py:115). With ``packed``
    (the default) W is read through its packed copy (``fast_gemm.packed_weight``, made once per
    weight) on the packed GEMM's pipeline; ``packed=False`` reads W row-major."""
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"lm_head_verify expects x[R,K] and w[V,K], got {tuple(x.shape)} and {tuple(w.shape)}")
    if x.dtype not in HALF_DTYPES or w.dtype != x.dtype:
        raise TypeError(f"lm_head_verify needs matching bf16/fp16 operands, got {x.dtype} and {w.dtype}")
    if round_to not in ROUND_MODES:
        raise ValueError(f"round_to must be one of {sorted(ROUND_MODES)}")
    R, K = x.shape
    V = w.shape[0]
    if pending.shape != (R,) or pending.dtype != torch.int64 or pending.device != x.device:
        raise ValueError(f"pending must be an int64 [{R}] tensor on {x.device}")
    if not (x.is_cuda and w.is_cuda):
        raise RuntimeError("lm_head_verify runs on the GPU only; got a CPU tensor")
    cfg = (VERIFY_CONFIG if packed else ROWMAJOR_VERIFY_CONFIG) if cfg is None else cfg
    tile = _lib.Tile.from_config(cfg)
    x = x if (x.stride(1) == 1 and x.stride(0) % 8 == 0) else x.contiguous()
    w = w if (w.stride(1) == 1 and w.stride(0) % 8 == 0) else w.contiguous()
    pending = pending.contiguous()
    # The kernel writes one byte 0/1 per row: a bool tensor's storage directly.
    direct = accept is not None and accept.dtype == torch.bool and accept.is_contiguous() and accept.shape == (R,)
    accept_out = accept if direct else torch.empty(R, dtype=torch.bool, device=x.device)
    if argmax is None:
        argmax = torch.empty(R, dtype=torch.int64, device=x.device)
    lib = _lib.lib()
    need = int(lib.plm_lm_head_verify_workspace_bytes(R, V, K, tile))
    ws = workspace(x.device, need)
    common = (pending.data_ptr(), float(p), ROUND_MODES[round_to], accept_out.data_ptr(), argmax.data_ptr(), tile,
              ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device))
    if packed:
        status = lib.plm_lm_head_verify_packed(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0),
                                               packed_weight(w).data_ptr(), R, V, K, *common)
        _lib.check(status, f"plm_lm_head_verify_packed(R={R}, V={V}, K={K}, cfg={cfg})")
    else:
        status = lib.plm_lm_head_verify(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0), w.data_ptr(),
                                        w.stride(0), R, V, K, *common)
        _lib.check(status, f"plm_lm_head_verify(R={R}, V={V}, K={K}, cfg={cfg})")
    if accept is not None and not direct:
        accept.copy_(accept_out)
        return accept, argmax
    return accept_out, argmax
