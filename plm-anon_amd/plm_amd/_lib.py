"""ctypes binding of ``libplm_amd.so`` (the C ABI in ``include/plm_amd.h``).

The library is the only compute path: if it is missing or fails to load, every entry point raises
``RuntimeError`` naming the problem. There is no CPU or library fallback behind it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # loads the HIP runtime the kernels register with, before the library is opened

LIBRARY = Path(__file__).resolve().parent / "libplm_amd.so"

PLM_BF16, PLM_F16 = 0, 1
PLM_ROUND_F32, PLM_ROUND_BF16, PLM_ROUND_F16 = 0, 1, 2
PLM_RULE_NUCLEUS, PLM_RULE_FLOOR = 0, 1
PLM_OUT_MODEL, PLM_OUT_F32, PLM_OUT_SILU_MUL = 0, 1, 2   # plm_chain_gemm.out_f32
DTYPE_CODES = {torch.bfloat16: PLM_BF16, torch.float16: PLM_F16}
# PLM_WORKSPACE_COUNTER_BYTES: the zero-between-calls counter area at the start of every workspace.
COUNTER_BYTES = 1 << 18

# PLM_NOALLOC_SCRATCH_BYTES: the device array plm_gemm_packed_noalloc uses instead of a workspace.
NOALLOC_SCRATCH_BYTES = COUNTER_BYTES + (8 << 20)

# PLM_WORKSPACE_ERROR_INDEX: the int in the counter area a chained launch sets when a wait gave up.
ERROR_INDEX = 2

# Every symbol include/plm_amd.h declares.
EXPORTS = (
    "plm_gemm",
    "plm_gemm_f32out",
    "plm_gemm_chain_prepare",
    "plm_gemm_chain",
    "plm_gemm_workspace_bytes",
    "plm_gemm_tile_supported",
    "plm_packed_weight_bytes",
    "plm_pack_weight",
    "plm_unpack_weight",
    "plm_gemm_packed",
    "plm_gemm_packed_f32out",
    "plm_gemm_packed_noalloc",
    "plm_gemm_packed_workspace_bytes",
    "plm_gemm_packed_tile_supported",
    "plm_gemm_chain_packed_prepare",
    "plm_gemm_chain_packed",
    "plm_gemm_chain_packed_sync_mode",
    "plm_gemm_packed_resident_workgroups",
    "plm_lm_head_verify",
    "plm_lm_head_verify_workspace_bytes",
    "plm_lm_head_verify_packed",
    "plm_lm_head_verify_packed_logits",
    "plm_round_epilogue",
    "plm_round_verify_packed",
    "plm_gemm_packed_lora",
    "plm_gemm_packed_lora_workspace_bytes",
    "plm_gemm_packed_silu_mul",
    "plm_voronoi_shortlist",
    "plm_voronoi_spread",
    "plm_voronoi_prior",
    "plm_voronoi_condense",
    "plm_voronoi_fit",
    "plm_voronoi_argmin",
    "plm_voronoi_assign",
    "plm_voronoi_assign_workspace_bytes",
    "plm_status_string",
)


class Tile(ctypes.Structure):
    """``struct plm_tile``: wave_frags, k_waves, split_k, unroll."""

    _fields_ = [("wave_frags", ctypes.c_int32), ("k_waves", ctypes.c_int32), ("split_k", ctypes.c_int32),
                ("unroll", ctypes.c_int32)]

    @classmethod
    def from_config(cls, cfg: dict) -> "Tile":
        return cls(int(cfg["wave_frags"]), int(cfg["k_waves"]), int(cfg.get("split_k", 1)), int(cfg["unroll"]))


class ChainGemm(ctypes.Structure):
    """``struct plm_chain_gemm``: one linear of a chain (88 bytes, natural alignment)."""

    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("ldx", ctypes.c_int64), ("ldw", ctypes.c_int64), ("ldy", ctypes.c_int64),
                ("N", ctypes.c_int32), ("K", ctypes.c_int32), ("split_k", ctypes.c_int32), ("dep", ctypes.c_int32),
                ("out_f32", ctypes.c_int32), ("consumed", ctypes.c_int32), ("arrive_base", ctypes.c_int32),
                ("done_base", ctypes.c_int32), ("partial_offset", ctypes.c_int64)]


_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def _declare(lib: ctypes.CDLL) -> None:
    c_i32, c_i64, c_p, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    tile_p = ctypes.POINTER(Tile)
    lib.plm_gemm.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, tile_p, c_p, c_sz, c_p]
    lib.plm_gemm.restype = ctypes.c_int
    lib.plm_gemm_f32out.argtypes = lib.plm_gemm.argtypes
    lib.plm_gemm_f32out.restype = ctypes.c_int
    chain_p = ctypes.POINTER(ChainGemm)
    lib.plm_gemm_chain_prepare.argtypes = [chain_p, c_i32, c_i64, tile_p]
    lib.plm_gemm_chain_prepare.restype = c_i64
    lib.plm_gemm_chain.argtypes = [c_i32, chain_p, c_p, c_i32, c_i64, tile_p, c_p, c_sz, c_p]
    lib.plm_gemm_chain.restype = ctypes.c_int
    lib.plm_gemm_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, tile_p]
    lib.plm_gemm_workspace_bytes.restype = c_sz
    lib.plm_gemm_tile_supported.argtypes = [c_i32, c_i64, c_i64, tile_p]
    lib.plm_gemm_tile_supported.restype = ctypes.c_int
    lib.plm_packed_weight_bytes.argtypes = [c_i64, c_i64]
    lib.plm_packed_weight_bytes.restype = c_sz
    lib.plm_pack_weight.argtypes = [c_i32, c_p, c_i64, c_i64, c_i64, c_p, c_sz, c_p]
    lib.plm_pack_weight.restype = ctypes.c_int
    lib.plm_unpack_weight.argtypes = [c_i32, c_p, c_sz, c_i64, c_i64, c_p, c_i64, c_p]
    lib.plm_unpack_weight.restype = ctypes.c_int
    lib.plm_gemm_packed.argtypes = [c_i32, c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_i64, tile_p, c_p, c_sz, c_p]
    lib.plm_gemm_packed.restype = ctypes.c_int
    lib.plm_gemm_packed_f32out.argtypes = lib.plm_gemm_packed.argtypes
    lib.plm_gemm_packed_f32out.restype = ctypes.c_int
    lib.plm_gemm_packed_noalloc.argtypes = [c_i32, c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_i64, tile_p, c_p]
    lib.plm_gemm_packed_noalloc.restype = ctypes.c_int
    lib.plm_gemm_packed_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, tile_p]
    lib.plm_gemm_packed_workspace_bytes.restype = c_sz
    lib.plm_gemm_packed_tile_supported.argtypes = [c_i32, c_i64, c_i64, tile_p]
    lib.plm_gemm_packed_tile_supported.restype = ctypes.c_int
    lib.plm_gemm_chain_packed_prepare.argtypes = [chain_p, c_i32, c_i64, tile_p]
    lib.plm_gemm_chain_packed_prepare.restype = c_i64
    lib.plm_gemm_chain_packed.argtypes = [c_i32, chain_p, c_p, c_i32, c_i64, tile_p, c_p, c_sz, c_p]
    lib.plm_gemm_chain_packed.restype = ctypes.c_int
    lib.plm_gemm_chain_packed_sync_mode.argtypes = [chain_p, c_i32, tile_p]
    lib.plm_gemm_chain_packed_sync_mode.restype = ctypes.c_int
    lib.plm_gemm_packed_resident_workgroups.argtypes = [c_i32, c_i64, tile_p]
    lib.plm_gemm_packed_resident_workgroups.restype = ctypes.c_int
    lib.plm_lm_head_verify.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_p, c_i32, ctypes.c_float,
                                       c_i32, c_p, c_p, tile_p, c_p, c_sz, c_p]
    lib.plm_lm_head_verify.restype = ctypes.c_int
    lib.plm_lm_head_verify_packed.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i32, ctypes.c_float,
                                              c_i32, c_p, c_p, tile_p, c_p, c_sz, c_p]
    lib.plm_lm_head_verify_packed.restype = ctypes.c_int
    lib.plm_lm_head_verify_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, tile_p]
    lib.plm_lm_head_verify_workspace_bytes.restype = c_sz
    lib.plm_round_epilogue.argtypes = [c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_i64, c_p, c_p, c_p,
                                       c_p]
    lib.plm_round_epilogue.restype = ctypes.c_int
    lib.plm_round_verify_packed.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i32, ctypes.c_float, c_i32, c_p,
                                            c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, tile_p,
                                            c_p, c_sz, c_p]
    lib.plm_round_verify_packed.restype = ctypes.c_int
    lib.plm_gemm_packed_lora.argtypes = [c_i32, c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_i64,
                                         c_i32, c_p, tile_p, c_p, c_sz, c_p]
    lib.plm_gemm_packed_lora.restype = ctypes.c_int
    lib.plm_gemm_packed_lora_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, tile_p]
    lib.plm_gemm_packed_lora_workspace_bytes.restype = c_sz
    lib.plm_gemm_packed_silu_mul.argtypes = lib.plm_gemm_packed.argtypes
    lib.plm_gemm_packed_silu_mul.restype = ctypes.c_int
    lib.plm_lm_head_verify_packed_logits.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_i32,
                                                     ctypes.c_float, c_i32, c_p, c_p, c_p, c_i64, c_i64, tile_p, c_p,
                                                     c_sz, c_p]
    lib.plm_lm_head_verify_packed_logits.restype = ctypes.c_int
    c_f = ctypes.c_float
    lib.plm_voronoi_shortlist.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                          c_p, c_p, c_p]
    lib.plm_voronoi_shortlist.restype = ctypes.c_int
    lib.plm_voronoi_spread.argtypes = [c_i32, c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_p]
    lib.plm_voronoi_spread.restype = ctypes.c_int
    lib.plm_voronoi_prior.argtypes = [c_p, c_p, c_i64, c_i64, c_i64, c_f, c_p, c_p]
    lib.plm_voronoi_prior.restype = ctypes.c_int
    lib.plm_voronoi_condense.argtypes = [c_i32, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_p, c_p]
    lib.plm_voronoi_condense.restype = ctypes.c_int
    lib.plm_voronoi_fit.argtypes = [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_f, c_f, c_f, c_p, c_p]
    lib.plm_voronoi_fit.restype = ctypes.c_int
    lib.plm_voronoi_argmin.argtypes = [c_i32, c_p, c_i64, c_i64, c_p, c_p, c_i64, c_i64, c_p, c_p]
    lib.plm_voronoi_argmin.restype = ctypes.c_int
    lib.plm_voronoi_assign.argtypes = [c_i32, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_f,
                                       c_f, c_f, c_f, c_f, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_sz, c_p]
    lib.plm_voronoi_assign.restype = ctypes.c_int
    lib.plm_voronoi_assign_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, c_i64]
    lib.plm_voronoi_assign_workspace_bytes.restype = c_sz
    lib.plm_status_string.argtypes = [c_i32]
    lib.plm_status_string.restype = ctypes.c_char_p


def lib() -> ctypes.CDLL:
    """The loaded kernel library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIBRARY.exists():
                    raise RuntimeError(f"{LIBRARY} is missing: build it with __graft_entry__.build() "
                                       "(or `python -m plm_amd._build` in plm-anon_amd/)")
                handle = ctypes.CDLL(str(LIBRARY))
                missing = [name for name in EXPORTS if not hasattr(handle, name)]
                if missing:
                    raise RuntimeError(f"{LIBRARY} does not export {missing}")
                _declare(handle)
                _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().plm_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream
