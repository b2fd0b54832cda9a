"""Gated LoRA on the HIP kernel: the adapter acts on a round's auxiliary rows only (plm/gated_lora.py).

The reference's ``GatedLoraMethod.apply`` runs the base linear over every row, a second GEMM
``h = x[g:] A^T`` and one ``addmm_`` per shard of a fused projection (plm/gated_lora.py:45-57). Here a
tuned, eligible call is one launch of ``plm_gemm_packed_lora``: its first workgroups form ``h`` into
the workspace, the rest run the base GEMM on its tuned tile and add every shard's rank-r correction
to the gated rows before they store them. Calls the reference itself would not route to its fast
GEMM (a bias, an untuned shape, a non-half dtype) take the reference's unfused composition through
``fast_gemm``'s dispatch slot.

``rows_from(g)`` sets the first gated row for the calls inside it, as the reference's context manager
does; ``install(model, tensors)`` attaches stacked ``lora_a`` buffers and wraps each adapted layer's
linear method (plm/gated_lora.py:60-89).
"""

from __future__ import annotations

import ctypes
from collections.abc import Iterator
from contextlib import contextmanager

import torch

from . import _lib, tiles
from .fast_gemm import CONFIGS, HALF_DTYPES, Config, dispatch_unquantized_gemm, packed_weight, workspace

_rows_from: int | None = None

# A fused projection's shards in the order its output columns hold them (plm/gated_lora.py:20).
FUSED_PROJECTIONS = {"qkv_proj": ("q_proj", "k_proj", "v_proj"), "gate_up_proj": ("gate_proj", "up_proj")}
LORA_SUFFIXES = (".lora_a", ".lora_b")


@contextmanager
def rows_from(first_gated_row: int | None) -> Iterator[None]:
    """Rows ``first_gated_row`` onwards of every gated call inside the block carry the adapter."""
    global _rows_from
    saved, _rows_from = _rows_from, first_gated_row
    try:
        yield
    finally:
        _rows_from = saved


MAX_RANK = 1024


def stack_b(lora_bs: list[torch.Tensor]) -> torch.Tensor:
    """The shards' up-projections stacked by output column ([N, rank], row-major): the layout
    ``plm_gemm_packed_lora`` reads. A new tensor; callers that apply the same adapter repeatedly
    (``GatedLoraMethod``) stack once and pass it as ``lora_b``."""
    return torch.cat([b.contiguous() for b in lora_bs], dim=0).contiguous()


def _eligible(x, weight, lora_a, lora_bs, first_gated_row, bias, cfg) -> bool:
    """Whether the fused HIP path takes this call: everything ``plm_gemm_packed_lora`` checks, so
    that an ineligible call takes the reference's composition instead of failing."""
    from .fast_gemm import WIDE_ROWS, tile_supported

    shards = len(lora_bs)
    if cfg is None or bias is not None or x.dim() != 2 or x.dtype not in HALF_DTYPES or not x.is_cuda:
        return False
    if weight.dtype != x.dtype or lora_a.dtype != x.dtype or any(b.dtype != x.dtype for b in lora_bs):
        return False
    if not 1 <= shards <= 3 or lora_a.shape[0] % shards:
        return False
    rank = lora_a.shape[0] // shards
    if rank < 8 or rank > MAX_RANK or rank % 8 or any(b.dim() != 2 or b.shape[1] != rank for b in lora_bs):
        return False
    M, K = x.shape
    if sum(b.shape[0] for b in lora_bs) != weight.shape[0] or K % 8:
        return False
    # The one-launch correction runs on the skinny packed kernel only (plm_gemm_packed_lora takes
    # up to WIDE_ROWS rows); wider calls (prefill chunks) take the reference's composition, whose
    # GEMMs fast_gemm routes to the wide kernel or F.linear.
    if M > WIDE_ROWS:
        return False
    # Sixteen-wavefront tiles above 48 estimated registers even at depth 2 have no LoRA kernel (its
    # epilogue would spill: packed_fits in csrc/packed_gemm.h).
    if cfg["k_waves"] == 16 and tiles._regs(-(-M // 16), cfg["wave_frags"], 2, 16) > 48:
        return False
    return tile_supported(M, K, cfg, x.dtype)


def gated_linear(x: torch.Tensor, weight: torch.Tensor, lora_a: torch.Tensor, lora_bs: list[torch.Tensor],
                 first_gated_row: int | None, bias: torch.Tensor | None = None,
                 cfg: Config | None = None, lora_b: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ weight^T`` with rows ``first_gated_row..`` corrected by ``(x A^T) B_s^T`` per shard.

    ``lora_a`` is ``[shards*rank, K]``, ``lora_bs[s]`` is ``[N_s, rank]`` with ``sum N_s = N``;
    ``lora_b`` may carry them already stacked (``stack_b``). The HIP path runs when the call is
    eligible for the tuned GEMM (no bias, 2-D half-precision operands, a tile in ``cfg`` or
    installed for ``(M, N, K)``, a rank the kernel takes); otherwise the reference's composition.
    The HIP path's workgroups wait on each other within the launch (bounded):
    ``fast_gemm.check_workspace`` reports a wait that gave up."""
    M = x.shape[0]
    if first_gated_row is None or first_gated_row >= M:
        return dispatch_unquantized_gemm()(None, x, weight, bias)
    first_gated_row = max(int(first_gated_row), 0)
    cfg = cfg if cfg is not None else CONFIGS.get((M, weight.shape[0], weight.shape[1]))
    shards = len(lora_bs)
    rank = lora_a.shape[0] // shards
    if not _eligible(x, weight, lora_a, lora_bs, first_gated_row, bias, cfg):
        gemm = dispatch_unquantized_gemm()
        output = gemm(None, x, weight, bias)
        hidden = gemm(None, x[first_gated_row:], lora_a)
        col = 0
        for s, b in enumerate(lora_bs):
            output[first_gated_row:, col:col + b.shape[0]].addmm_(hidden[:, s * rank:(s + 1) * rank], b.t().contiguous())
            col += b.shape[0]
        return output
    if not (x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0):
        x = x.contiguous()
    N, K = weight.shape
    out = torch.empty(M, N, device=x.device, dtype=x.dtype)
    if lora_b is None:
        lora_b = stack_b(lora_bs)
    elif lora_b.shape != (N, rank) or lora_b.stride() != (rank, 1) or lora_b.data_ptr() % 16:
        raise ValueError(f"lora_b must be the shards' B's stacked row-major as [{N}, {rank}]")
    tile = _lib.Tile.from_config(cfg)
    lib = _lib.lib()
    g = first_gated_row
    ws = workspace(x.device, int(lib.plm_gemm_packed_lora_workspace_bytes(M, N, K, g, rank, shards, tile)))
    sizes = (ctypes.c_int64 * shards)(*[b.shape[0] for b in lora_bs])
    status = lib.plm_gemm_packed_lora(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0),
                                      packed_weight(weight).data_ptr(), out.data_ptr(), out.stride(0), M, N, K, g,
                                      packed_weight(lora_a).data_ptr(), lora_b.data_ptr(), rank, shards, sizes, tile,
                                      ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device))
    _lib.check(status, f"plm_gemm_packed_lora(M={M}, N={N}, K={K}, rank={rank}, shards={shards})")
    return out


class GatedLoraMethod:
    """Wraps a layer's linear method: ``weight`` over every row, plus the rank-r correction on the
    gated rows (plm/gated_lora.py:35-57)."""

    def __init__(self, inner, lora_bs: list[torch.Tensor]) -> None:
        self.inner = inner
        self.lora_bs = lora_bs
        # Stacked once here, at install, so no call concatenates (or caches) during graph capture.
        self.lora_b = stack_b(lora_bs)

    def __getattr__(self, name: str):
        return getattr(self.inner, name)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        first = _rows_from
        if first is None or first >= x.shape[0]:
            return self.inner.apply(layer, x, bias)
        return gated_linear(x, layer.weight, layer.lora_a, self.lora_bs, first, bias, lora_b=self.lora_b)


def _module_names(tensors: dict[str, torch.Tensor], suffix: str) -> dict[str, torch.Tensor]:
    return {name[: -len(suffix)]: t for name, t in tensors.items() if name.endswith(suffix)}


def _fuse(per_module: dict[str, torch.Tensor], combine) -> dict[str, object]:
    """Per-projection export names (``...self_attn.q_proj``) to the fused module names the model
    uses, combining a fused projection's shards with ``combine`` in shard order."""
    fused: dict[str, object] = {}
    shard_of = {shard: (proj, shards) for proj, shards in FUSED_PROJECTIONS.items() for shard in shards}
    for name in sorted(per_module):
        parent, projection = name.rsplit(".", 1)
        if projection not in shard_of:
            fused[name] = per_module[name]
            continue
        proj, shards = shard_of[projection]
        if projection == shards[0]:
            fused[f"{parent}.{proj}"] = combine([per_module[f"{parent}.{s}"] for s in shards])
    return fused


def install(model: torch.nn.Module, tensors: dict[str, torch.Tensor]) -> None:
    """Attach the adapter: each adapted layer gets a ``lora_a`` buffer (a fused projection's shards'
    A's stacked, since they share the input) and its linear method wrapped in ``GatedLoraMethod``
    with the per-shard B's (plm/gated_lora.py:82-89)."""
    modules = dict(model.named_modules())
    ups = _fuse(_module_names(tensors, LORA_SUFFIXES[1]), list)
    for name, down in _fuse(_module_names(tensors, LORA_SUFFIXES[0]), lambda ts: torch.cat(ts)).items():
        layer = modules[name]
        place = dict(device=layer.weight.device, dtype=layer.weight.dtype)
        layer.register_buffer("lora_a", down.to(**place), persistent=False)
        shards = ups[name] if isinstance(ups[name], list) else [ups[name]]
        layer.quant_method = GatedLoraMethod(layer.quant_method, [b.to(**place) for b in shards])
