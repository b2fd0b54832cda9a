"""Tile selection for shapes without a tuned table entry, and the candidate set the tuner sweeps.

A tile is ``{"wave_frags", "k_waves", "split_k", "unroll"}`` (``struct plm_tile`` in
``include/plm_amd.h``): ``k_waves`` (= 4) compute wavefronts each own ``16*wave_frags`` weight
rows, so a tile is ``64*wave_frags`` rows over its whole K range; ``split_k`` workgroups split K;
``unroll`` (= 2) 32-wide K steps are streamed per chunk. Items (tile x split) =
``ceil(N / (64*wave_frags)) * split_k``; the persistent grid has one workgroup per compute unit
(more where LDS allows).
"""

from __future__ import annotations

import math

CU_COUNT = 256          # MI355X compute units
K_WAVES = 4
UNROLL = 2
WAVE_FRAGS = (1, 2, 4)
SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)
LDS_BYTES = 160 * 1024 - 256
TABLE_RESERVE = 16 * 1024
LOADERS = 4             # loader wavefronts per workgroup (PLM_STREAM_LOADERS in csrc/stream_gemm.h)


def _slot(M: int, nf: int) -> int:
    """Ring slot bytes of csrc/stream_gemm.h: one chunk (two K steps) of the X rows and of the
    tile's 64*nf weight rows."""
    mt = math.ceil(M / 16)
    x_groups = -(-2 * mt // LOADERS) * LOADERS     # X row groups, padded to the loader count
    return x_groups * 1024 + K_WAVES * nf * 16 * 128


def ring_slots(M: int, cfg: dict, table_bytes: int = TABLE_RESERVE) -> int:
    """Chunk slots of the workgroup's LDS ring (mirrors ``ring_for_table`` in csrc/stream_gemm.h):
    what fits beside the descriptor table, at most 8; 0 if under two."""
    slot = _slot(M, cfg["wave_frags"])
    free = LDS_BYTES - table_bytes
    if free <= 0:
        return 0
    r = min(free // slot, 8)
    return r if r >= 2 else 0


def compiled(M: int, cfg: dict) -> bool:
    """Whether the library has a kernel for this tile at width M (mirrors ``stream_compiled`` in
    csrc/stream_gemm.h: a ring at least two chunks deep with the largest descriptor table, and at
    most 64 accumulator VGPRs per compute wavefront)."""
    mt, nf = math.ceil(M / 16), cfg["wave_frags"]
    if not (1 <= mt <= 8 and nf in WAVE_FRAGS and cfg["unroll"] == UNROLL and cfg["k_waves"] == K_WAVES):
        return False
    if ring_slots(M, cfg) < 2:
        return False
    return nf * mt <= 16


def items(N: int, cfg: dict) -> int:
    return math.ceil(N / (64 * cfg["wave_frags"])) * cfg["split_k"]


def chunks_per_item(K: int, cfg: dict) -> int:
    return math.ceil(math.ceil(K / 32) / cfg["split_k"] / UNROLL)


def candidates(M: int, N: int, K: int, supported=None) -> list[dict]:
    """Every sensible tile for ``(M, N, K)``; ``supported(cfg) -> bool`` filters to compiled kernels."""
    out = []
    for nf in WAVE_FRAGS:
        for split in SPLITS:
            cfg = {"wave_frags": nf, "k_waves": K_WAVES, "split_k": split, "unroll": UNROLL}
            if chunks_per_item(K, cfg) < 2 or items(N, cfg) > 64 * CU_COUNT:
                continue
            if split > 1 and items(N, dict(cfg, split_k=max(1, split // 2))) >= 2 * CU_COUNT:
                continue  # plenty of items with half the splitting
            if supported is not None and not supported(cfg):
                continue
            out.append(cfg)
    return out


def heuristic_tile(M: int, N: int, K: int, supported=None) -> dict:
    """A reasonable tile without measurement: the widest weight tile that is compiled, and enough
    K splitting to give every compute unit an item while each item keeps at least four chunks."""
    for nf in (2, 1, 4):
        cfg = {"wave_frags": nf, "k_waves": K_WAVES, "split_k": 1, "unroll": UNROLL}
        if not compiled(M, cfg) or (supported is not None and not supported(cfg)):
            continue
        split = 1
        while (items(N, dict(cfg, split_k=split)) < CU_COUNT and chunks_per_item(K, dict(cfg, split_k=2 * split)) >= 4
               and split < 16):
            split *= 2
        return dict(cfg, split_k=split)
    raise ValueError(f"no compiled tile fits (M={M}, N={N}, K={K})")


# Tile of a chained round (plm_gemm_chain): 64-row tiles.
CHAIN_TILE = {"wave_frags": 1, "k_waves": K_WAVES, "split_k": 1, "unroll": UNROLL}


def chain_tile(M: int) -> dict:
    """CHAIN_TILE at width M (64-row tiles are compiled at every width up to 128)."""
    if not compiled(M, CHAIN_TILE):
        raise ValueError(f"no chain tile is compiled at M={M}")
    return dict(CHAIN_TILE)


def chain_split(N: int, K: int, cfg: dict = CHAIN_TILE, workgroups: int = CU_COUNT) -> int:
    """K split of one linear inside a chain: the smallest power of two that gives about one item
    per resident workgroup, keeping at least two chunks per item."""
    tiles = math.ceil(N / (64 * cfg["wave_frags"]))
    split = 1
    while (tiles * split < workgroups * 3 // 4 and chunks_per_item(K, dict(cfg, split_k=2 * split)) >= 2
           and split < 16):
        split *= 2
    return split
