"""Tile selection for shapes without a tuned table entry, and the candidate set the tuner sweeps.

A tile is ``{"wave_frags", "k_waves", "split_k", "unroll"}`` (``struct plm_tile`` in
``include/plm_amd.h``). For the packed-weight GEMM behind ``fast_gemm`` (plm_gemm_packed), each
wavefront of a workgroup streams ``16*wave_frags`` weight rows, and either
``k_waves`` = 4, 8 or 16: that many wavefronts split the K range of one ``16*wave_frags``-row tile
(summed in LDS), or ``k_waves`` = 1: four wavefronts take adjacent rows of a ``64*wave_frags``-row
tile over the whole K range and share one copy of X through LDS. ``split_k`` workgroups split K further (fp32 partials summed
in split order); ``unroll`` (2, 4, 6 or 8) K steps of loads are in flight per wavefront. Items
(tile x split) = ``ceil(ceil(N/16) / tile_frags) * split_k`` over a persistent grid.

The chained round (plm_gemm_chain) uses the streaming kernel's tiles: ``64*wave_frags`` rows,
``unroll`` = 2 (``chain_tile``, ``chain_split`` below).
"""

from __future__ import annotations

import math

CU_COUNT = 256          # MI355X compute units
K_WAVES = 4             # wavefronts per workgroup of the row-split layout
LAYOUTS = (4, 8, 16, 1)  # k_waves: K split across 4, 8 or 16 wavefronts, or rows split across 4
LDS_LIMIT = 160 * 1024
FRAG = 1024             # bytes of one packed fragment
X_TILE = 16 * 80        # LDS transpose tile of one X fragment
WAVE_FRAGS = (1, 2, 4)
DEPTHS = (2, 4, 6, 8)
SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)


def _regs(mt: int, nf: int, d: int, kw: int) -> int:
    xn = (mt + 3) // 4 if kw == 1 else mt
    return (d * (nf + xn) + nf * mt + (mt if kw == 1 else 0)) * 4


def pair_x(mt: int, kw: int) -> bool:
    """Whether X is staged two K steps at a time (mirrors ``packed_pair_x``)."""
    return kw == 1 or (kw == 8 and mt >= 4 and 2 * kw * mt * X_TILE + FRAG <= LDS_LIMIT)


def lds_body(mt: int, nf: int, kw: int) -> int:
    """LDS bytes before the warm-up sink (mirrors ``packed_lds_body``)."""
    red, xts = kw * nf * mt * FRAG, kw * mt * X_TILE * (2 if kw != 1 and pair_x(mt, kw) else 1)
    if kw == 1:
        return 4 * mt * X_TILE
    return red + xts if kw == 4 else max(red, xts)


def two_per_cu(M: int, cfg: dict) -> bool:
    """Whether two workgroups of this tile share a CU (mirrors ``packed_two_per_cu``)."""
    mt, nf, d, kw = math.ceil(M / 16), cfg["wave_frags"], cfg["unroll"], cfg["k_waves"]
    r = _regs(mt, nf, d, kw)
    if kw == 1:
        return r <= 100
    if kw > 4:
        return False
    return r <= 128 and (mt <= 6 or r <= 104)


def compiled(M: int, cfg: dict) -> bool:
    """Whether the library has a packed-GEMM kernel for this tile at width M (mirrors
    ``packed_compiled`` in csrc/packed_gemm.h: at most 20 accumulator fragments, and two
    workgroups per CU, or one with the pipeline within 320 registers)."""
    mt, nf, d, kw = math.ceil(M / 16), cfg["wave_frags"], cfg["unroll"], cfg["k_waves"]
    if not (1 <= mt <= 8 and nf in WAVE_FRAGS and d in DEPTHS and kw in LAYOUTS) or nf * mt > 20:
        return False
    if kw > 4:
        return lds_body(mt, nf, kw) + FRAG <= LDS_LIMIT and _regs(mt, nf, d, kw) <= (144 if kw == 8 else 60)
    return two_per_cu(M, cfg) or _regs(mt, nf, d, kw) <= 320


def tile_frags(cfg: dict) -> int:
    """16-row weight fragments of one workgroup tile."""
    return cfg["wave_frags"] * (K_WAVES if cfg["k_waves"] == 1 else 1)


def items(N: int, cfg: dict) -> int:
    return math.ceil(math.ceil(N / 16) / tile_frags(cfg)) * cfg["split_k"]


def steps_per_wave(K: int, cfg: dict) -> int:
    """32-wide K steps each wavefront streams per item (K-split layouts: the shortest share)."""
    return math.ceil(K / 32) // cfg["split_k"] // (1 if cfg["k_waves"] == 1 else cfg["k_waves"])


def candidates(M: int, N: int, K: int, supported=None) -> list[dict]:
    """Every sensible tile for ``(M, N, K)``; ``supported(cfg) -> bool`` filters to compiled kernels."""
    out = []
    for kw in LAYOUTS:
        for nf in WAVE_FRAGS:
            for d in DEPTHS:
                for split in SPLITS:
                    cfg = {"wave_frags": nf, "k_waves": kw, "split_k": split, "unroll": d}
                    if not compiled(M, cfg) or items(N, cfg) > 64 * CU_COUNT:
                        continue
                    if split > 1 and (steps_per_wave(K, cfg) < 2 or
                                      items(N, dict(cfg, split_k=max(1, split // 2))) >= 4 * CU_COUNT):
                        continue  # too little K per wavefront, or plenty of items with half the splitting
                    if supported is not None and not supported(cfg):
                        continue
                    out.append(cfg)
    return out


def _first_compiled(M: int, nf: int, layouts, supported) -> dict | None:
    for kw in layouts:
        for d in DEPTHS:
            cfg = {"wave_frags": nf, "k_waves": kw, "split_k": 1, "unroll": d}
            if compiled(M, cfg) and (supported is None or supported(cfg)):
                return cfg
    return None


def heuristic_tile(M: int, N: int, K: int, supported=None) -> dict:
    """A reasonable tile without measurement (what the MI355X measurements of the round shapes
    favour): 32 rows per wavefront with a two-stage pipeline; rows split across the wavefronts
    (128-row tiles) when that alone gives every compute unit a tile (the LM head: one round of
    tiles instead of three and a fraction), else K split across 8 wavefronts (4 where 8 is not
    compiled), and K splitting until about three quarters of the compute units have an item,
    keeping at least two K steps per wavefront."""
    for nf in (2, 4, 1):
        layouts = (1,) if math.ceil(N / 16) // (K_WAVES * nf) >= CU_COUNT else (8, 4)
        cfg = _first_compiled(M, nf, layouts, supported)
        if cfg is None:
            continue
        split = 1
        while (items(N, dict(cfg, split_k=split)) < CU_COUNT * 3 // 4 and
               steps_per_wave(K, dict(cfg, split_k=2 * split)) >= 2 and split < 16):
            split *= 2
        return dict(cfg, split_k=split)
    raise ValueError(f"no compiled tile fits (M={M}, N={N}, K={K})")


def packed_chain_split(N: int, K: int, cfg: dict, workgroups: int) -> int:
    """K split of one linear of a packed chain (every linear ends at a grid barrier, so its time
    is that of the busiest workgroup): the split with the least estimated busiest-workgroup time,
    counting each item's K steps per wavefront plus a fixed cost of a few steps for the item's end
    (reduction, stores; with split > 1 the partial round trip)."""
    tiles_ = math.ceil(math.ceil(N / 16) / tile_frags(cfg))
    ks = math.ceil(K / 32)
    kw = 1 if cfg["k_waves"] == 1 else cfg["k_waves"]
    best, best_cost = 1, None
    for split in SPLITS:
        if split > 1 and ks // split // kw < 2:
            break
        per_wg = math.ceil(tiles_ * split / workgroups)
        steps = max(cfg["unroll"], math.ceil(ks / split / kw))
        cost = per_wg * (steps + (3 if split == 1 else 8))
        if best_cost is None or cost < best_cost:
            best, best_cost = split, cost
    return best


# ---------------------------------------------------------------- streaming kernel (chains)

STREAM_UNROLL = 2
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
    """Chunk slots of the streaming kernel's LDS ring (mirrors ``ring_for_table`` in
    csrc/stream_gemm.h): what fits beside the descriptor table, at most 8; 0 if under two."""
    slot = _slot(M, cfg["wave_frags"])
    free = LDS_BYTES - table_bytes
    if free <= 0:
        return 0
    r = min(free // slot, 8)
    return r if r >= 2 else 0


def stream_compiled(M: int, cfg: dict) -> bool:
    """Whether the streaming kernel (plm_gemm, plm_gemm_chain) is compiled for this tile at width M
    (mirrors ``stream_compiled`` in csrc/stream_gemm.h)."""
    mt, nf = math.ceil(M / 16), cfg["wave_frags"]
    if not (1 <= mt <= 8 and nf in WAVE_FRAGS and cfg["unroll"] == STREAM_UNROLL and cfg["k_waves"] == K_WAVES):
        return False
    if ring_slots(M, cfg) < 2:
        return False
    return nf * mt <= 16


def chunks_per_item(K: int, cfg: dict) -> int:
    return math.ceil(math.ceil(K / 32) / cfg["split_k"] / STREAM_UNROLL)


# Tile of a chained round (plm_gemm_chain): 64-row tiles.
CHAIN_TILE = {"wave_frags": 1, "k_waves": K_WAVES, "split_k": 1, "unroll": STREAM_UNROLL}


def chain_tile(M: int) -> dict:
    """CHAIN_TILE at width M (64-row tiles are compiled at every width up to 128)."""
    if not stream_compiled(M, CHAIN_TILE):
        raise ValueError(f"no chain tile is compiled at M={M}")
    return dict(CHAIN_TILE)


def packed_chain_tile(M: int) -> dict:
    """Tile of a packed chained round at width M: 32-row tiles of eight wavefronts splitting K, one
    workgroup per CU. At M > 48 (four X fragments) the two-stage pipeline has that residency; at
    M <= 48 the two-stage kernel's smaller register count admits two workgroups per CU, which
    measured slower (1167 against 1025 us for the 1.3B-shape round at M = 42), so the four-stage
    pipeline is used."""
    return {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2 if M > 48 else 4}


def chain_split(N: int, K: int, cfg: dict = CHAIN_TILE, workgroups: int = CU_COUNT) -> int:
    """K split of one linear inside a chain: the smallest power of two that gives about one item
    per resident workgroup, keeping at least two chunks per item."""
    tiles = math.ceil(N / (64 * cfg["wave_frags"]))
    split = 1
    while (tiles * split < workgroups * 3 // 4 and chunks_per_item(K, dict(cfg, split_k=2 * split)) >= 2
           and split < 16):
        split *= 2
    return split
