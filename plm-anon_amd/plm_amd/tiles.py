"""Tile selection for shapes without a tuned table entry, and the candidate set the tuner sweeps.

A tile is ``{"wave_frags", "k_waves", "split_k", "unroll"}`` (``struct plm_tile`` in
``include/plm_amd.h``): tiles of ``16*wave_frags`` weight rows, ``k_waves`` (= 4) compute wavefronts
splitting each tile's K range, ``split_k`` workgroups splitting K further, and ``unroll`` 32-wide K
steps per weight chunk. Items (tile x split) = ``ceil(N / (16*wave_frags)) * split_k``; the
persistent grid has one workgroup per compute unit (two where registers and LDS allow).
"""

from __future__ import annotations

import math

CU_COUNT = 256          # MI355X compute units
K_WAVES = 4
WAVE_FRAGS = (1, 2, 4)
UNROLLS = (1, 2, 4)
SPLITS = (1, 2, 3, 4, 6, 8)


def ring_slots(M: int, cfg: dict) -> int:
    """Depth of each compute wavefront's weight ring in LDS (mirrors ``ring_slots`` in
    csrc/stream_gemm.h): what fits beside the spill area (two partial tiles), the X rings (two
    chunks per wavefront) and a 16 KiB descriptor reserve, at most 8."""
    mt, nf, u = math.ceil(M / 16), cfg["wave_frags"], cfg["unroll"]
    avail = 160 * 1024 - 256 - 16 * 1024 - 2 * nf * mt * 1024 - K_WAVES * 2 * mt * u * 1024
    return min(8, avail // (K_WAVES * nf * u * 1024))


def compiled(M: int, cfg: dict) -> bool:
    """Whether the library has a kernel for this tile at width M (mirrors ``stream_compiled`` in
    csrc/stream_gemm.h: a weight ring at least two chunks deep, and the compute wavefronts'
    registers within 256 VGPRs)."""
    mt, nf, u = math.ceil(M / 16), cfg["wave_frags"], cfg["unroll"]
    if not (1 <= mt <= 8 and nf in WAVE_FRAGS and u in UNROLLS and cfg["k_waves"] == K_WAVES):
        return False
    if ring_slots(M, cfg) < 2:
        return False
    return nf * mt * 4 + (nf + mt) * 4 + 64 <= 256


def items(N: int, cfg: dict) -> int:
    return math.ceil(N / (16 * cfg["wave_frags"])) * cfg["split_k"]


def steps_per_wave(K: int, cfg: dict) -> int:
    return math.ceil(math.ceil(K / 32) / (cfg["split_k"] * cfg["k_waves"]))


def candidates(M: int, N: int, K: int, supported=None) -> list[dict]:
    """Every sensible tile for ``(M, N, K)``; ``supported(cfg) -> bool`` filters to compiled kernels."""
    out = []
    for nf in WAVE_FRAGS:
        for split in SPLITS:
            for u in UNROLLS:
                cfg = {"wave_frags": nf, "k_waves": K_WAVES, "split_k": split, "unroll": u}
                spw = steps_per_wave(K, cfg)
                if spw < 1 or (u == 4 and spw <= 2):
                    continue
                if items(N, cfg) > 64 * CU_COUNT:
                    continue
                if supported is not None and not supported(cfg):
                    continue
                out.append(cfg)
    return out


def heuristic_tile(M: int, N: int, K: int, supported=None) -> dict:
    """A reasonable tile without measurement: the widest weight tile the registers allow, and
    enough K splitting to give every compute unit an item while each wavefront keeps at least
    four K steps per item."""
    steps = math.ceil(K / 32)
    for nf in (4, 2, 1):
        for u in (4, 2, 1):
            tiles = math.ceil(N / (16 * nf))
            split = 1
            while tiles * split < CU_COUNT and steps // (2 * split * K_WAVES) >= 4 and split < 8:
                split *= 2
            cfg = {"wave_frags": nf, "k_waves": K_WAVES, "split_k": split, "unroll": u}
            if compiled(M, cfg) and (supported is None or supported(cfg)):
                return cfg
    raise ValueError(f"no compiled tile fits (M={M}, N={N}, K={K})")


# Tile of a chained round (plm_gemm_chain): 64-row tiles, as a consumed output needs.
CHAIN_TILE = {"wave_frags": 4, "k_waves": K_WAVES, "split_k": 1, "unroll": 2}


def chain_tile(M: int) -> dict:
    """CHAIN_TILE at width M, with the unroll lowered until the weight ring fits in LDS (at M > 48
    two-step chunks leave room for only one ring slot)."""
    for u in (2, 1):
        cfg = dict(CHAIN_TILE, unroll=u)
        if compiled(M, cfg):
            return cfg
    raise ValueError(f"no chain tile is compiled at M={M}")


def chain_split(N: int, K: int, cfg: dict = CHAIN_TILE, workgroups: int = CU_COUNT) -> int:
    """K split of one linear inside a chain: the smallest power of two that gives about one item
    per resident workgroup, keeping at least two K steps per compute wavefront."""
    tiles = math.ceil(N / (16 * cfg["wave_frags"]))
    steps = math.ceil(K / 32)
    split = 1
    while tiles * split < workgroups * 3 // 4 and steps // (2 * split * K_WAVES) >= 2 and split < 8:
        split *= 2
    return split
