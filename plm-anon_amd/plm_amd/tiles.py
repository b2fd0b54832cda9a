"""Tile selection for shapes without a tuned table entry, and the candidate set the tuner sweeps.

A tile is ``{"wave_frags", "k_waves", "split_k", "unroll"}`` (see ``struct plm_tile`` in
``include/plm_amd.h``). Workgroups = ``ceil(N / (16*wave_frags)) * split_k``; each wavefront takes
``ceil(ceil(K/32) / (split_k*k_waves))`` 32-wide K steps, loaded in batches of ``unroll``.
"""

from __future__ import annotations

import math

CU_COUNT = 256          # MI355X compute units
UNROLLS = (2, 4, 8)
WAVE_FRAGS = (1, 2, 4)
K_WAVES = (4, 8)
SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)


def steps_per_wave(K: int, cfg: dict) -> int:
    return math.ceil(math.ceil(K / 32) / (cfg["split_k"] * cfg["k_waves"]))


def workgroups(N: int, cfg: dict) -> int:
    return math.ceil(N / (16 * cfg["wave_frags"])) * cfg["split_k"]


def candidates(M: int, N: int, K: int, supported=None) -> list[dict]:
    """Every sensible tile for ``(M, N, K)``; ``supported(cfg) -> bool`` filters to compiled kernels."""
    steps = math.ceil(K / 32)
    out = []
    for nf in WAVE_FRAGS:
        for kw in K_WAVES:
            for split in SPLITS:
                if split * kw > steps:
                    continue
                for u in UNROLLS:
                    cfg = {"wave_frags": nf, "k_waves": kw, "split_k": split, "unroll": u}
                    spw = steps_per_wave(K, cfg)
                    if u > 2 and spw <= u // 2:      # a smaller batch already covers the slice
                        continue
                    wgs = workgroups(N, cfg)
                    if wgs < CU_COUNT // 4 or wgs > 16 * CU_COUNT:
                        continue
                    if supported is not None and not supported(cfg):
                        continue
                    out.append(cfg)
    return out


def heuristic_tile(M: int, N: int, K: int, supported=None) -> dict:
    """A reasonable tile without measurement: 32-row tiles, 8 wavefronts, enough K splitting to put
    about two workgroups on every CU, and a single load batch per wavefront when it fits. With
    ``supported(cfg) -> bool`` it falls back to 4 wavefronts, then 16-row tiles, until a compiled
    kernel exists."""
    steps = math.ceil(K / 32)
    for nf, kw in ((2, 8), (2, 4), (1, 8), (1, 4)):
        tiles = math.ceil(N / (16 * nf))
        split = 1
        while tiles * split < 2 * CU_COUNT and split * 2 * kw <= steps and split < 16:
            split *= 2
        cfg = {"wave_frags": nf, "k_waves": kw, "split_k": split, "unroll": 8}
        spw = steps_per_wave(K, cfg)
        cfg["unroll"] = 2 if spw <= 2 else 4 if spw <= 4 else 8 if spw <= 8 else 4
        if supported is None or supported(cfg):
            return cfg
        if spw > 2:
            cfg["unroll"] = 4 if spw <= 4 or cfg["unroll"] == 8 else 2
            if supported(cfg):
                return cfg
    raise ValueError(f"no compiled tile fits (M={M}, N={N}, K={K})")
