"""Install the MI355X GEMM tile table for one round width (the reference's ``plm.gemm_tables``,
plm/gemm_tables.py).

``gpu_tuning/tiles_hidden<H>.json`` holds the tiles for one model width, keyed ``"M,N,K"``, for the
round widths the reference tunes (42 at every released hidden size, 56 and 110 at 2048 and 3072)
plus the GPT-style shapes the MI355X benchmark runs. A missing table or shape is an error, never a
silent fallback (plm/gemm_tables.py:1-5).
"""

from __future__ import annotations

import json
from pathlib import Path

from . import fast_gemm

TABLES = Path(__file__).resolve().parent / "gpu_tuning"
# The LM head's row count is the vocabulary rounded up to a multiple of this (the padded head the
# serving engine allocates), so the table keys the head on the padded N.
VOCAB_PADDING = 64
WIDEST_TUNED_DOWN_ROUND = 72
# Above W=72 the `down` projection uses this fixed tile instead of the table entry (the reference's
# override, plm/gemm_tables.py:17-19, 41-42). On MI355X the split-K combine costs no extra launch,
# so the fixed tile splits K 8 ways (256 items at hidden 2048); 64-row tiles are compiled up to M=128.
DOWN_SPLIT_K1 = {"wave_frags": 1, "k_waves": 4, "split_k": 8, "unroll": 2}


def model_shapes(hf_config) -> dict[str, tuple[int, int]]:
    """``(N, K)`` of the five round GEMMs of a Llama-style config (plm/gemm_tables.py:22-27)."""
    hidden, intermediate, head_dim = hf_config.hidden_size, hf_config.intermediate_size, hf_config.head_dim
    heads, kv_heads = hf_config.num_attention_heads, hf_config.num_key_value_heads
    vocab = -(-hf_config.vocab_size // VOCAB_PADDING) * VOCAB_PADDING
    return {"qkv": ((heads + 2 * kv_heads) * head_dim, hidden), "o": (hidden, heads * head_dim),
            "gate_up": (2 * intermediate, hidden), "down": (hidden, intermediate), "lm_head": (vocab, hidden)}


def read_table(hidden: int) -> dict[tuple[int, int, int], dict]:
    """Every ``(M, N, K) -> tile`` entry of ``tiles_hidden<hidden>.json``; SystemExit if absent."""
    path = TABLES / f"tiles_hidden{hidden}.json"
    if not path.exists():
        raise SystemExit(f"--mode fast has no tile table for hidden size {hidden}; use --mode default")
    return {tuple(int(v) for v in key.split(",")): cfg for key, cfg in json.loads(path.read_text()).items()}


def read_act_table(hidden: int) -> dict[tuple[int, int, int], dict]:
    """``act_tiles_hidden<hidden>.json``: per key the fastest tile with an even wave_frags, which
    the fused gate/up projection with its SiLU-and-multiply runs (empty if there is none)."""
    path = TABLES / f"act_tiles_hidden{hidden}.json"
    if not path.exists():
        return {}
    return {tuple(int(v) for v in key.split(",")): cfg for key, cfg in json.loads(path.read_text()).items()}


def read_chain_table(hidden: int) -> dict[int, dict]:
    """``chain_tiles_hidden<hidden>.json``: per round width M the tile a chained round of that
    hidden size runs fastest on (measured; empty if the size was not tuned)."""
    path = TABLES / f"chain_tiles_hidden{hidden}.json"
    if not path.exists():
        return {}
    return {int(M): cfg for M, cfg in json.loads(path.read_text()).items()}


def round_chain_tile(hidden: int, M: int, act: bool = False) -> dict:
    """The tile of a chained round of hidden size ``hidden`` at width ``M``: the measured entry,
    else ``tiles.packed_chain_tile(M)`` (also when ``act``, a chain with a gate/up link carrying
    its SiLU-and-multiply, meets an entry whose wave_frags is odd)."""
    from .tiles import packed_chain_tile

    cfg = read_chain_table(hidden).get(M)
    if cfg is None or (act and cfg["wave_frags"] % 2):
        cfg = packed_chain_tile(M)
    return dict(cfg)


def load_table(hf_config, width: int) -> dict[tuple[int, int, int], dict]:
    """The five tiles of ``hf_config`` at round width ``width`` (plm/gemm_tables.py:30-43)."""
    path = TABLES / f"tiles_hidden{hf_config.hidden_size}.json"
    table = read_table(hf_config.hidden_size)
    shapes = model_shapes(hf_config)
    wanted = {name: (width, *shape) for name, shape in shapes.items()}
    missing = set(wanted.values()) - set(table)
    if missing:
        raise SystemExit(f"--mode fast has no tuned tile for (width, N, K) {sorted(missing)} in {path.name}; "
                         "use --mode default or a tuned --k")
    configs = {key: table[key] for key in wanted.values()}
    if width > WIDEST_TUNED_DOWN_ROUND:
        configs[wanted["down"]] = DOWN_SPLIT_K1
    return configs


def install(hf_config, width: int) -> None:
    fast_gemm.install(load_table(hf_config, width))
    gate_up = (width, *model_shapes(hf_config)["gate_up"])
    act = read_act_table(hf_config.hidden_size).get(gate_up)
    if act is not None:
        fast_gemm.ACT_CONFIGS[gate_up] = act
