"""CPU checks of the C ABI and the host logic: the library loads, exports every symbol the header
declares, validates arguments before touching the GPU, and the tile tables follow the reference's
contract (plm/gemm_tables.py). No kernel is launched here."""

from __future__ import annotations

import ctypes
import math
import json
import re
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from plm_amd import _lib, fast_gemm, gemm_tables, tiles, workloads

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "plm_amd.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(plm_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert "plm_gemm" in names and "plm_lm_head_verify" in names
    lib = ctypes.CDLL(str(_lib.LIBRARY))
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.EXPORTS)


def test_status_strings():
    lib = _lib.lib()
    assert lib.plm_status_string(0).decode() == "ok"
    for code in (-1, -2, -3, -4, -5):
        assert lib.plm_status_string(code).decode() != "unknown status"


def test_argument_validation_happens_before_launch():
    lib = _lib.lib()
    tile = _lib.Tile(2, 4, 1, 2)
    fake = 1 << 20  # never dereferenced: every call below fails validation first
    # K not a multiple of 8.
    assert lib.plm_gemm(0, fake, 1024, fake, 1024, fake, 4096, 42, 4096, 1020, tile, None, 0, None) == -1
    # M out of range.
    assert lib.plm_gemm(0, fake, 1024, fake, 1024, fake, 4096, 0, 4096, 1024, tile, None, 0, None) == -1
    assert lib.plm_gemm(0, fake, 1024, fake, 1024, fake, 4096, 129, 4096, 1024, tile, None, 0, None) == -1
    # Misaligned pointer.
    assert lib.plm_gemm(0, fake + 2, 1024, fake, 1024, fake, 4096, 42, 4096, 1024, tile, None, 0, None) == -2
    # Unknown dtype.
    assert lib.plm_gemm(7, fake, 1024, fake, 1024, fake, 4096, 42, 4096, 1024, tile, None, 0, None) == -1
    # Split-K without a workspace.
    split = _lib.Tile(2, 4, 4, 2)
    assert lib.plm_gemm(0, fake, 1024, fake, 1024, fake, 4096, 42, 4096, 1024, split, None, 0, None) == -4
    # A tile with no compiled kernel.
    odd = _lib.Tile(3, 4, 1, 4)
    assert lib.plm_gemm(0, fake, 1024, fake, 1024, fake, 4096, 42, 4096, 1024, odd, None, 0, None) == -3
    # Verify: bad round mode, R too large.
    vt = _lib.Tile(2, 4, 1, 4)
    assert lib.plm_lm_head_verify(0, fake, 2048, fake, 2048, 56, 50257, 2048, fake, 0, 0.94, 9, fake, fake, vt, fake,
                                  1 << 30, None) == -1
    assert lib.plm_lm_head_verify(0, fake, 2048, fake, 2048, 65, 50257, 2048, fake, 0, 0.94, 0, fake, fake, vt, fake,
                                  1 << 30, None) == -1
    # Unknown acceptance rule.
    assert lib.plm_lm_head_verify(0, fake, 2048, fake, 2048, 56, 50257, 2048, fake, 2, 0.94, 0, fake, fake, vt, fake,
                                  1 << 30, None) == -1
    # Packed verify: the same checks, K limits, and only row-split tiles without split-K.
    pt = _lib.Tile(2, 1, 1, 2)
    assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 56, 50257, 2048, fake, 0, 0.94, 9, fake, fake, pt, fake,
                                         1 << 30, None) == -1
    assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 65, 50257, 2048, fake, 0, 0.94, 0, fake, fake, pt, fake,
                                         1 << 30, None) == -1
    assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 56, 50257, 2044, fake, 0, 0.94, 0, fake, fake, pt, fake,
                                         1 << 30, None) == -1
    assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 56, 50257, 2048, fake, 0, 0.94, 0, fake, fake, pt, fake,
                                         16, None) == -4
    assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 56, 50257, 2048, fake, -1, 0.94, 0, fake, fake, pt, fake,
                                         1 << 30, None) == -1
    for bad in (_lib.Tile(2, 4, 1, 2), _lib.Tile(2, 1, 2, 2), _lib.Tile(1, 1, 1, 2), _lib.Tile(2, 1, 1, 6)):
        assert lib.plm_lm_head_verify_packed(0, fake, 2048, fake, 56, 50257, 2048, fake, 0, 0.94, 0, fake, fake, bad,
                                             fake, 1 << 30, None) == -3


def test_epilogue_argument_validation_happens_before_launch():
    lib = _lib.lib()
    fake = 1 << 20
    full = (fake, fake, fake, fake, fake, fake, 100, fake, fake, fake, 10, fake, None, None, None)
    # k outside [1, 64].
    assert lib.plm_round_epilogue(0, *full) == -1
    assert lib.plm_round_epilogue(65, *full) == -1
    # Proposals without decisions; a round sequence without its step counter; a negative out length.
    assert lib.plm_round_epilogue(7, None, *full[1:]) == -1
    assert lib.plm_round_epilogue(7, *full[:11], None, *full[12:]) == -1
    assert lib.plm_round_epilogue(7, *full[:6], -1, *full[7:]) == -1
    # An empty round sequence.
    assert lib.plm_round_epilogue(7, *full[:10], 0, *full[11:]) == -1


def test_round_verify_argument_validation_happens_before_launch():
    lib = _lib.lib()
    fake = 1 << 20
    pt = _lib.Tile(2, 1, 1, 2)

    def call(k, verify=fake, rule=0, seq=fake, seq_len=8):
        return lib.plm_round_verify_packed(0, fake, 2048, fake, k, 50257, 2048, rule, 0.94, 0, verify, fake, fake, fake,
                                           100, fake, fake, seq, seq_len, fake, None, None, None, None, pt, fake,
                                           1 << 30, None)

    assert call(0) == -1 and call(8) == -1          # k + k*k must be within 1..64
    assert call(7, verify=None) == -1                # no verify tokens
    assert call(7, rule=3) == -1                     # unknown rule
    assert call(7, seq=None) == -1                   # a step counter without its sequence
    assert call(7, seq_len=0) == -1


def test_packed_argument_validation_happens_before_launch():
    lib = _lib.lib()
    tile = _lib.Tile(2, 4, 1, 2)
    fake = 1 << 20
    # K not a multiple of 8; M out of range; misaligned X; unknown dtype.
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 42, 4096, 1020, tile, None, 0, None) == -1
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 0, 4096, 1024, tile, None, 0, None) == -1
    # Wider than 128 rows: the wide kernel (its own tiling; the tile must still be a valid one).
    # 4096 x 640 at K = 1024 is 160 tiles of 128 x 128, split twice in K: a workspace is needed.
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 640, 4096, 1024, _lib.Tile(2, 4, 1, 3), None, 0,
                               None) == -3
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 640, 4096, 1024, tile, None, 0, None) == -4
    assert lib.plm_gemm_packed(0, fake + 2, 1024, fake, fake, 4096, 640, 4096, 1024, tile, None, 0, None) == -2
    assert lib.plm_gemm_packed_tile_supported(0, 129, 1024, _lib.Tile(4, 1, 1, 4)) == 1
    assert lib.plm_gemm_packed_tile_supported(0, 16, 1024, _lib.Tile(4, 1, 1, 4)) == 1
    assert lib.plm_gemm_packed_workspace_bytes(640, 4096, 1024, tile) == _lib.COUNTER_BYTES + 160 * 2 * 64 * 1024
    assert lib.plm_gemm_packed_workspace_bytes(640, 6144, 2048, tile) == 0   # 240 tiles: no split
    assert lib.plm_gemm_packed(0, fake + 2, 1024, fake, fake, 4096, 42, 4096, 1024, tile, None, 0, None) == -2
    assert lib.plm_gemm_packed(7, fake, 1024, fake, fake, 4096, 42, 4096, 1024, tile, None, 0, None) == -1
    # Split-K without a workspace; a pipeline depth with no kernel.
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 42, 4096, 1024, _lib.Tile(2, 4, 4, 2), None, 0,
                               None) == -4
    assert lib.plm_gemm_packed(0, fake, 1024, fake, fake, 4096, 42, 4096, 1024, _lib.Tile(2, 4, 1, 3), None, 0,
                               None) == -3
    # Packing: K not a multiple of 8, destination too small.
    assert lib.plm_pack_weight(0, fake, 1024, 4096, 1020, fake, 1 << 30, None) == -1
    assert lib.plm_pack_weight(0, fake, 1024, 4096, 1024, fake, 1024, None) == -4
    # A chain whose linear reads a later one's output.
    arr = (_lib.ChainGemm * 2)()
    for g in arr:
        g.x, g.w, g.y, g.ldx, g.ldw, g.ldy, g.N, g.K, g.split_k = fake, fake, fake, 1024, 1024, 1024, 1024, 1024, 1
    arr[0].dep, arr[1].dep = 1, -1
    assert lib.plm_gemm_chain_packed_prepare(arr, 2, 56, tile) == -1


def test_silu_mul_argument_validation_happens_before_launch():
    """plm_gemm_packed_silu_mul and chain links with the SiLU-and-multiply epilogue (out_f32 =
    PLM_OUT_SILU_MUL) refuse what the epilogue cannot do, before touching the device."""
    lib = _lib.lib()
    fake = 1 << 20
    tile = _lib.Tile(2, 8, 1, 2)

    def silu(N, t=tile, ldy=None, y=fake, M=56):
        return lib.plm_gemm_packed_silu_mul(0, fake, 2048, fake, y, N // 2 if ldy is None else ldy, M, N, 2048, t,
                                            None, 0, None)

    assert silu(11264 + 16) == -1                       # N not a multiple of 32
    assert silu(16) == -1                               # fewer than one gate/up pair of fragments
    assert silu(11264, t=_lib.Tile(1, 8, 1, 2)) == -1   # wave_frags 1: gate and up unpaired
    assert silu(11264, ldy=5631) == -1                  # ldy below N/2
    assert silu(11264, ldy=5634) == -1                  # ldy not a multiple of 4
    assert silu(11264, y=fake + 2) == -2                # Y not 8-byte aligned
    assert silu(11264, M=129) == -1                     # the skinny kernel's widths only
    assert silu(11264, t=_lib.Tile(2, 8, 1, 3)) == -3   # no such pipeline depth
    # Chains: an act link needs an even wave_frags, and its reader's K is at most N/2.
    arr = (_lib.ChainGemm * 2)()
    arr[0].x, arr[0].w, arr[0].y, arr[0].ldx, arr[0].ldw, arr[0].ldy = fake, 1 << 33, 1 << 24, 2048, 2048, 5632
    arr[0].N, arr[0].K, arr[0].split_k, arr[0].dep, arr[0].out_f32 = 11264, 2048, 1, -1, _lib.PLM_OUT_SILU_MUL
    arr[1].x, arr[1].w, arr[1].y, arr[1].ldx, arr[1].ldw, arr[1].ldy = 1 << 24, 1 << 34, 1 << 26, 5632, 5632, 2048
    arr[1].N, arr[1].K, arr[1].split_k, arr[1].dep = 2048, 5632, 1, 0

    def chain(t):
        need = lib.plm_gemm_chain_packed_prepare(arr, 2, 56, t)
        assert need > 0
        return lib.plm_gemm_chain_packed(0, arr, fake, 2, 56, t, None, 0, None)

    assert chain(tile) == -4                            # valid: it stops at the missing workspace
    assert chain(_lib.Tile(1, 8, 1, 2)) == -1
    arr[1].K = arr[1].ldw = 5664                        # reads past the activation's 5632 columns
    arr[1].ldx = 5664
    assert chain(tile) == -1


def test_packed_sizes_and_chain_prepare():
    lib = _lib.lib()
    # Fragments of 16 rows x 32 K: N and K round up.
    # Fragment rows padded to a multiple of 16, K steps to a multiple of 8 (50257 rows: 3142
    # fragment rows -> 3152; K 1416: 45 steps -> 48).
    assert lib.plm_packed_weight_bytes(50257, 2048) == 3152 * 64 * 1024
    assert lib.plm_packed_weight_bytes(1000, 1416) == 64 * 48 * 1024
    assert lib.plm_gemm_packed_workspace_bytes(56, 2048, 8192, _lib.Tile(2, 4, 1, 2)) == 0
    # One fp32 fragment (1 KiB) per (tile, split, fragment of the tile).
    tiles_ = math.ceil(2048 / 16 / 2)
    assert lib.plm_gemm_packed_workspace_bytes(56, 2048, 8192, _lib.Tile(2, 4, 4, 2)) == \
        _lib.COUNTER_BYTES + tiles_ * 4 * 2 * 4 * 1024
    # Chains number the consumed linears. Where every linear reads the one before it (tile-done
    # flags, no grid barrier), every linear has its own partials and arrival counters.
    per_linear = 64 * 2 * 2 * 4 * 1024   # tiles x split x fragments x MT x 1 KiB
    arr = (_lib.ChainGemm * 3)()
    for i, g in enumerate(arr):
        g.x, g.w, g.y, g.ldx, g.ldw, g.ldy = 1 << 20, 1 << 21, (1 << 22) + i * (1 << 20), 2048, 2048, 2048
        g.N, g.K, g.split_k, g.dep = 2048, 2048, 2, i - 1
    need = lib.plm_gemm_chain_packed_prepare(arr, 3, 56, _lib.Tile(2, 4, 1, 2))
    assert [g.consumed for g in arr] == [1, 1, 0]
    assert [g.done_base for g in arr] == [1, 2, 0]
    assert [g.arrive_base for g in arr] == [49152, 49152 + 64, 49152 + 128]
    assert [g.partial_offset for g in arr] == [0, per_linear // 4, 2 * per_linear // 4]
    assert need == _lib.COUNTER_BYTES + 3 * per_linear
    # Otherwise (here two linears read the first) a grid barrier follows every consumed linear,
    # and partials and arrival counters are reused after it.
    for i, g in enumerate(arr):
        g.dep = [-1, 0, 0][i]
    need = lib.plm_gemm_chain_packed_prepare(arr, 3, 56, _lib.Tile(2, 4, 1, 2))
    assert [g.consumed for g in arr] == [1, 0, 0]
    assert [g.done_base for g in arr] == [1, 0, 0]
    assert [g.arrive_base for g in arr] == [49152, 49152, 49152 + 64]
    assert [g.partial_offset for g in arr] == [0, 0, per_linear // 4]
    assert need == _lib.COUNTER_BYTES + 2 * per_linear


def test_workspace_sizes():
    lib = _lib.lib()
    m = re.search(r"#define PLM_WORKSPACE_COUNTER_BYTES \(1u << (\d+)\)", HEADER.read_text())
    assert m and _lib.COUNTER_BYTES == 1 << int(m.group(1))
    assert lib.plm_gemm_workspace_bytes(56, 2048, 8192, _lib.Tile(2, 4, 1, 2)) == 0
    n = lib.plm_gemm_workspace_bytes(56, 2048, 8192, _lib.Tile(2, 4, 4, 2))
    assert n == _lib.COUNTER_BYTES + 4 * 56 * 2048 * 4
    # Partial planes pad N to a multiple of 4 floats.
    assert lib.plm_gemm_workspace_bytes(42, 50257, 1024, _lib.Tile(2, 4, 2, 2)) == _lib.COUNTER_BYTES + (2 * 42 * 50260 + 63) // 64 * 64 * 4
    assert lib.plm_lm_head_verify_workspace_bytes(56, 50257, 2048, _lib.Tile(2, 4, 1, 4)) > 56 * 4


def test_default_config_has_a_kernel_at_every_width():
    for M in (1, 7, 33, 56, 64, 110, 128, 129, 200, 256, 640, 1000):
        for N, K in ((2048, 2048), (6144, 2048), (8192, 2048), (2048, 8192), (50257, 2048), (1000, 1416)):
            cfg = fast_gemm.default_config(M, N, K)
            assert fast_gemm.tile_supported(M, K, cfg), (M, N, K, cfg)
            assert cfg["split_k"] >= 1 and math.ceil(K / 32) // cfg["split_k"] >= 2


def test_tile_support_matches_register_budget():
    # Every heuristic tile for the measured shapes has a compiled kernel.
    for w in workloads.WORKLOADS.values():
        for g in w.gemms:
            cfg = tiles.heuristic_tile(w.M, g.N, g.K)
            assert fast_gemm.tile_supported(w.M, g.K, cfg), (g, cfg)
    assert not fast_gemm.tile_supported(56, 2048, {"wave_frags": 4, "k_waves": 8, "split_k": 1, "unroll": 8})
    # The Python mirror of the compiled set agrees with the library everywhere.
    for M in (1, 7, 16, 17, 42, 56, 64, 65, 110, 128):
        for nf in (1, 2, 3, 4):
            for u in (1, 2, 4, 8):
                for kw in (1, 4, 8, 16, 5):
                    cfg = {"wave_frags": nf, "k_waves": kw, "split_k": 1, "unroll": u}
                    assert tiles.compiled(M, cfg) == fast_gemm.tile_supported(M, 2048, cfg), (M, cfg)


# --------------------------------------------------------------------------- tile tables


def llama(hidden, intermediate, heads, kv_heads, vocab=50257):
    return SimpleNamespace(hidden_size=hidden, intermediate_size=intermediate, head_dim=hidden // heads,
                           num_attention_heads=heads, num_key_value_heads=kv_heads, vocab_size=vocab)


def test_model_shapes_follow_reference_formula():
    cfg = llama(2048, 5632, 16, 4)
    shapes = gemm_tables.model_shapes(cfg)
    assert shapes == {"qkv": (3072, 2048), "o": (2048, 2048), "gate_up": (11264, 2048), "down": (2048, 5632),
                      "lm_head": (50304, 2048)}


def test_every_table_covers_the_reference_keys():
    # The reference's tile tables' keys (plm/gpu_tuning/*.json), at the widths it tunes.
    expect = {
        512: {(42, 768, 512), (42, 512, 512), (42, 2816, 512), (42, 512, 1408), (42, 50304, 512)},
        768: {(42, 1152, 768), (42, 768, 768), (42, 4096, 768), (42, 768, 2048), (42, 50304, 768)},
        1024: {(42, 1536, 1024), (42, 1024, 1024), (42, 5120, 1024), (42, 1024, 2560), (42, 50304, 1024)},
        2048: {(w, n, k) for w in (42, 56, 110)
               for n, k in ((3072, 2048), (2048, 2048), (11264, 2048), (2048, 5632), (50304, 2048))},
        3072: {(w, n, k) for w in (42, 56, 110)
               for n, k in ((4608, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (50304, 3072))},
    }
    for hidden, keys in expect.items():
        table = gemm_tables.read_table(hidden)
        assert keys <= set(table), (hidden, sorted(keys - set(table)))


def test_tables_hold_only_compiled_tiles():
    for path in sorted(gemm_tables.TABLES.glob("tiles_hidden*.json")):
        for key, cfg in json.loads(path.read_text()).items():
            M, N, K = map(int, key.split(","))
            assert set(cfg) == {"wave_frags", "k_waves", "split_k", "unroll"}, (path.name, key)
            assert fast_gemm.tile_supported(M, K, cfg), (path.name, key, cfg)


def test_act_tables_pair_gate_and_up_fragments():
    """act_tiles_hidden<H>.json covers every key of tiles_hidden<H>.json with a compiled tile whose
    wave_frags is even (the SiLU-and-multiply epilogue pairs gate and up fragments), and
    gemm_tables.install puts the gate/up projection's entry where gate_up_silu reads it."""
    for path in sorted(gemm_tables.TABLES.glob("tiles_hidden*.json")):
        hidden = int(path.stem.removeprefix("tiles_hidden"))
        act = gemm_tables.read_act_table(hidden)
        assert set(act) == set(gemm_tables.read_table(hidden)), path.name
        for (M, N, K), cfg in act.items():
            assert cfg["wave_frags"] % 2 == 0 and fast_gemm.tile_supported(M, K, cfg), (hidden, M, N, K, cfg)

    class Cfg:   # the 1.3B Llama shapes
        hidden_size, intermediate_size, head_dim = 2048, 5632, 64
        num_attention_heads, num_key_value_heads, vocab_size = 32, 8, 50257

    try:
        gemm_tables.install(Cfg, 56)
        assert fast_gemm.ACT_CONFIGS[(56, 11264, 2048)] == gemm_tables.read_act_table(2048)[(56, 11264, 2048)]
    finally:
        fast_gemm.uninstall()
    assert not fast_gemm.ACT_CONFIGS


def test_chain_tables_hold_compiled_tiles_and_fall_back_to_the_rule():
    """chain_tiles_hidden<H>.json: one tile per round width, each a compiled packed tile for that
    width (tile_supported) with the fields a chain reads; a width or hidden size without an entry
    gets tiles.packed_chain_tile."""
    from plm_amd import tiles

    paths = sorted(gemm_tables.TABLES.glob("chain_tiles_hidden*.json"))
    assert paths
    for path in paths:
        hidden = int(path.stem.removeprefix("chain_tiles_hidden"))
        table = gemm_tables.read_chain_table(hidden)
        assert table, path.name
        for M, cfg in table.items():
            assert set(cfg) == {"wave_frags", "k_waves", "split_k", "unroll"} and cfg["split_k"] == 1, (hidden, M)
            assert fast_gemm.tile_supported(M, hidden, cfg), (hidden, M, cfg)
            assert gemm_tables.round_chain_tile(hidden, M) == cfg
    assert gemm_tables.round_chain_tile(2560, 42) == tiles.packed_chain_tile(42)
    assert gemm_tables.round_chain_tile(1536, 56) == tiles.packed_chain_tile(56)
    for path in paths:
        hidden = int(path.stem.removeprefix("chain_tiles_hidden"))
        for M in gemm_tables.read_chain_table(hidden):
            assert gemm_tables.round_chain_tile(hidden, M, act=True)["wave_frags"] % 2 == 0


def test_tuner_tie_rules():
    """Per-GEMM tables: a tie within 1 % goes to the fastest even wave_frags; outside it, the fastest
    tile. Chain tables: the width's default chain tile wins a tie, else the fastest."""
    from plm_amd import tune

    odd, even = {"wave_frags": 1, "k_waves": 8, "split_k": 1, "unroll": 2}, {"wave_frags": 2, "k_waves": 8,
                                                                             "split_k": 1, "unroll": 2}
    assert tune.pick([(10.0, odd), (10.05, even)]) == (even, 10.05)
    assert tune.pick([(10.0, odd), (10.2, even)]) == (odd, 10.0)
    default = tiles.packed_chain_tile(56)
    other = dict(default, wave_frags=4, k_waves=4)
    assert tune._pick_chain([(10.0, other), (10.05, default)], default) == (default, 10.05)
    assert tune._pick_chain([(10.0, other), (10.5, default)], default) == (other, 10.0)
    assert tune._pick_chain([(10.0, other)], default) == (other, 10.0)


def test_load_table_missing_hidden_size_exits():
    with pytest.raises(SystemExit, match="no tile table for hidden size 1536"):
        gemm_tables.load_table(llama(1536, 4096, 12, 12), 42)


def test_load_table_missing_shape_exits():
    # hidden 1024 is tuned only at width 42.
    with pytest.raises(SystemExit, match="no tuned tile"):
        gemm_tables.load_table(llama(1024, 2560, 16, 4), 56)


def test_load_table_wide_round_overrides_down():
    cfg = llama(2048, 5632, 16, 4)
    table = gemm_tables.load_table(cfg, 110)
    assert table[(110, 2048, 5632)] == gemm_tables.DOWN_SPLIT_K1
    narrow = gemm_tables.load_table(cfg, 56)
    assert narrow[(56, 2048, 5632)] == gemm_tables.read_table(2048)[(56, 2048, 5632)]
    assert len(table) == 5


def test_fast_gemm_routes_only_eligible_calls(monkeypatch):
    calls = []
    monkeypatch.setattr(fast_gemm, "hip_linear", lambda a, w, cfg, out=None: calls.append(cfg) or "hip")
    monkeypatch.setitem(fast_gemm.CONFIGS, (4, 16, 8), {"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 2})
    x = torch.randn(4, 8).bfloat16()
    w = torch.randn(16, 8).bfloat16()
    assert fast_gemm.fast_gemm(None, x, w) == "hip"                      # tuned, eligible
    assert torch.is_tensor(fast_gemm.fast_gemm(None, x, w, torch.zeros(16).bfloat16()))   # bias -> F.linear
    assert torch.is_tensor(fast_gemm.fast_gemm(None, x.float(), w.float()))              # fp32 -> F.linear
    assert torch.is_tensor(fast_gemm.fast_gemm(None, x[None], w))                          # 3-D -> F.linear
    assert torch.is_tensor(fast_gemm.fast_gemm(None, torch.randn(5, 8).bfloat16(), w))    # untuned M
    assert len(calls) == 1


def test_install_rejects_uncompiled_tiles():
    with pytest.raises(ValueError, match="no compiled MI355X kernel"):
        fast_gemm.install({(56, 2048, 2048): {"wave_frags": 3, "k_waves": 8, "split_k": 1, "unroll": 8}})
    assert (56, 2048, 2048) not in fast_gemm.CONFIGS


def test_install_sets_the_dispatch_slot():
    try:
        fast_gemm.install({(42, 4096, 1024): tiles.heuristic_tile(42, 4096, 1024)})
        assert fast_gemm.dispatch_unquantized_gemm() is fast_gemm.fast_gemm
    finally:
        fast_gemm.uninstall()
    assert fast_gemm.dispatch_unquantized_gemm() is not fast_gemm.fast_gemm


def test_workload_bytes_match_the_published_roofline_table():
    assert workloads.SINGLE_GEMM.bytes == 8_818_688
    assert workloads.BLOCK_1P3B.bytes == 104_333_312
    assert workloads.ROUND_1P3B.bytes == 2_715_710_320
    assert workloads.ROUND_3B.bytes == 5_443_196_784
    for M, b in zip(workloads.M_SWEEP, (2_633_514_094, 2_645_256_412, 2_668_741_048, 2_692_225_684, 2_715_710_320)):
        assert workloads.ROUND_1P3B.at(M).bytes == b


def _chain_table(widths, K0, base=1 << 30, pad=None, dep_prev=True):
    """A chain of linears x -> y_0 -> y_1 -> ... over fake, never-dereferenced device pointers:
    widths[i] output columns; rows of y_i ``pad(widths[i])`` elements apart (default: unpadded)."""
    n = len(widths)
    arr = (_lib.ChainGemm * n)()
    addr = base
    ldys = [pad(w) if pad else w for w in widths]
    ys = []
    for ld in ldys:
        ys.append(addr)
        addr += (56 * ld * 2 + 4095) // 4096 * 4096
    for i, w in enumerate(widths):
        g = arr[i]
        g.x = base - (1 << 24) if i == 0 else ys[i - 1]
        g.w = addr + (i << 26)
        g.y = ys[i]
        g.ldx = K0 if i == 0 else ldys[i - 1]
        g.ldw = g.K = K0 if i == 0 else widths[i - 1]
        g.ldy = ldys[i]
        g.N = w
        g.split_k = 1
        g.dep = (i - 1) if (dep_prev and i > 0) else -1
    return arr


def test_chain_sync_mode_requires_line_aligned_consumed_rows():
    """Tile-flag waits widen a wavefront's columns to whole 128-byte lines of one row; they are only
    chosen when no line can span two rows of a consumed Y (y 128-byte aligned, ldy % 64 == 0)."""
    lib = _lib.lib()
    tile = _lib.Tile(2, 8, 1, 2)
    mode = lambda arr: lib.plm_gemm_chain_packed_sync_mode(arr, len(arr), tile)  # noqa: E731
    assert mode(_chain_table([2048, 8192, 2048], 2048)) == 2
    # A consumed width that is not a multiple of 64 elements: rows 2000 B apart.
    assert mode(_chain_table([1000, 2048, 512], 1024)) == 1
    # The same widths with the rows padded to a multiple of 64 elements.
    assert mode(_chain_table([1000, 2048, 512], 1024, pad=lambda w: -(-w // 64) * 64)) == 2
    # The last linear is read by none: its Y may have any width.
    assert mode(_chain_table([2048, 1000], 1024)) == 2
    # A consumed Y that starts off a 128-byte boundary.
    arr = _chain_table([2048, 2048, 512], 1024)
    arr[0].y += 64
    arr[1].x = arr[0].y
    assert mode(arr) == 1
    # No dependencies at all, and any other dependency pattern.
    assert mode(_chain_table([2048, 2048], 1024, dep_prev=False)) == 0
    arr = _chain_table([2048, 2048, 2048], 2048)
    arr[2].dep = 0
    assert mode(arr) == 1
    assert lib.plm_gemm_chain_packed_sync_mode(arr, 0, tile) == -1
    assert lib.plm_gemm_chain_packed_sync_mode(arr, 3, _lib.Tile(3, 8, 1, 2)) == -3


def test_voronoi_argument_validation_happens_before_launch():
    lib = _lib.lib()
    fake = 1 << 20  # never dereferenced: every call below fails validation first

    def assign(n=7, V=50257, A=1024, M=128, k=8, rounds=2, values=fake, decoded=fake, ws=fake, ws_bytes=1 << 30,
               dtype=0, ld=50264):
        return lib.plm_voronoi_assign(dtype, fake, ld, fake, n, V, A, M, k, rounds, 12, 0.1, 0.15, 0.35, 1.9, 0.0087,
                                      0.25, values, decoded, None, None, None, None, ws, ws_bytes, None)

    assert assign(M=100) == -1                       # n_targets a power of two
    assert assign(M=256) == -1                       # at most 128 (the key's 7 target bits)
    assert assign(k=3) == -1 and assign(k=32) == -1  # k a power of two <= 16
    assert assign(A=1000) == -1 and assign(A=16384) == -1
    assert assign(A=8192, k=8) == -1                 # k * A / 1024 <= 32
    assert assign(V=65529) == -1 and assign(V=64) == -1
    assert assign(n=0) == -1 and assign(rounds=0) == -1
    assert assign(dtype=2) == -1
    assert assign(ld=50000) == -1                    # a row stride below the vocabulary
    assert assign(values=None) == -1                 # values and decoded go together
    assert assign(ws=None) == -4 and assign(ws_bytes=1024) == -4
    need = lib.plm_voronoi_assign_workspace_bytes(7, 128, 8, 1024)
    assert need >= _lib.COUNTER_BYTES + 7 * 8 * 1024 * 4
    assert lib.plm_voronoi_assign_workspace_bytes(0, 128, 8, 1024) == 0
    assert lib.plm_voronoi_fit(fake, fake, fake, fake, 7, 128, 8, 1024, 12, -0.1, 1.9, 0.0087, 0.25, fake, None) == -1
    assert lib.plm_voronoi_fit(fake, fake, fake, fake, 7, 128, 16, 4096, 12, 0.15, 1.9, 0.0087, 0.25, fake, None) == -1
    assert lib.plm_voronoi_condense(0, fake, 50257, 1024, fake, fake, 7, 128, 256, fake, None) == -1
    assert lib.plm_voronoi_spread(0, fake, 50257, 1024, fake, 7, 128, 65, fake, None) == -1
    assert lib.plm_voronoi_shortlist(0, fake, 50257, fake, 7, 50257, 1024, 128, 0.1, None, fake, None, fake, fake,
                                     None, None) == -1
    tile = _lib.Tile(2, 1, 1, 2)
    # The verify rows' logits are the model dtype's: fp32 rounding is refused, as are misaligned rows.
    assert lib.plm_lm_head_verify_packed_logits(0, fake, 2048, fake, 56, 50257, 2048, fake, 6, 0, 0.94, 0, fake, fake,
                                                fake, 50264, 7, tile, fake, 1 << 30, None) == -1
    assert lib.plm_lm_head_verify_packed_logits(0, fake, 2048, fake, 56, 50257, 2048, fake, 6, 0, 0.94, 1, fake, fake,
                                                fake, 50260, 7, tile, fake, 1 << 30, None) == -2
    assert lib.plm_lm_head_verify_packed_logits(0, fake, 2048, fake, 56, 50257, 2048, fake, 57, 0, 0.94, 1, fake, fake,
                                                fake, 50264, 7, tile, fake, 1 << 30, None) == -1


def test_voronoi_host_checks_refuse_cpu_and_bad_sizes():
    from plm_amd import voronoi

    with pytest.raises(RuntimeError, match="GPU only"):
        voronoi.Voronoi.from_table(torch.zeros(300, 64, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        voronoi.Voronoi.from_table(torch.zeros(300, 64, dtype=torch.float32))
    with pytest.raises(ValueError):
        voronoi._check_sizes(7, 50257, 1000, 128)
    with pytest.raises(ValueError):
        voronoi._check_sizes(7, 50257, 8192, 128, 8)
    voronoi._check_sizes(7, 50257, 8192, 128, 4)
    with pytest.raises(ValueError):
        voronoi.LogitVoronoiAuxiliary(1024, 64, 1000, top_m=96)
    with pytest.raises(ValueError):
        voronoi.LogitVoronoiAuxiliary(1024, 64, 1000, backend="exact")
    scheme = voronoi.LogitVoronoiAuxiliary(1024, 64, 1000)
    assert scheme.masked_value == 1024 and scheme.placeholder_token_id == 1000
    assert set(scheme.state_dict()) == {"auxiliary_vocabulary", "mask_auxiliary"}


def test_chain_check_resets_the_whole_counter_area(monkeypatch):
    """A chained launch whose wait gave up can leave any counter of the shared workspace off zero
    (a late workgroup counting in after the owner's reset): check() raises and zeroes the whole
    counter area, not only the error int, and leaves the scratch past it alone."""
    from plm_amd.chain import LinearChain

    ws = torch.full((_lib.COUNTER_BYTES + 4096,), 7, dtype=torch.uint8)
    ws[: _lib.COUNTER_BYTES].view(torch.int32)[_lib.ERROR_INDEX] = 1
    chain = LinearChain.__new__(LinearChain)
    chain.ws, chain.device, chain.links = ws, torch.device("cpu"), [None]
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    with pytest.raises(RuntimeError, match="give up"):
        chain.check()
    assert int(ws[: _lib.COUNTER_BYTES].count_nonzero()) == 0
    assert bool((ws[_lib.COUNTER_BYTES:] == 7).all())
    chain.check()  # a clean workspace passes
