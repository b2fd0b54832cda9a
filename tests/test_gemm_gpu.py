"""GPU parity of the HIP skinny GEMM against the CPU oracle (the reference's own F.linear path).

Tolerance, per output element of the bf16/fp16 result:
* within one rounding of the exact (fp64) product, up to fp32 accumulation error:
  |got - exact| <= ulp(exact) + 2^-20 * sum_k |x_k w_k|;
* against the oracle's own rounded output: within 1e-3 relative / 2e-2 absolute, or one step of
  the output dtype apart (two correctly rounded values of sums taken in different orders can
  land on either side of a rounding midpoint; at |y| >= 4 one bf16 step, 2^-5, exceeds the
  absolute tolerance), with at most 0.1% of the elements one step apart.
The fp32 accumulator itself (``hip_linear_f32``) is held to 1e-3 relative / 2e-2 absolute and
tighter."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from conftest import golden_names, load_golden
from plm_amd import fast_gemm, gemm_tables, tiles, tune, workloads
from plm_amd.fast_gemm import hip_linear, hip_linear_f32

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-2


def _inputs(M, N, K, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    return x, w


def _inputs_on_gpu(M, N, K, seed, device, dtype=torch.bfloat16):
    """Large weights drawn directly on the GPU (seeded); the oracle reads a CPU copy of the rows it
    checks, so both sides see the same bits."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=device).to(dtype)
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).to(dtype)
    return x, w


def check_cols(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, cols: torch.Tensor):
    """Columns ``cols`` of GPU ``y`` against the oracle on CPU copies of x and of those W rows."""
    cols_d = cols.to(w.device)
    got = y[:, cols_d].cpu().float()
    xc, wc = x.cpu(), w[cols_d].cpu()
    _assert_parity(got, xc, wc)


def _ulp(v: torch.Tensor, dtype) -> torch.Tensor:
    bits = 8 if dtype == torch.bfloat16 else 11
    e = torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -14)))
    return 2.0 ** (e - (bits - 1))


def _assert_parity(got: torch.Tensor, x: torch.Tensor, w: torch.Tensor) -> None:
    _within_one_rounding(got, x, w)
    ref = oracle.linear(x, w).float()
    diff = (got - ref).abs()
    in_tol = diff <= ATOL + RTOL * ref.abs()
    one_step = diff <= _ulp(ref, x.dtype) * 1.0001
    assert bool((in_tol | one_step).all()), f"max |got - oracle| {diff.max():.4g}"
    assert int((~in_tol).sum()) <= max(1, got.numel() // 1000), int((~in_tol).sum())


def _within_one_rounding(got: torch.Tensor, x: torch.Tensor, w: torch.Tensor) -> None:
    """Each output is the fp64 product rounded once to the output dtype, up to fp32 accumulation
    error: |got - exact| <= ulp(exact) + 2^-20 * sum_k |x_k w_k|. The second term matters only
    where the dot product cancels to a value much smaller than its terms."""
    exact = torch.from_numpy(oracle.linear_fp64(x, w))
    absdot = x.double().abs() @ w.double().abs().T
    bound = _ulp(exact, x.dtype) + 2.0 ** -20 * absdot
    err = (got.double() - exact).abs()
    assert bool((err <= bound).all()), f"max error {err.max():.3g}, worst ratio {(err / bound).max():.3g}"


def check(y: torch.Tensor, x: torch.Tensor, w: torch.Tensor):
    """GPU ``y`` against the oracle on the CPU operands x, w."""
    wc = w
    got = y.cpu().float()
    _assert_parity(got, x, wc)


def _run(x, w, cfg, device):
    return hip_linear(x.to(device), w.to(device), cfg)


@pytest.mark.parametrize("which", ["table", "heuristic"])
def test_single_gemm_350m_mlp_up(device, which):
    M, N, K = 42, 4096, 1024
    x, w = _inputs(M, N, K, 1)
    cfg = gemm_tables.read_table(1024)[(M, N, K)] if which == "table" else tiles.heuristic_tile(M, N, K)
    check(_run(x, w, cfg, device), x, w)


@pytest.mark.parametrize("gemm", workloads.gpt_block(2048, 8192), ids=lambda g: g.name)
def test_block_1p3b(device, gemm):
    M = 56
    x, w = _inputs(M, gemm.N, gemm.K, 2)
    cfg = gemm_tables.read_table(2048)[(M, gemm.N, gemm.K)]
    check(_run(x, w, cfg, device), x, w)


@pytest.mark.parametrize("M", workloads.M_SWEEP)
def test_lm_head_m_sweep(device, M):
    N, K = workloads.GPT2_VOCAB, 2048
    x, w = _inputs_on_gpu(M, N, K, 3, device)
    cols = torch.cat([torch.arange(0, 96), torch.randperm(N, generator=torch.Generator().manual_seed(M))[:400],
                      torch.arange(N - 81, N)])
    check_cols(hip_linear(x, w, gemm_tables.read_table(2048)[(M, N, K)]), x, w, cols)


@pytest.mark.parametrize("shape", [(56, 2048, 2048), (42, 4096, 1024), (56, 2048, 8192), (110, 2048, 2048)])
def test_every_candidate_tile(device, shape):
    M, N, K = shape
    x, w = _inputs(M, N, K, 4)
    xd, wd = x.to(device), w.to(device)
    cands = tiles.candidates(M, N, K, lambda c: fast_gemm.tile_supported(M, K, c))
    assert cands
    for cfg in cands:
        y = hip_linear(xd, wd, cfg)
        check(y, x, w)


@pytest.mark.parametrize("M", [1, 15, 16, 17, 33, 64, 65, 96, 97, 110, 128])
def test_round_widths_edge_cases(device, M):
    N, K = 1000, 1416   # N not a multiple of any tile; K a multiple of 8 but not of 32
    x, w = _inputs(M, N, K, 5)
    supported = lambda c: fast_gemm.tile_supported(M, K, c)  # noqa: E731
    for cfg in (tiles.heuristic_tile(M, N, K, supported=supported),
                {"wave_frags": 4, "k_waves": 4, "split_k": 1, "unroll": 4},   # 64-row tiles (M <= 80)
                {"wave_frags": 4, "k_waves": 4, "split_k": 3, "unroll": 2},
                {"wave_frags": 4, "k_waves": 1, "split_k": 1, "unroll": 6},   # depth capped where it spills
                {"wave_frags": 1, "k_waves": 4, "split_k": 3, "unroll": 2},
                {"wave_frags": 1, "k_waves": 1, "split_k": 1, "unroll": 2},
                {"wave_frags": 2, "k_waves": 1, "split_k": 3, "unroll": 4},
                {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2},
                # eight wavefronts stage X two K steps at a time from MT = 4: odd step ranges per
                # wavefront and split, the masked last step inside a pair
                {"wave_frags": 2, "k_waves": 8, "split_k": 3, "unroll": 4},
                {"wave_frags": 4, "k_waves": 8, "split_k": 2, "unroll": 6},
                {"wave_frags": 1, "k_waves": 16, "split_k": 2, "unroll": 2}):
        if supported(cfg):
            check(_run(x, w, cfg, device), x, w)


def test_seeded_random_shapes_and_tiles(device):
    """Forty seeded random (M, N, K) with a random compiled tile each (every layout, split and depth
    the library has for the width): K a multiple of 8 from 8 to 4096, so K steps per wavefront come
    out odd or even, pairs of X steps straddle item and split ends, and the last step is masked;
    each product against the oracle."""
    rng = torch.Generator().manual_seed(2026)
    checked = 0
    for case in range(40):
        M = int(torch.randint(1, 129, (1,), generator=rng))
        N = int(torch.randint(16, 3001, (1,), generator=rng))
        K = 8 * int(torch.randint(1, 513, (1,), generator=rng))
        cands = tiles.candidates(M, N, K, lambda c: fast_gemm.tile_supported(M, K, c))
        if not cands:
            continue
        cfg = cands[int(torch.randint(0, len(cands), (1,), generator=rng))]
        x, w = _inputs(M, N, K, 100 + case)
        print(f"case {case}: M={M} N={N} K={K} {cfg}", flush=True)
        check(_run(x, w, cfg, device), x, w)
        checked += 1
    assert checked >= 30


def test_split_k_is_deterministic_and_consistent(device):
    M, N, K = 56, 2048, 8192
    x, w = _inputs(M, N, K, 6)
    xd, wd = x.to(device), w.to(device)
    split = {"wave_frags": 2, "k_waves": 4, "split_k": 8, "unroll": 2}
    a = hip_linear_f32(xd, wd, split)
    b = hip_linear_f32(xd, wd, split)
    assert torch.equal(a, b)
    single = hip_linear_f32(xd, wd, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2})
    torch.testing.assert_close(a, single, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(a.cpu(), oracle.linear_fp32(x, w), rtol=1e-4, atol=1e-4)


def test_workspace_shared_across_shapes_and_entry_points(device):
    # Split-K GEMMs with different tile counts, and the verify step, take turns on one workspace:
    # each must find the counter area zero whatever the previous call left in the scratch area.
    from plm_amd.verify import lm_head_verify

    cases = [((56, 6144, 2048), {"wave_frags": 2, "k_waves": 4, "split_k": 4, "unroll": 2}),
             ((56, 8192, 2048), {"wave_frags": 2, "k_waves": 4, "split_k": 2, "unroll": 2}),
             ((56, 2048, 2048), {"wave_frags": 1, "k_waves": 4, "split_k": 8, "unroll": 2}),
             ((56, 8192, 2048), {"wave_frags": 1, "k_waves": 4, "split_k": 3, "unroll": 2})]
    for i, ((M, N, K), cfg) in enumerate(cases):
        x, w = _inputs(M, N, K, 40 + i)
        check(_run(x, w, cfg, device), x, w)
        xv, wv = _inputs(56, 3000, K, 50 + i)
        lm_head_verify(xv.to(device), wv.to(device), torch.zeros(56, dtype=torch.int64, device=device), 0.9)


def test_fp16(device):
    M, N, K = 56, 3072, 2048
    x, w = _inputs(M, N, K, 7, torch.float16)
    for cfg in ({"wave_frags": 2, "k_waves": 4, "split_k": 2, "unroll": 2},
                {"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 2},
                {"wave_frags": 2, "k_waves": 1, "split_k": 2, "unroll": 2}):
        check(_run(x, w, cfg, device), x, w)


def test_small_integers_are_exact(device):
    M, N, K = 56, 512, 2048
    g = torch.Generator().manual_seed(8)
    x = torch.randint(-2, 3, (M, K), generator=g).bfloat16()
    w = torch.randint(-1, 2, (N, K), generator=g).bfloat16()
    exact = oracle.linear_fp64(x, w)
    assert abs(exact).max() < 256
    for cfg in ({"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2},
                {"wave_frags": 1, "k_waves": 4, "split_k": 4, "unroll": 2},
                {"wave_frags": 1, "k_waves": 1, "split_k": 1, "unroll": 8},
                {"wave_frags": 2, "k_waves": 1, "split_k": 4, "unroll": 2},
                {"wave_frags": 2, "k_waves": 8, "split_k": 3, "unroll": 4},
                {"wave_frags": 1, "k_waves": 16, "split_k": 1, "unroll": 2}):
        y = _run(x, w, cfg, device).cpu().double().numpy()
        assert (y == exact).all()


def test_one_hot_weight_selects_columns(device):
    M, K = 42, 1024
    x, _ = _inputs(M, 1, K, 9)
    cols = torch.tensor([0, 5, 1023, 512, 77, 31, 32, 999])
    w = torch.zeros(len(cols), K).bfloat16()
    w[torch.arange(len(cols)), cols] = 1.0
    y = _run(x, w, {"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 2}, device)
    assert torch.equal(y.cpu(), x[:, cols])


def test_strided_activation_view(device):
    # X as the first K columns of a wider buffer (ldx > K), as when a QKV output feeds the next GEMM.
    M, N, K = 56, 2048, 2048
    g = torch.Generator().manual_seed(10)
    wide = torch.randn(M, 3 * K, generator=g).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16()
    xd = wide.to(device)[:, :K]
    assert xd.stride(0) == 3 * K
    y = hip_linear(xd, w.to(device), gemm_tables.read_table(2048)[(M, N, K)])
    check(y, wide[:, :K].contiguous(), w)


def test_lm_head_every_column_at_the_bench_tile(device):
    """The LM head 2048 -> 50257 at M = 56 with the tile the benchmark runs, every column checked."""
    M, N, K = 56, workloads.GPT2_VOCAB, 2048
    x, w = _inputs_on_gpu(M, N, K, 31, device)
    y = hip_linear(x, w, gemm_tables.read_table(2048)[(M, N, K)])
    check(y, x.cpu(), w.cpu())


# Elements of the round's linears (M = 56, table tiles) outside 1e-3 rel / 2e-2 abs of the oracle but
# one output step from it: the two sums are taken in different orders and land on either side of a
# rounding midpoint. Bounded at 0.1 % by _assert_parity; the measured rate is printed here.
@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 2048), (8192, 2048), (2048, 8192), (50257, 2048)])
def test_one_step_rate_at_round_shapes(device, N, K):
    M = 56
    x, w = _inputs_on_gpu(M, N, K, 32, device)
    y = hip_linear(x, w, gemm_tables.read_table(2048)[(M, N, K)]).cpu().float()
    xc, wc = x.cpu(), w.cpu()
    check(y, xc, wc)
    ref = oracle.linear(xc, wc).float()
    diff = (y - ref).abs()
    beyond = int((diff > ATOL + RTOL * ref.abs()).sum())
    print(f"one-step elements N={N} K={K}: {beyond} of {y.numel()} ({100.0 * beyond / y.numel():.4f} %), "
          f"bit-equal to the oracle: {100.0 * float((diff == 0).float().mean()):.2f} %")
    assert beyond <= y.numel() // 1000


def test_wide_round_down_override(device):
    """At round width 110 (k = 10) the reference forces `down` to a split-K tile of its own
    (plm/gemm_tables.py:17-19, 41-42): installed through gemm_tables, fast_gemm routes the 1.3B
    down projection (5632 -> 2048) to DOWN_SPLIT_K1 and the result matches the oracle."""
    from types import SimpleNamespace

    cfg = SimpleNamespace(hidden_size=2048, intermediate_size=5632, head_dim=128, num_attention_heads=16,
                          num_key_value_heads=4, vocab_size=50257)
    try:
        gemm_tables.install(cfg, 110)
        assert fast_gemm.CONFIGS[(110, 2048, 5632)] == gemm_tables.DOWN_SPLIT_K1
        x, w = _inputs(110, 2048, 5632, 33)
        y = fast_gemm.dispatch_unquantized_gemm()(None, x.to(device), w.to(device))
        check(y, x, w)
        direct = hip_linear(x.to(device), w.to(device), gemm_tables.DOWN_SPLIT_K1)
        assert torch.equal(y, direct)
    finally:
        fast_gemm.uninstall()


def test_fast_gemm_install_routes_table_shapes(device):
    from types import SimpleNamespace

    cfg = SimpleNamespace(hidden_size=2048, intermediate_size=5632, head_dim=128, num_attention_heads=16,
                          num_key_value_heads=4, vocab_size=50257)
    try:
        gemm_tables.install(cfg, 56)
        gemm = fast_gemm.dispatch_unquantized_gemm()
        for (M, N, K) in gemm_tables.load_table(cfg, 56):
            x, w = _inputs_on_gpu(M, N, K, 11, device)
            cols = torch.cat([torch.arange(0, min(N, 320)), torch.arange(N - 64, N)])
            check_cols(gemm(None, x, w), x, w, cols)
        x, w = _inputs(57, 64, 2048, 12)     # untuned width: F.linear on the GPU
        torch.testing.assert_close(gemm(None, x.to(device), w.to(device)).cpu().float(),
                                   oracle.linear(x, w).float(), rtol=RTOL, atol=ATOL)
    finally:
        fast_gemm.uninstall()


@pytest.mark.parametrize("hidden", tune.all_hidden())
def test_every_table_entry(device, hidden):
    table = gemm_tables.read_table(hidden)
    for (M, N, K), cfg in table.items():
        x, w = _inputs_on_gpu(M, N, K, 13, device)
        cols = torch.cat([torch.arange(0, min(N, 160)), torch.arange(max(0, N - 70), N)]).unique()
        check_cols(hip_linear(x, w, cfg), x, w, cols)


@pytest.mark.parametrize("gemm", workloads.gpt_block(2560, 10240), ids=lambda g: g.name)
def test_config4_linears_all_columns(device, gemm):
    """Config 4's block linears (hidden 2560) at M = 56 with their table tiles, every column
    against the oracle (test_every_table_entry samples columns of every key)."""
    M = 56
    x, w = _inputs(M, gemm.N, gemm.K, 15)
    check(_run(x, w, gemm_tables.read_table(2560)[(M, gemm.N, gemm.K)], device), x, w)


def test_graph_capture_and_replay(device):
    shapes = [(56, 2048, 8192), (56, 6144, 2048), (56, 2048, 2048)]
    table = gemm_tables.read_table(2048)
    data = [_inputs(*s, 14 + i) for i, s in enumerate(shapes)]
    dev = [(x.to(device), w.to(device)) for x, w in data]
    outs = [torch.empty(s[0], s[1], device=device, dtype=torch.bfloat16) for s in shapes]
    cfgs = [table[s] for s in shapes]
    for (x, w), o, c in zip(dev, outs, cfgs):
        hip_linear(x, w, c, o)                        # eager: sizes the workspace
    eager = [o.clone() for o in outs]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for (x, w), o, c in zip(dev, outs, cfgs):
            hip_linear(x, w, c, o)
    for rep in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), rep
        hip_linear(dev[0][0], dev[0][1], cfgs[0], outs[0])   # eager work between replays
        torch.cuda.synchronize()
    check(outs[1], *data[1])


@pytest.mark.parametrize("cfg", [{"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 2},
                                 {"wave_frags": 2, "k_waves": 4, "split_k": 4, "unroll": 2}],
                         ids=lambda c: f"nf{c['wave_frags']}s{c['split_k']}")
def test_rowmajor_streaming_kernel(device, cfg):
    # plm_gemm reads W row-major (no packed copy): the same parity bar.
    from plm_amd.fast_gemm import hip_linear_rowmajor

    for (M, N, K) in ((56, 2048, 2048), (42, 1000, 1416)):
        x, w = _inputs(M, N, K, 16)
        check(hip_linear_rowmajor(x.to(device), w.to(device), cfg), x, w)


def test_packed_weight_cache_follows_the_tensor(device):
    # The packed copy is made once per weight and remade when the weight changes in place.
    M, N, K = 56, 512, 1024
    x, w = _inputs(M, N, K, 17)
    xd, wd = x.to(device), w.to(device)
    cfg = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2}
    first = fast_gemm.packed_weight(wd)
    assert fast_gemm.packed_weight(wd) is first
    check(hip_linear(xd, wd, cfg), x, w)
    w2 = (0.02 * torch.randn(N, K)).bfloat16()
    wd.copy_(w2.to(device))
    assert fast_gemm.packed_weight(wd) is not first
    check(hip_linear(xd, wd, cfg), x, w2)


def test_wide_workgroup_count_stays_in_bounds(device):
    # Many items (N = 50304 at 64-row tiles, split 8: 6288 items, 24 per workgroup): every
    # workgroup index maps to a real tile and split slot.
    M, N, K = 42, 50304, 1024
    x, w = _inputs_on_gpu(M, N, K, 15, device)
    cfg = {"wave_frags": 1, "k_waves": 4, "split_k": 8, "unroll": 2}
    assert tiles.items(N, cfg) > 16 * tiles.CU_COUNT
    cols = torch.cat([torch.arange(0, 64), torch.arange(N - 64, N)])
    check_cols(hip_linear(x, w, cfg), x, w, cols)


@pytest.mark.parametrize("name", golden_names("gemm_"))
def test_golden_fixtures(device, name):
    """The committed fp64 fixtures, through the tile table's kind of tile (heuristic) and a split-K
    tile: within one rounding of the exact product (bit-exact for the small-integer case)."""
    z = load_golden(name)
    x, w = z["x"], z["w"]
    M, K = x.shape
    N = w.shape[0]
    supported = lambda c: fast_gemm.tile_supported(M, K, c)  # noqa: E731
    for cfg in (tiles.heuristic_tile(M, N, K, supported=supported),
                {"wave_frags": 1, "k_waves": 4, "split_k": 2, "unroll": 2}):
        y = _run(x, w, cfg, device).cpu()
        got = y.view(torch.int16).numpy().view("uint16")
        if name.endswith("_int"):
            assert (got == z["y_bf16"]).all(), cfg
        else:
            _within_one_rounding(y.float(), x, w)
            steps = abs(got.astype("int32") - z["y_bf16"].astype("int32"))
            assert steps.max() <= 1 and (steps > 0).mean() <= 2e-3, (cfg, int((steps > 0).sum()))
