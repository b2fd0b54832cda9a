"""GPU parity of the chained launches: linears back to back in one persistent grid, over packed
weights (plm_gemm_chain_packed: tile-done flags when every linear reads the one before it, else
grid barriers of per-workgroup progress flags) and over row-major weights (plm_gemm_chain: each
consumer tile starts once the producer tiles it reads are written).

Checks: every link's output equals the single-linear kernel's on the same operands bit for bit
(same kernel, same K partition), and the CPU oracle's within the GEMM tolerance; repeated launches
and HIP-graph replays give identical results (flags are per launch); the error flag stays clear."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from plm_amd import workloads
from plm_amd.chain import Link, LinearChain
from plm_amd.fast_gemm import hip_linear, hip_linear_rowmajor
from plm_amd.tiles import chain_tile

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-2
CFG = chain_tile(56)


def _weights(shapes, seed, device, dtype=torch.bfloat16):
    g = torch.Generator(device=device).manual_seed(seed)
    return [(0.02 * torch.randn(n, k, generator=g, device=device)).to(dtype) for n, k in shapes]


def _chain(x, ws, splits, deps=None, ys=None):
    """Links y_i = x_i @ w_i.T with x_0 = x and x_i = y_{i-1}[:, :K_i] (or an external input)."""
    links = []
    ys = ys or [torch.empty(x.shape[0], w.shape[0], device=x.device, dtype=x.dtype) for w in ws]
    for i, (w, y, s) in enumerate(zip(ws, ys, splits)):
        dep = (i - 1) if (deps is None and i > 0) else (deps[i] if deps is not None else -1)
        xi = x if dep < 0 else ys[dep][:, : w.shape[1]]
        links.append(Link(xi, w, y, dep, s))
    return links, ys


def _check_against_single(links, cfg=CFG, packed=True):
    """Bit for bit the single-linear kernel; against the oracle within 1e-3 rel / 2e-2 abs, or one
    output rounding step where the oracle's own fp32 sum lands on the other side of a rounding
    midpoint (at |y| >= 4 one bf16 step exceeds 2e-2), for at most 0.1 % of a link's elements."""
    for i, ln in enumerate(links):
        linear = hip_linear if packed else hip_linear_rowmajor
        single = linear(ln.x, ln.w, dict(cfg, split_k=ln.split_k))
        assert torch.equal(ln.y, single), f"link {i} differs from the single-linear kernel"
        got = ln.y.cpu().float()
        ref = oracle.linear(ln.x.cpu(), ln.w.cpu()).float()
        diff = (got - ref).abs()
        in_tol = diff <= ATOL + RTOL * ref.abs()
        bits = 8 if ln.y.dtype == torch.bfloat16 else 11
        step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - (bits - 1))
        assert bool((in_tol | (diff <= step * 1.0001)).all()), f"link {i}: max |got - oracle| {diff.max():.4g}"
        assert int((~in_tol).sum()) <= max(1, got.numel() // 1000), (i, int((~in_tol).sum()))


@pytest.mark.parametrize("packed", [True, False], ids=["packed", "rowmajor"])
@pytest.mark.parametrize("splits", [(1, 1, 1), (2, 4, 1), (3, 1, 8)])
def test_three_links(device, splits, packed):
    M = 56
    g = torch.Generator(device=device).manual_seed(20)
    x = torch.randn(M, 512, generator=g, device=device).bfloat16()
    ws = _weights([(1024, 512), (512, 1024), (2000, 512)], 21, device)
    links, _ = _chain(x, ws, splits)
    chain = LinearChain(links, CFG, packed=packed)
    chain.run()
    _check_against_single(links, packed=packed)
    assert chain.error_flag() == 0


@pytest.mark.parametrize("cfg", [{"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2},
                                 {"wave_frags": 4, "k_waves": 4, "split_k": 1, "unroll": 8},
                                 {"wave_frags": 1, "k_waves": 4, "split_k": 1, "unroll": 4},
                                 {"wave_frags": 2, "k_waves": 1, "split_k": 1, "unroll": 2},
                                 {"wave_frags": 1, "k_waves": 1, "split_k": 1, "unroll": 8},
                                 {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2},
                                 {"wave_frags": 1, "k_waves": 16, "split_k": 1, "unroll": 2}],
                         ids=lambda c: f"nf{c['wave_frags']}d{c['unroll']}kw{c['k_waves']}")
def test_packed_chain_tiles(device, cfg):
    # Deep and shallow pipelines, and widths whose K is not a multiple of 32 in the middle link.
    M = 42
    g = torch.Generator(device=device).manual_seed(30)
    x = torch.randn(M, 1024, generator=g, device=device).bfloat16()
    ws = _weights([(1416, 1024), (2048, 1416), (3000, 2048)], 31, device)
    links, _ = _chain(x, ws, (2, 3, 1))
    chain = LinearChain(links, cfg, packed=True)
    chain.run()
    _check_against_single(links, cfg)
    assert chain.error_flag() == 0


def _padded_outputs(M, ws, device, dtype=torch.bfloat16):
    """Outputs whose rows start 128 bytes apart (ldy a multiple of 64 elements): views of wider
    buffers where N is not a multiple of 64, so a chain reading them keeps its tile-flag mode."""
    return [torch.empty(M, -(-w.shape[0] // 64) * 64, device=device, dtype=dtype)[:, : w.shape[0]] for w in ws]


def test_tile_flag_chain_long_and_wide_links(device):
    """The tile-flag chain with the round's tile: items of 2 to 32 K steps per wavefront, several
    items per workgroup (625 and 1250 tiles), a K that ends inside a step, a split link."""
    M = 56
    cfg = {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2}
    g = torch.Generator(device=device).manual_seed(40)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    ws = _weights([(8192, 2048), (2048, 8192), (20000, 2048), (1000, 20000), (40000, 1000)], 41, device)
    links, _ = _chain(x, ws, (1, 1, 1, 2, 1), ys=_padded_outputs(M, ws, device))
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 2
    for _ in range(2):
        x.copy_(torch.randn(M, 2048, generator=g, device=device).bfloat16())
        chain.run()
        _check_against_single(links, cfg)
    assert chain.error_flag() == 0


def test_unaligned_consumed_output_takes_grid_barriers(device):
    """A consumed Y whose rows are not 128 bytes apart (N = 1000) would let a 128-byte line span the
    tail of one row and the head of the next, outside the tile-flag wait's widening: the launch uses
    grid barriers instead, and stays exact with new inputs on every launch."""
    M = 56
    cfg = {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2}
    g = torch.Generator(device=device).manual_seed(42)
    x = torch.randn(M, 1024, generator=g, device=device).bfloat16()
    ws = _weights([(1000, 1024), (3000, 1000), (1000, 3000)], 43, device)
    links, ys = _chain(x, ws, (1, 2, 1))
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 1
    for _ in range(3):
        x.copy_(torch.randn(M, 1024, generator=g, device=device).bfloat16())
        for y in ys:
            y.fill_(float("nan"))
        chain.run()
        _check_against_single(links, cfg)
    chain.check()


def test_repeated_launches_and_external_input(device):
    M = 42
    g = torch.Generator(device=device).manual_seed(22)
    x = torch.randn(M, 1024, generator=g, device=device).bfloat16()
    x_ext = torch.randn(M, 768, generator=g, device=device).bfloat16()
    ws = _weights([(2048, 1024), (1024, 2048), (640, 768), (1536, 640)], 23, device)
    ys = [torch.empty(M, w.shape[0], device=device, dtype=torch.bfloat16) for w in ws]
    links = [Link(x, ws[0], ys[0], -1, 2), Link(ys[0][:, :2048], ws[1], ys[1], 0, 4),
             Link(x_ext, ws[2], ys[2], -1, 1), Link(ys[2], ws[3], ys[3], 2, 2)]
    chain = LinearChain(links, CFG)
    chain.run()
    first = [y.clone() for y in ys]
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        chain.run()
        for y, f in zip(ys, first):
            assert torch.equal(y, f), rep
    # New inputs in place between launches: every output changes, so a consumer that read a line
    # left over from an earlier launch would show up here.
    for rep in range(3):
        x.copy_(torch.randn(M, 1024, generator=g, device=device).bfloat16())
        x_ext.copy_(torch.randn(M, 768, generator=g, device=device).bfloat16())
        chain.run()
        _check_against_single(links)
    assert chain.error_flag() == 0


def test_block_chain_1p3b(device):
    # Two GPT-style 1.3B-shape blocks back to back at M = 56, as the round benchmark runs them.
    M = 56
    shapes = [(g.N, g.K) for g in workloads.gpt_block(2048, 8192)] * 2
    ws = _weights(shapes, 24, device)
    g = torch.Generator(device=device).manual_seed(25)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    links, _ = _chain(x, ws, [2, 8, 2, 8, 2, 8, 2, 8])
    chain = LinearChain(links, CFG)
    chain.run()
    _check_against_single(links)
    assert chain.error_flag() == 0


def test_graph_replay(device):
    M = 56
    g = torch.Generator(device=device).manual_seed(26)
    x = torch.randn(M, 1024, generator=g, device=device).bfloat16()
    ws = _weights([(3072, 1024), (1024, 2048), (4000, 1024)], 27, device)
    links, ys = _chain(x, ws, [2, 4, 1])
    chain = LinearChain(links, CFG)
    chain.run()
    eager = [y.clone() for y in ys]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chain.run()
    for rep in range(4):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert torch.equal(y, e), rep
        chain.run()                                   # eager work between replays
        torch.cuda.synchronize()
    assert chain.error_flag() == 0


def test_fp32_last_link_and_fp16(device):
    M = 28
    g = torch.Generator(device=device).manual_seed(28)
    x = torch.randn(M, 512, generator=g, device=device).half()
    ws = _weights([(1024, 512), (3000, 1024)], 29, device, torch.float16)
    y0 = torch.empty(M, 1024, device=device, dtype=torch.float16)
    y1 = torch.empty(M, 3000, device=device, dtype=torch.float32)
    links = [Link(x, ws[0], y0, -1, 2), Link(y0, ws[1], y1, 0, 1)]
    chain = LinearChain(links, CFG)
    chain.run()
    torch.testing.assert_close(y1.cpu(), oracle.linear_fp32(y0.cpu(), ws[1].cpu()), rtol=1e-4, atol=1e-4)
    assert chain.error_flag() == 0


def _oracle_columns(x, w, y, cols):
    """``y[:, cols]`` against the CPU oracle on those weight rows: within 1e-3 rel / 2e-2 abs, or one
    output rounding step (at most 0.1 % of the sampled elements)."""
    got = y[:, cols].cpu().float()
    ref = oracle.linear(x.cpu(), w[cols].cpu()).float()
    diff = (got - ref).abs()
    in_tol = diff <= ATOL + RTOL * ref.abs()
    bits = 8 if y.dtype == torch.bfloat16 else 11
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - (bits - 1))
    assert bool((in_tol | (diff <= step * 1.0001)).all()), f"max |got - oracle| {diff.max():.4g}"
    assert int((~in_tol).sum()) <= max(1, got.numel() // 1000)


def _chain_table_entries():
    from plm_amd import gemm_tables

    return [(int(p.stem.removeprefix("chain_tiles_hidden")), M)
            for p in sorted(gemm_tables.TABLES.glob("chain_tiles_hidden*.json"))
            for M in sorted(gemm_tables.read_chain_table(int(p.stem.removeprefix("chain_tiles_hidden"))))]


@pytest.mark.parametrize("hidden,M", _chain_table_entries(), ids=lambda v: str(v))
def test_round_chain_table_tiles(device, hidden, M):
    """Every measured chain tile (chain_tiles_hidden<H>.json) on one block of the round it was
    measured on, at its width, each linear reading the one before it (the tile-flag launch), launched twice
    with a new input and NaN-filled outputs: bit for bit the single-linear kernel, and the oracle
    within the GEMM tolerance."""
    from plm_amd import _lib, gemm_tables
    from plm_amd.fast_gemm import _tile
    from plm_amd.tiles import packed_chain_split

    cfg = gemm_tables.round_chain_tile(hidden, M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _tile(cfg))
    assert G > 0
    from plm_amd.tune import chain_rounds

    shapes = [(gm.N, gm.K) for gm in chain_rounds()[hidden][0]]
    ws = _weights(shapes, 70 + M, device)
    g = torch.Generator(device=device).manual_seed(71 + hidden)
    x = torch.randn(M, hidden, generator=g, device=device).bfloat16()
    links, ys = _chain(x, ws, [packed_chain_split(n, k, cfg, G) for n, k in shapes])
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 2
    for _ in range(2):
        x.copy_(torch.randn(M, hidden, generator=g, device=device).bfloat16())
        for y in ys:
            y.fill_(float("nan"))
        chain.run()
        _check_against_single(links, cfg)
    assert chain.error_flag() == 0


def test_round_chain_graph_replays_with_new_inputs(device):
    """The benchmark's chained round, all 96 block linears of the 1.3B-shape round at M = 56 in one
    tile-flag launch, recorded as a HIP graph and replayed 8 times. Before every replay the round's
    input is rewritten and every output filled with NaN, so a consumer that read a line before its
    producer tiles were written (or a line left from an earlier replay) would show up: each replay
    must equal per-linear launches bit for bit, and sampled columns of the first and last block
    must match the CPU oracle."""
    from plm_amd import _lib, gemm_tables
    from plm_amd.fast_gemm import _tile
    from plm_amd.tiles import packed_chain_split

    M = 56
    cfg = gemm_tables.round_chain_tile(2048, M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _tile(cfg))
    assert G > 0
    block = workloads.gpt_block(2048, 8192)
    shapes = [(gm.N, gm.K) for gm in block] * 24
    ws = _weights(shapes, 60, device)
    g = torch.Generator(device=device).manual_seed(61)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    splits = [packed_chain_split(n, k, cfg, G) for n, k in shapes]
    links, ys = _chain(x, ws, splits)
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 2
    chain.run()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chain.run()
    refs = [torch.empty_like(y) for y in ys]
    sample = torch.randperm(2048, generator=torch.Generator().manual_seed(62))[:96]
    for rep in range(8):
        x.copy_(torch.randn(M, 2048, generator=g, device=device).bfloat16())
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for ln, ref in zip(links, refs):
            hip_linear(ln.x, ln.w, dict(cfg, split_k=ln.split_k), ref)
        torch.cuda.synchronize()
        bad = [i for i, (y, r) in enumerate(zip(ys, refs)) if not torch.equal(y, r)]
        assert not bad, f"replay {rep}: links {bad[:8]} differ from per-linear launches"
        if rep in (0, 7):
            for i in (0, 1, 2, 3, 92, 93, 94, 95):
                cols = sample[sample < ws[i].shape[0]]
                _oracle_columns(links[i].x, ws[i], ys[i], cols)
    chain.check()


def test_config4_round_chain_all_columns(device):
    """Config 4's round: all 128 block linears of the 32-block hidden-2560 round (QKV 2560 -> 7680,
    attn-out, MLP up 2560 -> 10240, down) at M = 56 in one tile-flag launch, with the round's chain
    tile and splits, launched twice with a new input and NaN-filled outputs. Every link equals its
    per-linear launch bit for bit, and the first and last blocks' four linears match the CPU oracle
    on every column."""
    from plm_amd import _lib, gemm_tables
    from plm_amd.fast_gemm import _tile
    from plm_amd.tiles import packed_chain_split

    M, hidden = 56, 2560
    cfg = gemm_tables.round_chain_tile(hidden, M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _tile(cfg))
    assert G > 0
    shapes = [(gm.N, gm.K) for gm in workloads.gpt_block(hidden, 4 * hidden)] * 32
    # Weights ~ N(0, 1/K), so that activations keep their scale over the 128 links (with a fixed
    # 0.02 they grow about 2x per block, to ~1e10: outputs with heavy cancellation then carry fp32
    # accumulation error beyond one bf16 step, on the oracle's side of the comparison as much as
    # on the kernel's).
    gw = torch.Generator(device=device).manual_seed(90)
    ws = [(torch.randn(n, k, generator=gw, device=device) / math.sqrt(k)).bfloat16() for n, k in shapes]
    g = torch.Generator(device=device).manual_seed(91)
    x = torch.randn(M, hidden, generator=g, device=device).bfloat16()
    links, ys = _chain(x, ws, [packed_chain_split(n, k, cfg, G) for n, k in shapes])
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 2
    refs = [torch.empty_like(y) for y in ys]
    for rep in range(2):
        x.copy_(torch.randn(M, hidden, generator=g, device=device).bfloat16())
        for y in ys:
            y.fill_(float("nan"))
        chain.run()
        for ln, ref in zip(links, refs):
            hip_linear(ln.x, ln.w, dict(cfg, split_k=ln.split_k), ref)
        torch.cuda.synchronize()
        bad = [i for i, (y, r) in enumerate(zip(ys, refs)) if not torch.equal(y, r)]
        assert not bad, f"launch {rep}: links {bad[:8]} differ from per-linear launches"
    for i in (0, 1, 2, 3, 124, 125, 126, 127):
        _oracle_columns(links[i].x, ws[i], ys[i], torch.arange(ws[i].shape[0]))
    chain.check()


def test_fp16_round_chain(device):
    """The 1.3B round in fp16, the reference's default round dtype (plm/rounds.py:50): all 96 block
    linears (24 GPT-style blocks, hidden 2048) at M = 56 in one tile-flag launch with the round's
    chain tile and splits, launched twice with a new input and NaN-filled outputs. Every link equals
    its per-linear launch bit for bit, and the first and last blocks' four linears match the CPU
    oracle on every column."""
    from plm_amd import _lib, gemm_tables
    from plm_amd.fast_gemm import _tile
    from plm_amd.tiles import packed_chain_split

    M, hidden = 56, 2048
    cfg = gemm_tables.round_chain_tile(hidden, M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.DTYPE_CODES[torch.float16], M, _tile(cfg))
    assert G > 0
    shapes = [(gm.N, gm.K) for gm in workloads.gpt_block(hidden, 4 * hidden)] * 24
    gw = torch.Generator(device=device).manual_seed(95)
    ws = [(torch.randn(n, k, generator=gw, device=device) / math.sqrt(k)).half() for n, k in shapes]
    g = torch.Generator(device=device).manual_seed(96)
    x = torch.randn(M, hidden, generator=g, device=device).half()
    links, ys = _chain(x, ws, [packed_chain_split(n, k, cfg, G) for n, k in shapes])
    chain = LinearChain(links, cfg, packed=True)
    assert chain.sync_mode == 2
    refs = [torch.empty_like(y) for y in ys]
    for rep in range(2):
        x.copy_(torch.randn(M, hidden, generator=g, device=device).half())
        for y in ys:
            y.fill_(float("nan"))
        chain.run()
        for ln, ref in zip(links, refs):
            hip_linear(ln.x, ln.w, dict(cfg, split_k=ln.split_k), ref)
        torch.cuda.synchronize()
        bad = [i for i, (y, r) in enumerate(zip(ys, refs)) if not torch.equal(y, r)]
        assert not bad, f"launch {rep}: links {bad[:8]} differ from per-linear launches"
    for i in (0, 1, 2, 3, 92, 93, 94, 95):
        _oracle_columns(links[i].x, ws[i], ys[i], torch.arange(ws[i].shape[0]))
    chain.check()


def test_wide_round_packed_chain_two_blocks(device):
    """Two 1.3B-shape blocks chained over packed weights at the relaxed setting's width M = 110
    (k = 10, seven 16-row fragments), with the tile and splits the benchmark's W = 110 round uses:
    bit for bit the per-linear launches, and the oracle."""
    from plm_amd import _lib
    from plm_amd.fast_gemm import _tile
    from plm_amd.tiles import packed_chain_split, packed_chain_tile

    M = 110
    cfg = packed_chain_tile(M)
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _tile(cfg))
    assert G > 0
    shapes = [(gm.N, gm.K) for gm in workloads.gpt_block(2048, 8192)] * 2
    ws = _weights(shapes, 70, device)
    g = torch.Generator(device=device).manual_seed(71)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    links, _ = _chain(x, ws, [packed_chain_split(n, k, cfg, G) for n, k in shapes])
    chain = LinearChain(links, cfg, packed=True)
    chain.run()
    _check_against_single(links, cfg)
    chain.check()
