"""GPU parity of the ring chain (plm_ring_chain): the round's linears in one launch with the packed
weights streamed into LDS by a wavefront of their own, each linear handing its output to the next
through an operand-layout copy.

Checks: a one-link chain is within the GEMM tolerance of the CPU oracle (torch F.linear, the
reference's default path, plm/fast_gemm.py:111) over round widths, ragged N and K, every tile
height and K splits; every link of a longer chain equals the one-link chain of the same geometry on
the same operands bit for bit (the result depends only on the link's own tile); repeated launches
and HIP-graph replays with new inputs give the fresh results (tile flags carry the launch epoch);
the error flag stays clear."""

from __future__ import annotations

import pytest
import torch

import oracle
from plm_amd.chain import Link
from plm_amd.ring import Geometry, RingChain

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-2


def _weights(shapes, seed, device, dtype=torch.bfloat16):
    g = torch.Generator(device=device).manual_seed(seed)
    return [(0.02 * torch.randn(n, k, generator=g, device=device)).to(dtype) for n, k in shapes]


def _links(x, ws, deps=None, ys=None):
    """y_i = x_i @ w_i.T with x_0 = x and x_i = y_{deps[i]}[:, :K_i] (default deps[i] = i - 1)."""
    ys = ys or [torch.empty(x.shape[0], w.shape[0], device=x.device, dtype=x.dtype) for w in ws]
    links = []
    for i, (w, y) in enumerate(zip(ws, ys)):
        dep = (i - 1) if deps is None else deps[i]
        links.append(Link(x if dep < 0 else ys[dep][:, : w.shape[1]], w, y, dep))
    return links


def _check_oracle(y, x, w, what):
    """Within 1e-3 rel / 2e-2 abs of the oracle, or one output rounding step where the oracle's own
    fp32 sum lands on the other side of a rounding midpoint, for at most 0.1 % of the elements."""
    got = y.cpu().float()
    ref = oracle.linear(x.cpu(), w.cpu()).float() if y.dtype != torch.float32 else oracle.linear_fp32(x.cpu(), w.cpu())
    diff = (got - ref).abs()
    in_tol = diff <= ATOL + RTOL * ref.abs()
    bits = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}[y.dtype]
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - (bits - 1))
    assert bool((in_tol | (diff <= step * 1.0001)).all()), f"{what}: max |got - oracle| {diff.max():.4g}"
    assert int((~in_tol).sum()) <= max(1, got.numel() // 1000), (what, int((~in_tol).sum()))


def _single(ln, geo, out_dtype=None):
    """The link alone: a one-link chain with the same geometry on the same X (read row-major)."""
    y = torch.empty_like(ln.y) if out_dtype is None else torch.empty(ln.y.shape, device=ln.y.device, dtype=out_dtype)
    RingChain([Link(ln.x, ln.w, y, -1)], {0: geo}).run()
    return y


def _check_links(chain):
    for i, (ln, geo) in enumerate(zip(chain.links, chain.geometry)):
        assert torch.equal(ln.y, _single(ln, geo)), f"link {i} ({geo}) differs from its one-link chain"
        _check_oracle(ln.y, ln.x, ln.w, f"link {i}")


SINGLE = [
    # M, N, K, tile_rows, split
    (56, 2048, 2048, 4, 8),
    (56, 6144, 2048, 3, 2),
    (56, 8192, 2048, 4, 2),
    (56, 2048, 8192, 4, 8),
    (42, 4096, 1024, 4, 1),
    (1, 1000, 520, 2, 1),
    (17, 200, 72, 1, 3),
    (64, 1040, 960, 3, 5),
    (7, 48, 32, 4, 1),
    (33, 4096, 4096, 4, 4),
    (49, 3000, 1000, 2, 16),
]


@pytest.mark.parametrize("M,N,K,tr,split", SINGLE, ids=lambda v: str(v))
def test_single_link_matches_the_oracle(device, M, N, K, tr, split):
    g = torch.Generator(device=device).manual_seed(M * 131 + N + K)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    (w,) = _weights([(N, K)], M + N, device)
    y = torch.full((M, N), float("nan"), device=device, dtype=torch.bfloat16)
    chain = RingChain([Link(x, w, y, -1)], {0: Geometry(tr, split)})
    chain.run()
    _check_oracle(y, x, w, f"M={M} N={N} K={K}")
    y32 = torch.empty(M, N, device=device, dtype=torch.float32)
    RingChain([Link(x, w, y32, -1)], {0: Geometry(tr, split)}).run()
    _check_oracle(y32, x, w, "fp32 out")
    assert torch.equal(y, y32.to(torch.bfloat16)), "the model-dtype output is the rounded fp32 accumulator"
    assert chain.error_flag() == 0


@pytest.mark.parametrize("M", [7, 56])
def test_blocks_equal_their_links_alone(device, M):
    hidden, mlp = 1024, 4096
    g = torch.Generator(device=device).manual_seed(50 + M)
    x = torch.randn(M, hidden, generator=g, device=device).bfloat16()
    shapes = [(3 * hidden, hidden), (hidden, hidden), (mlp, hidden), (hidden, mlp)] * 2
    chain = RingChain(_links(x, _weights(shapes, 51, device)))
    chain.run()
    _check_links(chain)
    assert chain.error_flag() == 0


def test_other_producers_external_inputs_and_geometries(device):
    """Links reading an earlier link other than the one before, a link with its own external X in
    the middle, a narrow producer (tile_rows 1) read by a split consumer, and an fp32 last link."""
    M = 40
    g = torch.Generator(device=device).manual_seed(60)
    x = torch.randn(M, 512, generator=g, device=device).bfloat16()
    x2 = torch.randn(M, 768, generator=g, device=device).bfloat16()
    ws = _weights([(1024, 512), (512, 1024), (640, 1024), (768, 640), (1536, 768), (520, 1536)], 61, device)
    deps = [-1, 0, 0, 2, -1, 4]
    ys = [torch.empty(M, w.shape[0], device=device, dtype=torch.bfloat16) for w in ws[:-1]]
    ys.append(torch.empty(M, ws[-1].shape[0], device=device, dtype=torch.float32))
    links = _links(x, ws, deps, ys)
    links[4] = Link(x2, ws[4], ys[4], -1)
    geo = {0: Geometry(1, 1), 1: Geometry(2, 4), 2: Geometry(3, 1), 3: Geometry(4, 2), 5: Geometry(2, 3)}
    chain = RingChain(links, geo)
    chain.run()
    for i, (ln, gm) in enumerate(zip(chain.links, chain.geometry)):
        assert torch.equal(ln.y, _single(ln, gm, ln.y.dtype)), f"link {i} differs from its one-link chain"
        _check_oracle(ln.y, ln.x, ln.w, f"link {i}")
    assert chain.error_flag() == 0


def test_relaunch_and_graph_replay_with_new_inputs(device):
    """Flags carry the launch epoch: every launch and graph replay reads this launch's outputs."""
    M = 56
    g = torch.Generator(device=device).manual_seed(70)
    x = torch.randn(M, 1024, generator=g, device=device).bfloat16()
    ws = _weights([(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)], 71, device)
    chain = RingChain(_links(x, ws))
    for _ in range(3):
        x.copy_(torch.randn(M, 1024, generator=g, device=device).bfloat16())
        chain.run()
        _check_links(chain)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=stream):
        chain.run()
    for _ in range(3):
        x.copy_(torch.randn(M, 1024, generator=g, device=device).bfloat16())
        for ln in chain.links:
            ln.y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        _check_links(chain)
    assert chain.error_flag() == 0


def test_runs_are_bitwise_reproducible(device):
    M = 56
    g = torch.Generator(device=device).manual_seed(80)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    ws = _weights([(2048, 2048), (8192, 2048), (2048, 8192)], 81, device)
    chain = RingChain(_links(x, ws))
    chain.run()
    first = [ln.y.clone() for ln in chain.links]
    for _ in range(3):
        chain.run()
        assert all(torch.equal(a, ln.y) for a, ln in zip(first, chain.links))
    assert chain.error_flag() == 0


def test_fp16(device):
    M = 42
    g = torch.Generator(device=device).manual_seed(90)
    x = torch.randn(M, 1024, generator=g, device=device).half()
    ws = _weights([(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)], 91, device, torch.float16)
    chain = RingChain(_links(x, ws))
    chain.run()
    _check_links(chain)
    assert chain.error_flag() == 0


@pytest.mark.parametrize("M", [56, 7])
def test_round_1p3b(device, M):
    """The 1.3B-shape round's 96 block linears (24 GPT-style blocks, hidden 2048, MLP 8192) as one
    ring chain: every link bit for bit its one-link chain, and within tolerance of the oracle."""
    from plm_amd import workloads

    g = torch.Generator(device=device).manual_seed(100 + M)
    x = torch.randn(M, 2048, generator=g, device=device).bfloat16()
    shapes = [(gm.N, gm.K) for gm in workloads.gpt_block(2048, 8192)] * 24
    chain = RingChain(_links(x, _weights(shapes, 101, device)))
    chain.run()
    for i, (ln, geo) in enumerate(zip(chain.links, chain.geometry)):
        assert torch.equal(ln.y, _single(ln, geo)), f"link {i} ({geo}) differs from its one-link chain"
    for i in (0, 1, 2, 3, 94, 95):
        _check_oracle(chain.links[i].y, chain.links[i].x, chain.links[i].w, f"link {i}")
    assert chain.error_flag() == 0
