"""GPU parity of packed chains with SiLU-and-multiply links (``Link(act=True)``, ``out_f32 =
PLM_OUT_SILU_MUL``): the Llama-style MLP's real dataflow, gate/up projection with its activation,
then down reading the activation's ``[M, I]`` output, inside one persistent launch.

Every link's output must equal its single-launch equivalent bit for bit (``gate_up_silu`` for an
act link, ``hip_linear`` otherwise, same tile and split): the chain runs the same kernel over the
same K partition. The tile-flag mode (each linear reads the one before it) is checked with inputs
rewritten and every output filled with NaN before each of several launches and graph replays, so a
consumer that read a producer's tile before it was written would show; the error flag stays clear."""

from __future__ import annotations

import pytest
import torch

import oracle
from plm_amd import _lib
from plm_amd.chain import Link, LinearChain
from plm_amd.fast_gemm import gate_up_silu, hip_linear
from plm_amd.tiles import packed_chain_split, packed_chain_tile

pytestmark = pytest.mark.gpu


def _w(n, k, gen, device, dtype=torch.bfloat16):
    return (0.03 * torch.randn(n, k, generator=gen, device=device)).to(dtype)


def _llama_links(x, layers, hidden, qkv, inter, gen, cfg, G, act=True):
    """Links of `layers` Llama-style blocks, each reading the one before it: qkv, o (the first
    `hidden` columns of qkv's output), gate_up (+ act), down (the activation's output)."""
    device, dtype, M = x.device, x.dtype, x.shape[0]
    links = []
    prev = x
    for _ in range(layers):
        for n, k, is_act in ((qkv, hidden, False), (hidden, hidden, False), (2 * inter, hidden, act),
                             (hidden, inter if act else 2 * inter, False)):
            w = _w(n, k, gen, device, dtype)
            y = torch.empty(M, n // 2 if is_act else n, device=device, dtype=dtype)
            links.append(Link(prev[:, :k], w, y, len(links) - 1, packed_chain_split(n, k, cfg, G), is_act))
            prev = y
    links[0].dep = -1
    return links


def _single(ln, cfg):
    c = dict(cfg, split_k=ln.split_k)
    return gate_up_silu(ln.x, ln.w, c) if ln.act else hip_linear(ln.x, ln.w, c)


def _grid(M, cfg):
    G = _lib.lib().plm_gemm_packed_resident_workgroups(_lib.PLM_BF16, M, _lib.Tile.from_config(cfg))
    assert G > 0
    return G


@pytest.mark.parametrize("M", [56, 7, 42])
def test_mlp_chain_matches_single_launches(device, M):
    gen = torch.Generator(device=device).manual_seed(100 + M)
    cfg = packed_chain_tile(M)
    G = _grid(M, cfg)
    x = torch.randn(M, 2048, generator=gen, device=device).bfloat16()
    w_gu, w_d = _w(11264, 2048, gen, device), _w(2048, 5632, gen, device)
    act = torch.empty(M, 5632, device=device, dtype=torch.bfloat16)
    out = torch.empty(M, 2048, device=device, dtype=torch.bfloat16)
    links = [Link(x, w_gu, act, -1, packed_chain_split(11264, 2048, cfg, G), True),
             Link(act, w_d, out, 0, packed_chain_split(2048, 5632, cfg, G))]
    chain = LinearChain(links, cfg)
    assert chain.sync_mode == 2
    chain.run()
    chain.check()
    want_act = _single(links[0], cfg)
    assert torch.equal(act, want_act)
    assert torch.equal(out, hip_linear(want_act, w_d, dict(cfg, split_k=links[1].split_k)))
    # The activation against the oracle: the projection on the CPU, then silu(g) * u.
    cols = torch.randperm(5632, generator=torch.Generator().manual_seed(M))[:128]
    rows = torch.cat([cols, cols + 5632]).to(device)
    ref = oracle.silu_mul(oracle.linear(x.cpu(), w_gu[rows].cpu())).float()
    sub = act[:, cols.to(device)].cpu().float()
    assert bool(((sub - ref).abs() <= 2e-2 + 1e-3 * ref.abs()).all())


def test_llama_blocks_chain_with_rewritten_inputs(device):
    """Three Llama-style 1.3B blocks (qkv 3072, o, gate_up 11264 with its activation, down from 5632)
    in one tile-flag launch: 6 launches and 3 graph replays, each after rewriting x and filling
    every output with NaN; each launch's outputs equal the single launches on that launch's x."""
    M = 56
    gen = torch.Generator(device=device).manual_seed(7)
    cfg = packed_chain_tile(M)
    G = _grid(M, cfg)
    x = torch.empty(M, 2048, device=device, dtype=torch.bfloat16)
    links = _llama_links(x, 3, 2048, 3072, 5632, gen, cfg, G)
    chain = LinearChain(links, cfg)
    assert chain.sync_mode == 2

    def fresh(seed):
        x.copy_(torch.randn(M, 2048, generator=torch.Generator(device=device).manual_seed(seed), device=device))
        for ln in links:
            ln.y.fill_(float("nan"))

    def check():
        chain.check()
        xi = x
        for i, ln in enumerate(links):
            want = _single(Link(xi[:, :ln.w.shape[1]], ln.w, ln.y, -1, ln.split_k, ln.act), cfg)
            assert torch.equal(ln.y, want), f"link {i} (act={ln.act}) differs from its single launch"
            xi = want

    for r in range(6):
        fresh(1000 + r)
        chain.run()
        check()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    fresh(2000)
    with torch.cuda.graph(graph, stream=stream):
        chain.run()
    for r in range(3):
        fresh(3000 + r)
        graph.replay()
        torch.cuda.synchronize()
        check()


def test_grid_barrier_mode_and_fp16(device):
    """An act link read by a later link that is not its successor (grid barriers), fp16."""
    M = 42
    gen = torch.Generator(device=device).manual_seed(9)
    cfg = packed_chain_tile(M)
    x = torch.randn(M, 1024, generator=gen, device=device).half()
    w_gu, w_o, w_d = _w(4096, 1024, gen, device, torch.float16), _w(1024, 1024, gen, device, torch.float16), \
        _w(1024, 2048, gen, device, torch.float16)
    act = torch.empty(M, 2048, device=device, dtype=torch.float16)
    side = torch.empty(M, 1024, device=device, dtype=torch.float16)
    out = torch.empty(M, 1024, device=device, dtype=torch.float16)
    links = [Link(x, w_gu, act, -1, 2, True), Link(x, w_o, side, -1, 1), Link(act, w_d, out, 0, 2)]
    chain = LinearChain(links, cfg)
    assert chain.sync_mode == 1
    for r in range(3):
        for ln in links:
            ln.y.fill_(float("nan"))
        chain.run()
        chain.check()
        want_act = _single(links[0], cfg)
        assert torch.equal(act, want_act)
        assert torch.equal(side, _single(links[1], cfg))
        assert torch.equal(out, hip_linear(want_act, w_d, dict(cfg, split_k=2)))


def test_act_link_checks(device):
    """An act link needs a packed chain, an even wave_frags, N a multiple of 32 and y [M, N/2]."""
    M = 8
    x = torch.randn(M, 256, device=device).bfloat16()
    w = _w(512, 256, torch.Generator(device=device).manual_seed(1), device)
    with pytest.raises(ValueError):
        LinearChain([Link(x, w, torch.empty(M, 512, device=device).bfloat16(), act=True)], packed_chain_tile(M))
    with pytest.raises(ValueError):
        LinearChain([Link(x, w, torch.empty(M, 256, device=device).bfloat16(), act=True)], packed_chain_tile(M),
                    packed=False)
    odd = dict(packed_chain_tile(M), wave_frags=1)
    chain = LinearChain([Link(x, w, torch.empty(M, 256, device=device).bfloat16(), act=True)], odd)
    with pytest.raises(RuntimeError):
        chain.run()
