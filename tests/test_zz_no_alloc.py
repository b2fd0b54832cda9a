"""The allocation-free entry point (plm_gemm_packed_noalloc) called through the C ABI: bit for bit
what plm_gemm_packed returns with a workspace, on consecutive calls that share the library's device
scratch (the second with a smaller input, so it runs over what the first left behind), with and
without split-K; sizes past the scratch are rejected before any launch."""

from __future__ import annotations

import pytest
import torch

from plm_amd import _lib
from plm_amd.fast_gemm import launch_packed, pack_weight

pytestmark = pytest.mark.gpu


def _noalloc(x, wp, N, cfg, out):
    M, K = x.shape
    status = _lib.lib().plm_gemm_packed_noalloc(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0), wp.data_ptr(),
                                                out.data_ptr(), out.stride(0), M, N, K, _lib.Tile.from_config(cfg),
                                                _lib.stream_handle(x.device))
    return status


CASES = [
    # (M, N, K, tile): split-K tiles use the scratch's counters and partials; the second of each pair
    # is smaller than the first.
    ((56, 2048, 8192, {"wave_frags": 2, "k_waves": 8, "split_k": 4, "unroll": 2}),
     (42, 1024, 4096, {"wave_frags": 2, "k_waves": 8, "split_k": 4, "unroll": 2})),
    ((56, 6144, 2048, {"wave_frags": 2, "k_waves": 4, "split_k": 2, "unroll": 4}),
     (7, 2048, 2048, {"wave_frags": 1, "k_waves": 4, "split_k": 8, "unroll": 2})),
    ((56, 8192, 2048, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}),
     (28, 4000, 1024, {"wave_frags": 4, "k_waves": 1, "split_k": 1, "unroll": 2})),
]


@pytest.mark.parametrize("pair", range(len(CASES)))
def test_noalloc_matches_the_workspace_entry(device, pair):
    g = torch.Generator(device=device).manual_seed(900 + pair)
    for M, N, K, cfg in CASES[pair]:
        x = torch.randn(M, K, generator=g, device=device).bfloat16()
        w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
        wp = pack_weight(w)
        ref = launch_packed(x, wp, N, cfg, torch.empty(M, N, device=device, dtype=torch.bfloat16))
        got = torch.full((M, N), float("nan"), device=device, dtype=torch.bfloat16)
        print(f"noalloc M={M} N={N} K={K} cfg={cfg}", flush=True)
        assert _noalloc(x, wp, N, cfg, got) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K, cfg)


def test_noalloc_rejects_sizes_past_its_scratch(device):
    M, N, K = 56, 50257, 2048
    cfg = {"wave_frags": 4, "k_waves": 1, "split_k": 8, "unroll": 2}
    need = _lib.lib().plm_gemm_packed_workspace_bytes(M, N, K, _lib.Tile.from_config(cfg))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(M, K, device=device, dtype=torch.bfloat16)
    wp = torch.zeros(_lib.lib().plm_packed_weight_bytes(N, K), device=device, dtype=torch.uint8)
    out = torch.empty(M, N, device=device, dtype=torch.bfloat16)
    assert _noalloc(x, wp, N, cfg, out) == -4


def _within_tolerance(got, x, w):
    import oracle

    ref = oracle.linear(x.cpu(), w.cpu()).float()
    diff = (got.cpu().float() - ref).abs()
    in_tol = diff <= 2e-2 + 1e-3 * ref.abs()
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - 7)
    assert bool((in_tol | (diff <= step * 1.0001)).all()), float(diff.max())
    assert int((~in_tol).sum()) <= max(1, got.numel() // 1000)


def test_noalloc_prefill_widths_fit_the_scratch_and_allocate_nothing(device):
    """Above 128 rows the wide kernel splits K only as far as the scratch holds (these shapes want
    20 MiB of partials with a workspace; here they run unsplit or split 2). Two calls in a row, the
    second smaller, then the same call captured in a graph and replayed: within tolerance of the
    oracle, replays bit-equal to the eager call, and the device's free memory unchanged throughout."""
    cfg = {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2}
    g = torch.Generator(device=device).manual_seed(950)
    ops = []
    for M, N, K in ((640, 2048, 2048), (256, 2048, 8192), (130, 1024, 1024)):
        x = torch.randn(M, K, generator=g, device=device).bfloat16()
        w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
        out = torch.full((M, N), float("nan"), device=device, dtype=torch.bfloat16)
        ops.append((x, w, pack_weight(w), out))
    # The wide kernel's first launch in the process (through the workspace entry) lets the runtime
    # finish its own lazy set-up for that kernel before the device's free memory is taken.
    for x, w, wp, out in ops:
        launch_packed(x, wp, w.shape[0], cfg, torch.empty_like(out))
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(device)[0]
    for _ in range(2):
        for x, w, wp, out in ops:
            print(f"noalloc wide M={x.shape[0]} N={w.shape[0]} K={x.shape[1]}", flush=True)
            assert _noalloc(x, wp, w.shape[0], cfg, out) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(device)[0] == free_before
    for x, w, wp, out in ops:
        _within_tolerance(out, x, w)
    x, w, wp, out = ops[0]
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=stream):
        assert _noalloc(x, wp, w.shape[0], cfg, out) == 0
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
