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
