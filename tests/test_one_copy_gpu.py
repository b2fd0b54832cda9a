"""One copy per weight: ``fast_gemm.release`` frees a weight's row-major storage and every product
with it runs on the packed copy, at the round widths (tuned tiles, plm/gemm_tables.py) and at the
prefill widths the reference hands to ``F.linear`` (M = 64 ... 640, plm/rounds.py:16; above 128 rows
as 128-row slices). Parity as tests/test_gemm_gpu.py (within one rounding of the exact product and
within tolerance of the oracle), on sampled columns for the wide calls."""

from __future__ import annotations

import gc

import pytest
import torch

from plm_amd import fast_gemm, gemm_tables
from plm_amd.fast_gemm import hip_linear, release, released_linear
from test_gemm_gpu import _inputs_on_gpu, check_cols

pytestmark = pytest.mark.gpu


def _fresh(N, K, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    return (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()


def test_release_keeps_one_copy(device):
    """Before: the row-major weight and, after the first product, its packed copy (two copies).
    After release: the packed copy alone, and products unchanged bit for bit."""
    N, K = 6144, 2048
    x, _ = _inputs_on_gpu(56, 8, K, 1, device)
    cfg = gemm_tables.read_table(K)[(56, N, K)]
    w = _fresh(N, K, 2, device)
    torch.cuda.synchronize()
    gc.collect()
    base = torch.cuda.memory_allocated(device)
    before = hip_linear(x, w, cfg)
    torch.cuda.synchronize()
    packed_bytes = fast_gemm.packed_weight(w).numel()
    assert torch.cuda.memory_allocated(device) - base >= packed_bytes  # two copies now
    release(w)
    gc.collect()
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated(device) - base
    # the row-major N*K*2 bytes are gone; what remains is the packed copy (and the output tensor)
    assert held <= packed_bytes + before.numel() * 2 + (1 << 20), (held, packed_bytes)
    assert fast_gemm.is_released(w) and w.shape == (N, K) and w.untyped_storage().nbytes() <= 2
    after = hip_linear(x, w, cfg)
    assert torch.equal(before, after)
    assert torch.equal(fast_gemm.fast_gemm(None, x, w), released_linear(x, w))


@pytest.mark.parametrize("M", [1, 7, 56, 64, 128, 200, 640])
def test_released_weight_every_width(device, M):
    """Every width runs on the packed copy and matches the oracle (tuned tile or default_config)."""
    N, K = 3072, 2048
    x, w = _inputs_on_gpu(M, N, K, 100 + M, device)
    ref_w = w.clone()
    release(w)
    y = released_linear(x, w)
    assert y.shape == (M, N)
    cols = torch.randperm(N, generator=torch.Generator().manual_seed(M))[:384]
    check_cols(y, x, ref_w, cols)
    # The same product on an unreleased copy of the weight, bit for bit: the packed kernel up to
    # 128 rows; wider, F.linear on the unpacked weight, i.e. the reference's own prefill product.
    if M <= fast_gemm.WIDE_ROWS:
        want = hip_linear(x, ref_w, fast_gemm.CONFIGS.get((M, N, K)) or fast_gemm.default_config(M, N, K))
    else:
        want = torch.nn.functional.linear(x, ref_w)
    assert torch.equal(y, want)


@pytest.mark.parametrize("N,K", [(24, 8), (1000, 1416), (300, 4096)])
def test_packed_layout_is_the_documented_one(device, N, K):
    """plm_pack_weight's bytes, element for element, against the format include/plm_amd.h states:
    fragment (f, s) = rows [16f, 16f+16) x K [32s, 32s+32), lane l = row 16f + l%16 and elements
    32s + 8(l/16) .. +8; rows padded to R (a multiple of 16 fragment rows), K steps to a multiple
    of 8, fragment (f, s) at KiB (s/8)*8R + 8f + s%8; everything past N or K zero."""
    import numpy as np

    w = _fresh(N, K, 77, device)
    p = fast_gemm.pack_weight(w).cpu().numpy()
    R = -(-(-(-N // 16)) // 16) * 16
    Ks = -(-K // 32)
    Ksp = -(-Ks // 8) * 8
    assert p.size == R * Ksp * 1024
    full = np.zeros((R * 16, Ksp * 32), dtype=np.uint16)
    full[:N, :K] = w.view(torch.int16).cpu().numpy().view(np.uint16)
    # [f, r16, s, kq, e] -> [f, s, lane = 16 kq + r16, e]
    frags = full.reshape(R, 16, Ksp, 4, 8).transpose(0, 2, 3, 1, 4).reshape(R, Ksp, 64, 8)
    # stored order: [s / 8][f][s % 8]
    want = frags.reshape(R, Ksp // 8, 8, 64, 8).transpose(1, 0, 2, 3, 4)
    got = p.view(np.uint16).reshape(Ksp // 8, R, 8, 64, 8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("N,K", [(6144, 2048), (50257, 2048), (1000, 1416), (24, 8)])
def test_unpack_restores_the_weight_bit_for_bit(device, N, K):
    w = _fresh(N, K, N + K, device)
    original = w.clone()
    release(w)
    assert torch.equal(fast_gemm.unpacked(w), original)


@pytest.mark.parametrize("M,N,K", [(129, 2048, 2048), (300, 6144, 2048), (640, 2048, 8192), (200, 1000, 1416),
                                   (777, 50257, 512)])
def test_wide_kernel(device, M, N, K):
    """plm_gemm_packed above 128 rows (the wide kernel; K split where the shape has few tiles):
    sampled columns match the oracle, the fp32 output rounds to the 16-bit one, and a second call
    is bit-identical (splits are summed in a fixed order)."""
    x, w = _inputs_on_gpu(M, N, K, 400 + M, device)
    cfg = fast_gemm.default_config(M, N, K)
    y = hip_linear(x, w, cfg)
    check_cols(y, x, w, torch.randperm(N, generator=torch.Generator().manual_seed(M))[:256])
    assert torch.equal(y, hip_linear(x, w, cfg))
    y32 = fast_gemm.hip_linear_f32(x, w, cfg)
    assert torch.equal(y32.bfloat16(), y)


def test_released_linear_shapes_bias_and_routing(device):
    """Leading dimensions and a bias, as F.linear takes them; fast_gemm routes a released weight
    through the packed kernel at an untuned width instead of F.linear."""
    N, K = 1024, 2048
    x3 = torch.randn(3, 70, K, generator=torch.Generator(device=device).manual_seed(5), device=device).bfloat16()
    w = _fresh(N, K, 6, device)
    bias = torch.randn(N, device=device).bfloat16()
    ref = torch.nn.functional.linear(x3.float(), w.float(), bias.float())
    release(w)
    got = released_linear(x3, w, bias)
    assert got.shape == (3, 70, N)
    torch.testing.assert_close(got.float(), ref, rtol=2e-2, atol=3e-2)
    fast_gemm.install({})
    try:
        routed = fast_gemm.dispatch_unquantized_gemm()(None, x3.reshape(-1, K), w, bias)
    finally:
        fast_gemm.uninstall()
    assert torch.equal(routed, got.reshape(-1, N))
    assert released_linear(x3[:0], w).shape == (0, 70, N)


def test_row_major_paths_refuse_a_released_weight(device):
    from plm_amd.verify import lm_head_verify

    N, K = 4096, 1024
    x, _ = _inputs_on_gpu(42, 8, K, 7, device)
    w = _fresh(N, K, 8, device)
    release(w)
    with pytest.raises(RuntimeError, match="released"):
        fast_gemm.hip_linear_rowmajor(x, w, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2})
    pending = torch.zeros(42, dtype=torch.int64, device=device)
    with pytest.raises(RuntimeError, match="released"):
        lm_head_verify(x, w, pending, 0.9, packed=False)
    # The packed verify reads the packed copy: the same decisions as on an unreleased copy.
    w2 = _fresh(N, K, 8, device)
    want = lm_head_verify(x, w2, pending, 0.9)
    got = lm_head_verify(x, w, pending, 0.9)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_prefill_matches_oracle_on_a_full_block(device):
    """The 1.3B block's four linears at a 640-row prefill chunk, released weights, sampled columns."""
    M, K = 640, 2048
    for i, (N, Kl) in enumerate(((6144, K), (2048, K), (8192, K), (2048, 8192))):
        x, w = _inputs_on_gpu(M, N, Kl, 300 + i, device)
        ref_w = w.clone()
        release(w)
        y = released_linear(x, w)
        cols = torch.randperm(N, generator=torch.Generator().manual_seed(i))[:256]
        check_cols(y, x, ref_w, cols)
        del ref_w
