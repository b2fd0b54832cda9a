"""GPU parity of the fused gate/up projection with its SiLU-and-multiply (plm_gemm_packed_silu_mul,
``fast_gemm.gate_up_silu``) against the oracle's restatement of the two launches the reference's
Llama-style rounds make through vLLM (the gate_up_proj GEMM, then ``SiluAndMul`` on its
model-dtype output: silu rounded to the model dtype, times u, rounded).

Two checks per case: against the same projection on this build's kernel with the same tile
(``hip_linear``, whose fp32 sums are the fused kernel's bit for bit: the interleaving only moves
rows) followed by the oracle's activation, at most one model-dtype step apart on at most 0.1 % of
the elements (the device's and the CPU's exp differ in the last fp32 bits); and against the oracle
end to end (F.linear on the CPU, then the activation) within 1e-3 relative / 2e-2 absolute, or
two steps (a projection output one step off is amplified by at most |u| or the SiLU slope)."""

from __future__ import annotations

import pytest
import torch

import oracle
from plm_amd import fast_gemm
from plm_amd.fast_gemm import gate_up_silu, hip_linear

pytestmark = pytest.mark.gpu


def _steps(got: torch.Tensor, ref: torch.Tensor, dtype) -> torch.Tensor:
    bits = 8 if dtype == torch.bfloat16 else 11
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - (bits - 1))
    return (got - ref).abs() / step


CASES = [
    # M, I (N = 2I), K, tile
    (56, 5632, 2048, {"wave_frags": 4, "k_waves": 8, "split_k": 1, "unroll": 2}),   # Llama 1.3B, tuned tile
    (56, 5632, 2048, {"wave_frags": 2, "k_waves": 8, "split_k": 4, "unroll": 2}),   # K split
    (42, 8192, 3072, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}),
    (7, 1024, 1024, {"wave_frags": 2, "k_waves": 16, "split_k": 2, "unroll": 2}),
    (110, 5632, 2048, {"wave_frags": 2, "k_waves": 1, "split_k": 1, "unroll": 4}),  # row-split
    (110, 5632, 2048, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}),  # seven X fragments, K split
    (96, 1408, 512, {"wave_frags": 2, "k_waves": 4, "split_k": 2, "unroll": 2}),
    (56, 1408, 512, {"wave_frags": 4, "k_waves": 1, "split_k": 3, "unroll": 2}),    # row-split, K split
]


@pytest.mark.parametrize("M,I,K,cfg", CASES)
def test_gate_up_silu_matches_the_two_launches(device, M, I, K, cfg):
    g = torch.Generator(device=device).manual_seed(M + I + K)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.03 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()
    got = gate_up_silu(x, w, cfg)
    assert got.shape == (M, I)
    # Same sums: this build's projection with the same tile, then the activation.
    same = oracle.silu_mul(hip_linear(x, w, cfg)).float()
    st = _steps(got.cpu().float(), same, torch.bfloat16)
    assert float(st.max()) <= 1.0001 and int((st > 0.5).sum()) <= max(1, got.numel() // 1000), float(st.max())
    # End to end against the oracle on CPU copies of sampled output columns.
    cols = torch.randperm(I, generator=torch.Generator().manual_seed(M))[:256]
    rows = torch.cat([cols, cols + I]).to(device)
    ref = oracle.silu_mul(oracle.linear(x.cpu(), w[rows].cpu())).float()
    sub = got[:, cols.to(device)].cpu().float()
    diff = (sub - ref).abs()
    ok = (diff <= 2e-2 + 1e-3 * ref.abs()) | (_steps(sub, ref, torch.bfloat16) <= 2.0001)
    assert bool(ok.all()), float(diff.max())


@pytest.mark.parametrize("M,I,K", [(1, 16, 64), (128, 48, 1416), (17, 1008, 200), (64, 2048, 8192)])
def test_edge_shapes_default_tile(device, M, I, K):
    """One row and the widest skinny width, the smallest pair of fragments (I = 16), K past the
    last 32-element step (1416, 200), a long K; the tile gate_up_silu picks by default."""
    g = torch.Generator(device=device).manual_seed(M * 7 + I + K)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.03 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()
    got = gate_up_silu(x, w)
    ref = oracle.silu_mul(oracle.linear(x.cpu(), w.cpu())).float()
    diff = (got.cpu().float() - ref).abs()
    ok = (diff <= 2e-2 + 1e-3 * ref.abs()) | (_steps(got.cpu().float(), ref, torch.bfloat16) <= 2.0001)
    assert bool(ok.all()), float(diff.max())


def test_fp16_wide_rows_and_released_weight(device):
    g = torch.Generator(device=device).manual_seed(5)
    I, K = 1024, 1024
    for M in (20, 200):   # 200 rows: the projection then the activation
        x = torch.randn(M, K, generator=g, device=device).half()
        w = (0.03 * torch.randn(2 * I, K, generator=g, device=device)).half()
        got = gate_up_silu(x, w)
        ref = oracle.silu_mul(oracle.linear(x.cpu(), w.cpu())).float()
        diff = (got.cpu().float() - ref).abs()
        ok = (diff <= 2e-2 + 1e-3 * ref.abs()) | (_steps(got.cpu().float(), ref, torch.float16) <= 2.0001)
        assert bool(ok.all()), (M, float(diff.max()))
    # A released weight: the interleaved copy is rebuilt from the packed one.
    x = torch.randn(56, K, generator=g, device=device).bfloat16()
    w = (0.03 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()
    want = gate_up_silu(x, w.clone())
    fast_gemm.release(w)
    assert torch.equal(gate_up_silu(x, w), want)


def test_argument_checks(device):
    """Shapes the entry point refuses (PLM_ERR_ARG) before launching; every buffer is sized for the
    call anyway."""
    from plm_amd import _lib

    lib = _lib.lib()
    M, K = 8, 64
    x = torch.randn(M, K, device=device).bfloat16()
    w = torch.zeros(int(lib.plm_packed_weight_bytes(96, K)), dtype=torch.uint8, device=device)
    y = torch.empty(M, 48, device=device).bfloat16()

    def call(N, tile, ldy=48):
        return lib.plm_gemm_packed_silu_mul(0, x.data_ptr(), K, w.data_ptr(), y.data_ptr(), ldy, M, N, K, tile,
                                            None, 0, None)

    assert call(80, _lib.Tile(2, 8, 1, 2)) == -1          # N not a multiple of 32
    assert call(64, _lib.Tile(1, 8, 1, 2)) == -1          # wave_frags 1: gate and up fragments unpaired
    assert call(96, _lib.Tile(2, 8, 1, 2), ldy=40) == -1  # ldy below N/2
    assert call(64, _lib.Tile(2, 8, 1, 2), ldy=34) == -1  # ldy not a multiple of 4
    assert call(64, _lib.Tile(2, 8, 1, 2)) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,I,K", [(56, 5632, 2048), (42, 8192, 3072), (7, 1408, 512), (200, 1408, 512)])
def test_llama_mlp_matches_the_reference_composition(device, M, I, K):
    """fast_gemm.llama_mlp: the gate/up projection, SiluAndMul and down (the reference's three
    steps, each rounded to the model dtype) against the oracle run end to end on the CPU: within
    1e-3 relative / 2e-2 absolute, or a few output steps where an intermediate value one step off is
    carried through down's sum, on at most 0.5 % of the elements; bit for bit this build's two
    launches."""
    g = torch.Generator().manual_seed(M + I)
    x = torch.randn(M, K, generator=g).bfloat16()
    wgu = (0.02 * torch.randn(2 * I, K, generator=g)).bfloat16()
    wd = (0.02 * torch.randn(K, I, generator=g)).bfloat16()
    got = fast_gemm.llama_mlp(x.to(device), wgu.to(device), wd.to(device)).cpu().float()
    ref = oracle.linear(oracle.silu_mul(oracle.linear(x, wgu)), wd).float()
    diff = (got - ref).abs()
    in_tol = diff <= 2e-2 + 1e-3 * ref.abs()
    assert bool((in_tol | (_steps(got, ref, torch.bfloat16) <= 4.0001)).all()), float(diff.max())
    assert int((~in_tol).sum()) <= max(1, got.numel() // 200), int((~in_tol).sum())
    if M <= 128:
        act = gate_up_silu(x.to(device), wgu.to(device))
        cfg = fast_gemm.CONFIGS.get((M, K, I)) or fast_gemm.default_config(M, K, I)
        assert torch.equal(got, hip_linear(act, wd.to(device), cfg).cpu().float())
