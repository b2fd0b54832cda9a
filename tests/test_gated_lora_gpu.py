"""GPU parity of the gated-LoRA linear (plm_gemm_packed_lora, GatedLoraMethod.apply at
plm/gated_lora.py:45-57) against the oracle's restatement of the reference's unfused composition.

Shapes are the reference's Llama-style fused projections at the round width M = 56 with the gate at
k = 7 (verify rows 0..6 plain, rows 7.. adapted): QKV 2048 -> 2048+512+512 (three shards), gate/up
2048 -> 5632+5632 (two), attention-out (one), and down with a split-K tile. Parity: within 1e-3
relative / 2e-2 absolute of the oracle, or at most two output rounding steps away (the base product
and the final sum each round to bf16, and either can land on the other side of a rounding midpoint
from the oracle's), for at most 0.5 % of the elements; rows before the gate bit for bit the plain
packed GEMM."""

from __future__ import annotations

import pytest
import torch

import oracle
from plm_amd.fast_gemm import hip_linear
from plm_amd.gated_lora import GatedLoraMethod, gated_linear, rows_from

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 2e-2


def _operands(M, shards, K, rank, seed, device, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    N = sum(shards)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    a = (0.05 * torch.randn(len(shards) * rank, K, generator=g)).to(dtype)
    bs = [(0.5 * torch.randn(n, rank, generator=g)).to(dtype) for n in shards]
    return x, w, a, bs, (x.to(device), w.to(device), a.to(device), [b.to(device) for b in bs])


def _check(got: torch.Tensor, ref: torch.Tensor, dtype=torch.bfloat16):
    got, ref = got.cpu().float(), ref.float()
    diff = (got - ref).abs()
    in_tol = diff <= ATOL + RTOL * ref.abs()
    bits = 8 if dtype == torch.bfloat16 else 11
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - (bits - 1))
    assert bool((in_tol | (diff <= 2 * step * 1.0001)).all()), f"max |got - oracle| {diff.max():.4g}"
    assert int((~in_tol).sum()) <= max(1, got.numel() // 200), int((~in_tol).sum())


CASES = {
    "qkv": ((2048, 512, 512), 2048, 16, {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2}),
    "gate_up": ((5632, 5632), 2048, 16, {"wave_frags": 4, "k_waves": 8, "split_k": 1, "unroll": 2}),
    "o": ((2048,), 2048, 32, {"wave_frags": 2, "k_waves": 8, "split_k": 4, "unroll": 2}),
    "down_rowsplit": ((2048,), 5632, 16, {"wave_frags": 2, "k_waves": 1, "split_k": 2, "unroll": 4}),
    # 384 base items: more than one workgroup per CU holds, so workgroups take several items and the
    # ones that form h go on to base items.
    "qkv_many_items": ((2048, 512, 512), 2048, 16, {"wave_frags": 1, "k_waves": 8, "split_k": 2, "unroll": 2}),
    "qkv_rank64": ((2048, 512, 512), 2048, 64, {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}),
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("gate", [7, 0, 55])
def test_gated_linear_matches_the_reference_composition(device, name, gate):
    shards, K, rank, cfg = CASES[name]
    x, w, a, bs, (xg, wg, ag, bsg) = _operands(56, shards, K, rank, 10 + len(name) + gate, device)
    got = gated_linear(xg, wg, ag, bsg, gate, cfg=cfg)
    ref = oracle.gated_lora(x, w, a, bs, gate)
    _check(got, ref)
    # Rows before the gate: the plain linear with the same tile, bit for bit.
    base = hip_linear(xg, wg, cfg)
    assert torch.equal(got[:gate], base[:gate])
    # The correction is real: rows from the gate differ from the base.
    assert not torch.equal(got[gate:], base[gate:])


def test_no_gated_rows_is_the_plain_linear(device):
    shards, K, rank, cfg = CASES["qkv"]
    _, _, _, _, (xg, wg, ag, bsg) = _operands(56, shards, K, rank, 3, device)
    from plm_amd import fast_gemm

    fast_gemm.install({(56, sum(shards), K): cfg})
    try:
        assert torch.equal(gated_linear(xg, wg, ag, bsg, 56), hip_linear(xg, wg, cfg))
        assert torch.equal(gated_linear(xg, wg, ag, bsg, None), hip_linear(xg, wg, cfg))
    finally:
        fast_gemm.uninstall()


def test_fp16_and_narrow_rounds(device):
    for M, gate in ((7, 1), (42, 6), (20, 3)):
        x, w, a, bs, (xg, wg, ag, bsg) = _operands(M, (1024, 256, 256), 1024, 8, M, device, torch.float16)
        cfg = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}
        got = gated_linear(xg, wg, ag, bsg, gate, cfg=cfg)
        _check(got, oracle.gated_lora(x, w, a, bs, gate), torch.float16)


@pytest.mark.parametrize("M,gate,d", [(110, 10, 4), (96, 90, 2)])
def test_wide_rounds(device, M, gate, d):
    """Seven and six X fragments per K step (the relaxed setting's width 110) on the four-wavefront
    K split: the reference composition within tolerance, the rows before the gate bit for bit the
    plain linear."""
    x, w, a, bs, (xg, wg, ag, bsg) = _operands(M, (2048, 512, 512), 2048, 16, 40 + M, device)
    cfg = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": d}
    from plm_amd import gated_lora

    assert gated_lora._eligible(xg, wg, ag, bsg, gate, None, cfg)   # the one-launch kernel runs
    got = gated_linear(xg, wg, ag, bsg, gate, cfg=cfg)
    _check(got, oracle.gated_lora(x, w, a, bs, gate))
    assert torch.equal(got[:gate], hip_linear(xg, wg, cfg)[:gate])


def test_sixteen_wave_tiles_without_a_lora_kernel_take_the_composition(device):
    """A 16-wavefront tile with four accumulator fragments has a plain kernel but no LoRA one (its
    epilogue would spill): the call takes the reference's composition and still matches."""
    from plm_amd import fast_gemm, gated_lora

    x, w, a, bs, (xg, wg, ag, bsg) = _operands(7, (1024, 256, 256), 1024, 8, 77, device)
    cfg = {"wave_frags": 4, "k_waves": 16, "split_k": 1, "unroll": 2}
    assert fast_gemm.tile_supported(7, 1024, cfg)
    assert not gated_lora._eligible(xg, wg, ag, bsg, 3, None, cfg)
    _check(gated_linear(xg, wg, ag, bsg, 3, cfg=cfg), oracle.gated_lora(x, w, a, bs, 3))


def test_method_wrapper_routes_through_rows_from(device):
    """GatedLoraMethod.apply: outside rows_from the inner method runs; inside, the gated linear."""
    shards, K, rank, cfg = CASES["gate_up"]
    x, w, a, bs, (xg, wg, ag, bsg) = _operands(56, shards, K, rank, 21, device)

    class Inner:
        def apply(self, layer, x, bias=None):
            return hip_linear(x, layer.weight, cfg)

    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(wg, requires_grad=False)
    layer.register_buffer("lora_a", ag)
    method = GatedLoraMethod(Inner(), bsg)
    from plm_amd import fast_gemm

    fast_gemm.install({(56, sum(shards), K): cfg})
    try:
        plain = method.apply(layer, xg)
        with rows_from(7):
            gated = method.apply(layer, xg)
    finally:
        fast_gemm.uninstall()
    assert torch.equal(plain, hip_linear(xg, wg, cfg))
    _check(gated, oracle.gated_lora(x, w, a, bs, 7))
    assert torch.equal(gated[:7], plain[:7])


def _error_flag(device) -> int:
    """The workspace's error flag: set when a launch's bounded wait gave up."""
    from plm_amd import _lib, fast_gemm

    ws = fast_gemm.workspace(device, 1 << 20)
    return int(ws[: 4 * (_lib.ERROR_INDEX + 1)].view(torch.int32)[_lib.ERROR_INDEX].item())


def test_graph_replays_with_new_inputs(device):
    """One launch per call: h formed by the launch's first workgroups, the base tiles waiting for it.
    Replays of a captured call with X rewritten in place before each must each match an eager call
    on the same X bit for bit (h and the counters are fresh every launch), and no wait gives up."""
    shards, K, rank, cfg = CASES["qkv"]
    _, _, _, _, (xg, wg, ag, bsg) = _operands(56, shards, K, rank, 31, device)
    from plm_amd.gated_lora import stack_b

    b = stack_b(bsg)
    x_static = xg.clone()
    gated_linear(x_static, wg, ag, bsg, 7, cfg=cfg, lora_b=b)   # packs the weights, sizes the workspace
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = gated_linear(x_static, wg, ag, bsg, 7, cfg=cfg, lora_b=b)
    g = torch.Generator().manual_seed(5)
    for _ in range(4):
        x_new = torch.randn(56, K, generator=g).bfloat16().to(device)
        x_static.copy_(x_new)
        graph.replay()
        torch.cuda.synchronize()
        want = gated_linear(x_new, wg, ag, bsg, 7, cfg=cfg, lora_b=b)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    assert _error_flag(device) == 0


def test_back_to_back_calls_and_smaller_width(device):
    """Consecutive launches on one workspace (each leaves its counters at zero), then a narrower
    round: every result matches the oracle's composition."""
    shards, K, rank, cfg = CASES["o"]
    for M, gate, seed in ((56, 7, 41), (56, 7, 42), (42, 6, 43), (56, 20, 44)):
        x, w, a, bs, (xg, wg, ag, bsg) = _operands(M, shards, K, rank, seed, device)
        _check(gated_linear(xg, wg, ag, bsg, gate, cfg=cfg), oracle.gated_lora(x, w, a, bs, gate))
    assert _error_flag(device) == 0


def test_check_workspace_reports_and_resets_the_error_flag(device):
    """The error flag a timed-out wait sets, forced from the host (no kernel waits or faults):
    check_workspace raises once and leaves a zeroed counter area, after which launches run clean."""
    from plm_amd import _lib, fast_gemm

    shards, K, rank, cfg = CASES["qkv"]
    x, w, a, bs, (xg, wg, ag, bsg) = _operands(56, shards, K, rank, 51, device)
    gated_linear(xg, wg, ag, bsg, 7, cfg=cfg)
    torch.cuda.synchronize()
    fast_gemm.check_workspace(device)   # clean
    ws = fast_gemm.workspace(device, 1 << 20)
    ws[4 * _lib.ERROR_INDEX: 4 * (_lib.ERROR_INDEX + 1)].view(torch.int32).fill_(1)
    with pytest.raises(RuntimeError, match="gave up"):
        fast_gemm.check_workspace(device)
    assert int(ws[: _lib.COUNTER_BYTES].count_nonzero().item()) == 0
    _check(gated_linear(xg, wg, ag, bsg, 7, cfg=cfg), oracle.gated_lora(x, w, a, bs, 7))
    fast_gemm.check_workspace(device)


def test_prefill_width_with_an_explicit_tile_takes_the_composition(device):
    """Above the skinny kernel's 128 rows the one-launch correction does not apply: a call with an
    explicit round tile (a prefill chunk, plm/rounds.py:16) takes the reference's composition
    instead of failing, and matches the oracle."""
    shards, K, rank, cfg = CASES["qkv"]
    x, w, a, bs, (xg, wg, ag, bsg) = _operands(129, shards, K, rank, 21, device)
    got = gated_linear(xg, wg, ag, bsg, 7, cfg=cfg)
    _check(got, oracle.gated_lora(x, w, a, bs, 7))
