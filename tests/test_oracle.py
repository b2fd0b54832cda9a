"""Pins the CPU oracle: every function against an independent fp64 brute force, closed forms and
special cases chosen so that a plausible slip (>= for >, a dropped term, a transposed operand,
max-index instead of min-index ties) fails at least one of them. CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import golden_names, load_golden
from oracle import plm_oracle as po


def _bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers around |v| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


# --------------------------------------------------------------------------- GEMM


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_matches_fp64_brute_force(dtype):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(13, 96, generator=g).to(dtype)
    w = (0.02 * torch.randn(40, 96, generator=g)).to(dtype)
    got = oracle.linear(x, w).double().numpy()
    ref = po.linear_fp64(x, w)
    assert got.shape == (13, 40)
    # One rounding of an (almost) exact fp32 sum: within one ulp of the output dtype.
    ulp = _bf16_ulp(ref) if dtype == torch.bfloat16 else np.maximum(np.abs(ref), 2.0 ** -14) * 2.0 ** -10
    assert np.all(np.abs(got - ref) <= ulp)


def test_linear_fp32_matches_fp64():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(9, 256, generator=g).bfloat16()
    w = (0.02 * torch.randn(33, 256, generator=g)).bfloat16()
    np.testing.assert_allclose(oracle.linear_fp32(x, w).numpy(), po.linear_fp64(x, w), rtol=1e-5, atol=1e-6)


def test_linear_orientation_is_x_times_w_transposed():
    # A non-square, non-symmetric case: y[m, n] = sum_k x[m, k] w[n, k].
    x = torch.tensor([[1.0, 2.0, 0.0], [0.0, 1.0, 3.0]]).bfloat16()
    w = torch.tensor([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0], [1.0, 1.0, 1.0], [2.0, 0.0, -1.0]]).bfloat16()
    expect = torch.tensor([[1.0, 0.0, 3.0, 2.0], [0.0, 3.0, 4.0, -3.0]])
    assert torch.equal(oracle.linear(x, w).float(), expect)


def test_linear_small_integers_are_exact():
    g = torch.Generator().manual_seed(13)
    x = torch.randint(-3, 4, (7, 128), generator=g).bfloat16()
    w = torch.randint(-3, 4, (24, 128), generator=g).bfloat16()
    exact = po.linear_fp64(x, w)  # |y| <= 9*128 < 256: exactly representable in bf16
    assert np.abs(exact).max() < 256
    assert np.array_equal(oracle.linear(x, w).double().numpy(), exact)


def test_linear_one_hot_weight_selects_columns():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(5, 64, generator=g).bfloat16()
    cols = torch.tensor([3, 0, 63, 17])
    w = torch.zeros(4, 64).bfloat16()
    w[torch.arange(4), cols] = 1.0
    assert torch.equal(oracle.linear(x, w), x[:, cols])


def test_linear_reduction_order_invariance():
    # Splitting K into chunks and summing the fp32 partials stays within fp32 rounding of the whole.
    g = torch.Generator().manual_seed(15)
    x = torch.randn(6, 512, generator=g).bfloat16()
    w = (0.02 * torch.randn(20, 512, generator=g)).bfloat16()
    whole = oracle.linear_fp32(x, w)
    parts = sum(oracle.linear_fp32(x[:, i:i + 128], w[:, i:i + 128]) for i in range(0, 512, 128))
    torch.testing.assert_close(parts, whole, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- verify epilogue


def _random_logits(rows=24, vocab=300, seed=21, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return scale * torch.randn(rows, vocab, generator=g), torch.randint(0, vocab, (rows,), generator=g)


@pytest.mark.parametrize("p", [0.0, 0.3, 0.9, 0.94, 0.999])
def test_nucleus_matches_sort_brute_force(p):
    logits, pending = _random_logits()
    got = oracle.nucleus_acceptance(logits, pending, p).numpy()
    ref = po.nucleus_acceptance_fp64(logits, pending, p)
    margin = po.nucleus_margin(logits, pending, p)
    safe = margin > 1e-5
    assert np.array_equal(got[safe], ref[safe])
    assert safe.sum() >= len(safe) - 1


def test_nucleus_special_cases():
    V = 10
    one_hot = torch.full((1, V), -1e4)
    one_hot[0, 4] = 0.0
    # Proposal is the hot token: it is the maximum -> accepted for any p > 0.
    assert oracle.nucleus_acceptance(one_hot, torch.tensor([4]), 0.5).item()
    # Proposal elsewhere: everything (mass ~1) lies above it -> rejected for p < 1.
    assert not oracle.nucleus_acceptance(one_hot, torch.tensor([2]), 0.94).item()
    # Uniform logits: no token is strictly above the proposal -> mass 0 < p -> accepted.
    uniform = torch.zeros(1, V)
    assert oracle.nucleus_acceptance(uniform, torch.tensor([7]), 0.01).item()
    # p <= 0 (exact matching) accepts nothing, even the maximum or a uniform row.
    assert not oracle.nucleus_acceptance(one_hot, torch.tensor([4]), 0.0).item()
    assert not oracle.nucleus_acceptance(uniform, torch.tensor([7]), -1.0).item()
    # Strictly-above: a proposal tied with the maximum has mass-above 0 and is the max -> accepted;
    # a proposal just below two equal tops has their whole mass above it.
    tied = torch.tensor([[0.0, 5.0, 5.0, 1.0]])
    assert oracle.nucleus_acceptance(tied, torch.tensor([2]), 0.1).item()
    assert not oracle.nucleus_acceptance(tied, torch.tensor([3]), 0.5).item()
    # A proposal tied with a token that is not the maximum: the tie is not "above" it.
    mid_tie = torch.log(torch.tensor([[0.5, 0.2, 0.2, 0.1]]))
    assert oracle.nucleus_acceptance(mid_tie, torch.tensor([2]), 0.6).item()       # above = 0.5
    assert not oracle.nucleus_acceptance(mid_tie, torch.tensor([3]), 0.85).item()  # above = 0.9


def test_nucleus_boundary_is_strict_less_than():
    # Two tokens: probs (q, 1-q). The proposal is the smaller; mass above it is exactly the larger.
    big = 0.75
    logits = torch.log(torch.tensor([[big, 1 - big]], dtype=torch.float32))
    above = torch.softmax(logits, -1)[0, 0].item()
    assert not oracle.nucleus_acceptance(logits, torch.tensor([1]), above).item()   # mass < p fails at p == mass
    assert oracle.nucleus_acceptance(logits, torch.tensor([1]), above + 1e-6).item()


@pytest.mark.parametrize("eps", [2e-3, 1e-2, 0.2])
def test_floor_matches_brute_force(eps):
    logits, pending = _random_logits(seed=31)
    got = oracle.floor_acceptance(logits, pending, eps).numpy()
    assert np.array_equal(got, po.floor_acceptance_fp64(logits, pending, eps))


def test_floor_uniform_closed_form():
    V = 100  # every token has probability 1/V = 0.01
    logits = torch.zeros(1, V)
    assert oracle.floor_acceptance(logits, torch.tensor([5]), 0.009).item()
    assert not oracle.floor_acceptance(logits, torch.tensor([5]), 0.011).item()


def test_argmax_ties_go_to_lowest_index():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [7.0, 7.0, 7.0, 7.0], [0.0, -1.0, 5.0, 5.0]])
    assert oracle.argmax(logits).tolist() == [1, 0, 2]
    assert po.argmax_fp64(logits).tolist() == [1, 0, 2]
    rand, _ = _random_logits(seed=41)
    assert np.array_equal(oracle.argmax(rand).numpy(), po.argmax_fp64(rand))


def test_verify_combines_both_rules():
    logits, pending = _random_logits(seed=51)
    acc, am = oracle.verify(logits, pending, 0.94)
    assert torch.equal(acc, oracle.nucleus_acceptance(logits, pending, 0.94))
    assert torch.equal(am, oracle.argmax(logits))


# --------------------------------------------------------------------------- round epilogue


def _round_logits(k, V, favourite):
    """Logits for one round whose rows all peak sharply at ``favourite[row]``."""
    W = k + k * k
    logits = torch.full((W, V), -20.0)
    logits[torch.arange(W), favourite] = 10.0
    return logits


def test_epilogue_all_accepted():
    k, V = 3, 16
    fav = torch.arange(12) % V
    logits = _round_logits(k, V, fav)
    pending = fav[: k - 1].clone()                 # every proposal is the verify row's favourite
    verify = torch.tensor([0, 1, 9])               # verify decodes (only the last is new)
    out = oracle.epilogue(logits, verify, pending, k, "nucleus", 0.94)
    assert out["accepted"].tolist() == [True, True]
    assert out["num_correct"] == 2
    assert out["committed"].tolist() == [0, 1, 9]  # both proposals, then the verify row's token
    # Next pending: proposal block 2 (rows k+2k .. k+3k), tokens 1..k-1 of its argmax row.
    assert out["next_pending"].tolist() == fav[k + 2 * k: k + 3 * k][1:].tolist()


def test_epilogue_first_rejection_stops_the_count():
    k, V = 3, 16
    fav = (torch.arange(12) * 5) % V
    logits = _round_logits(k, V, fav)
    pending = torch.tensor([int(fav[0]) + 1, int(fav[1])])   # first proposal off the peak: rejected
    verify = torch.tensor([int(fav[0]), 2, 3])
    out = oracle.epilogue(logits, verify, pending, k, "nucleus", 0.94)
    assert out["accepted"].tolist() == [False, True]
    assert out["num_correct"] == 0
    assert out["committed"].tolist() == [int(fav[0])]
    assert out["next_pending"].tolist() == fav[k: 2 * k][1:].tolist()


def test_epilogue_exact_match_accepts_by_equality_only():
    k, V = 3, 16
    fav = torch.arange(12) % V
    logits = _round_logits(k, V, fav)
    pending = torch.tensor([4, 5])
    verify = torch.tensor([4, 6, 7])               # first proposal equals the decode, second does not
    out = oracle.epilogue(logits, verify, pending, k, "nucleus", -1.0)
    assert out["accepted"].tolist() == [True, False]
    assert out["num_correct"] == 1
    assert out["committed"].tolist() == [4, 6]


def test_epilogue_state_writes_at_the_base_and_clamps_the_sequence():
    """Hand-worked state update: k = 4, base 10, the third proposal rejected (num_correct = 2)."""
    k = 4
    widened = torch.tensor([True, False, False], dtype=torch.bool)
    pending = torch.tensor([11, 12, 13])
    verify = torch.tensor([50, 12, 60, 70])       # proposal 1 matches its decode, 0 is widened, 2 neither
    hyp = torch.arange(100, 116)                  # 4 blocks of 4 hypotheses
    out = torch.full((20,), -1, dtype=torch.int64)
    out[14] = 99                                  # slot past the round's reach keeps its value
    st = oracle.epilogue_state(widened, hyp, verify, pending, torch.tensor([0]), out, torch.tensor(10),
                               torch.tensor(30), torch.zeros(3, dtype=torch.int64), torch.tensor([5]), k, 3)
    assert st["accepted"].tolist() == [True, True, False] and st["num_correct"] == 2
    assert st["out"][10:15].tolist() == [11, 12, 60, -1, 99]
    assert st["pending"].tolist() == [109, 110, 111]   # block 2 = 108..111, entries 1..3
    assert st["anchor"].tolist() == [60]
    assert int(st["base_t"]) == 13 and int(st["offset_t"]) == 33
    assert st["round_sequence"].tolist() == [0, 0, 2] and st["sequence_step"].tolist() == [6]


def test_epilogue_state_single_proposal_round():
    """k = 1: no proposals, nothing to accept; the verify row's token is committed."""
    st = oracle.epilogue_state(torch.zeros(0, dtype=torch.bool), torch.tensor([7]), torch.tensor([42]),
                               torch.zeros(0, dtype=torch.int64), torch.tensor([0]),
                               torch.full((4,), -1, dtype=torch.int64), torch.tensor(2), torch.tensor(0),
                               torch.zeros(2, dtype=torch.int64), torch.tensor([0]), 1, 2)
    assert st["num_correct"] == 0 and st["out"].tolist() == [-1, -1, 42, -1]
    assert st["pending"].numel() == 0 and int(st["base_t"]) == 3 and st["anchor"].tolist() == [42]


# --------------------------------------------------------------------------- gated LoRA


def _lora_operands(M, shards, K, rank, seed, dtype=torch.bfloat16, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    N = sum(shards)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    a = (scale * torch.randn(len(shards) * rank, K, generator=g)).to(dtype)
    bs = [(scale * torch.randn(n, rank, generator=g)).to(dtype) for n in shards]
    return x, w, a, bs


def test_gated_lora_matches_fp64_restatement():
    x, w, a, bs = _lora_operands(21, (96, 32, 32), 256, 8, 3)
    got = oracle.gated_lora(x, w, a, bs, 5).float().numpy()
    ref = po.gated_lora_fp64(x, w, a, bs, 5)
    step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - 7)
    assert np.all(np.abs(got - ref) <= step * 1.0001)
    assert np.mean(np.abs(got - ref) > 0) < 0.02
    assert not np.array_equal(got[5:], oracle.linear(x, w).float().numpy()[5:])   # the correction is there


def test_gated_lora_without_gated_rows_or_with_zero_b_is_the_linear():
    x, w, a, bs = _lora_operands(12, (64,), 128, 4, 4)
    base = oracle.linear(x, w)
    assert torch.equal(oracle.gated_lora(x, w, a, bs, None), base)
    assert torch.equal(oracle.gated_lora(x, w, a, bs, 12), base)
    assert torch.equal(oracle.gated_lora(x, w, a, [torch.zeros_like(b) for b in bs], 0), base)


def test_gated_lora_small_integers_are_exact_per_shard():
    """Small-integer operands make every product exact: the result is integer arithmetic, and each
    shard's columns use that shard's slice of the hidden product (a one-hot A per shard)."""
    g = torch.Generator().manual_seed(5)
    M, K, rank, shards = 6, 16, 2, (8, 4, 4)
    x = torch.randint(-2, 3, (M, K), generator=g).to(torch.bfloat16)
    w = torch.randint(-2, 3, (sum(shards), K), generator=g).to(torch.bfloat16)
    a = torch.zeros(len(shards) * rank, K)
    for r in range(a.shape[0]):
        a[r, r] = 1.0                      # hidden column r = x[:, r]
    a = a.to(torch.bfloat16)
    bs = [torch.randint(-2, 3, (n, rank), generator=g).to(torch.bfloat16) for n in shards]
    got = oracle.gated_lora(x, w, a, bs, 2).to(torch.int64)
    xi, wi = x.to(torch.int64), w.to(torch.int64)
    ref = xi @ wi.T
    col = 0
    for s_, b in enumerate(bs):
        h = xi[2:, s_ * rank:(s_ + 1) * rank]
        ref[2:, col:col + b.shape[0]] += h @ b.to(torch.int64).T
        col += b.shape[0]
    assert torch.equal(got, ref)


# --------------------------------------------------------------------------- planted mistakes


def test_planted_mistakes_are_caught():
    """Mutants of the nucleus rule (>= for > in the mass, <= for < in the threshold) each disagree
    with the oracle on one of the special cases above. (The reference's "own is the maximum" clause
    cannot change a decision for p > 0, since nothing lies strictly above a maximum; it is kept for
    fidelity and has no mutant here.)"""

    def mutant(logits, pending, p, ge=False, le=False, no_max=False):
        probs = torch.softmax(logits.float(), -1)
        own = probs.gather(1, pending[:, None]).squeeze(1)
        mask = probs >= own[:, None] if ge else probs > own[:, None]
        mass = (probs * mask).sum(-1)
        inside = mass <= p if le else mass < p
        return inside if no_max else inside | ((own >= probs.amax(-1)) & (p > 0))

    uniform = torch.zeros(1, 10)
    tied = torch.tensor([[0.0, 5.0, 5.0, 1.0]])
    logits = torch.log(torch.tensor([[0.75, 0.25]]))
    above = torch.softmax(logits, -1)[0, 0].item()
    one_hot = torch.full((1, 10), -1e4)
    one_hot[0, 4] = 0.0
    mid_tie = torch.log(torch.tensor([[0.5, 0.2, 0.2, 0.1]]))
    cases = [(uniform, torch.tensor([7]), 0.01), (tied, torch.tensor([2]), 0.1), (logits, torch.tensor([1]), above),
             (one_hot, torch.tensor([4]), 0.5), (mid_tie, torch.tensor([2]), 0.6)]
    for kwargs in ({"ge": True}, {"le": True}):
        assert any(mutant(lg, pd, p, **kwargs).item() != oracle.nucleus_acceptance(lg, pd, p).item()
                   for lg, pd, p in cases), kwargs


# --------------------------------------------------------------------------- golden fixtures


@pytest.mark.parametrize("name", golden_names("gemm_"))
def test_golden_gemm(name):
    """The oracle against the committed fp64 fixtures: the fp32 product within fp32 accumulation
    error of the exact one, and the bf16 output the correctly rounded value except where fp32
    accumulation lands on the other side of a rounding midpoint (at most one step, rarely)."""
    z = load_golden(name)
    x, w = z["x"], z["w"]
    exact = z["y_fp64"]
    absdot = x.double().abs().numpy() @ w.double().abs().numpy().T
    f32 = oracle.linear_fp32(x, w).double().numpy()
    assert np.all(np.abs(f32 - exact) <= 2.0 ** -20 * absdot + 1e-30)
    got = oracle.linear(x, w).contiguous().view(torch.int16).numpy().view(np.uint16)
    want = z["y_bf16"]
    if name.endswith("_int"):
        assert np.array_equal(got, want)
    else:
        step = np.abs(got.astype(np.int32) - want.astype(np.int32))
        assert step.max() <= 1 and (step > 0).mean() <= 1e-3, (step.max(), (step > 0).sum())


def test_golden_bf16_rounding_matches_torch():
    """The fixtures' own fp64 -> bf16 rounding agrees with torch's round-to-nearest-even."""
    for name in golden_names("gemm_"):
        z = load_golden(name)
        torch_bits = torch.from_numpy(z["y_fp64"]).float().bfloat16().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(torch_bits, z["y_bf16"]), name


@pytest.mark.parametrize("name", golden_names("verify_"))
def test_golden_verify(name):
    z = load_golden(name)
    pending = torch.from_numpy(z["pending"])
    logits = oracle.linear_fp32(z["x"], z["w"])
    acc, am = oracle.verify(logits, pending, float(z["p"]))
    safe_acc, safe_am = torch.from_numpy(z["safe_accept"]), torch.from_numpy(z["safe_argmax"])
    assert torch.equal(acc[safe_acc], torch.from_numpy(z["accept"])[safe_acc])
    assert torch.equal(am[safe_am], torch.from_numpy(z["argmax"])[safe_am])
    # The fp64 brute force on fp64 logits reproduces every row, safe or not.
    exact = torch.from_numpy(z["x"].double().numpy() @ z["w"].double().numpy().T)
    assert np.array_equal(po.nucleus_acceptance_fp64(exact, pending, float(z["p"])), z["accept"])
    assert 0 < int(z["accept"].sum()) < len(z["accept"])


def test_silu_mul_is_pinned():
    """silu_mul against its fp64 restatement (equal but for a rare neighbouring rounding of silu),
    the intermediate rounding (silu(g) is rounded before the product: a single-rounding version
    differs on a sizeable share of elements), and the closed forms: g = 0 gives 0, a large positive
    gate passes u * g, a large negative one gives (about) 0, and the halves are taken in order."""
    g = torch.Generator().manual_seed(9)
    for dtype, bits in ((torch.bfloat16, 8), (torch.float16, 11)):
        y = (3 * torch.randn(64, 256, generator=g)).to(dtype)
        got = oracle.silu_mul(y).double().numpy()
        ref = oracle.silu_mul_fp64(y)
        step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - (bits - 1))
        assert np.all(np.abs(got - ref) <= step * 1.0001) and np.mean(got != ref) < 0.002
        yd = y.double().numpy()
        once = torch.from_numpy(yd[:, :128] / (1 + np.exp(-yd[:, :128])) * yd[:, 128:]).to(dtype).double().numpy()
        assert np.mean(once != got) > 0.02
    z = torch.zeros(2, 8).bfloat16()
    z[:, 4:] = 5.0
    assert torch.equal(oracle.silu_mul(z), torch.zeros(2, 4).bfloat16())
    big = torch.tensor([[20.0, -20.0, 3.0, 3.0]]).bfloat16()
    out = oracle.silu_mul(big).float()
    assert out[0, 0].item() == pytest.approx(60.0, rel=1e-2) and abs(out[0, 1].item()) < 1e-6
    swapped = oracle.silu_mul(torch.tensor([[3.0, 20.0]]).bfloat16()).float()   # gate 3, up 20
    assert swapped.item() == pytest.approx(3.0 / (1 + np.exp(-3.0)) * 20.0, rel=1e-2)
