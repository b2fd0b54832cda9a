"""Pins the Voronoi-decode oracle (oracle/voronoi_oracle.py) against what the mathematics fixes:
brute force, closed forms, the reference's own tile route, torch's half-precision arithmetic, and
the optimal transport assignment the fit approximates. Each planted mistake fails a check."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy.optimize import linear_sum_assignment
from scipy.special import logsumexp

from oracle import voronoi_oracle as vo


def _bf16(a) -> np.ndarray:
    return vo.bf16_round(np.asarray(a, dtype=np.float32))


def _instance(seed: int, n: int = 3, v: int = 2003, a: int = 256, scale: float = 2.0):
    rng = np.random.default_rng(seed)
    table = _bf16(rng.normal(size=(v, a)))
    logits = _bf16(rng.normal(size=(n, v)) * scale)
    return table, logits


# --------------------------------------------------------------------------- bit helpers

def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).normal(size=4096).astype(np.float32) * 100
    x[:4] = [0.0, -0.0, np.float32(1 + 2 ** -8), np.float32(1 + 3 * 2 ** -8)]  # ties to even
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(vo.bf16_round(x).view(np.uint32), ref.view(np.uint32))


def test_pack_key_orders_and_truncates():
    rng = np.random.default_rng(1)
    cost = np.concatenate([rng.normal(size=2000) * 10, [0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    target = rng.integers(0, 128, size=cost.size).astype(np.int32)
    key = vo.pack_key(cost, target)
    t, carried = vo.unpack_key(key)
    assert np.array_equal(t, target)
    # The carried cost is the cost truncated toward -inf to 16 explicit mantissa bits.
    assert np.all(carried <= cost)
    assert np.all(cost - carried <= np.abs(cost) * 2.0 ** -16 + 1e-40)
    # Keys order as the costs do wherever truncation leaves them distinct.
    order = np.argsort(key, kind="stable")
    assert np.all(np.diff(carried[order].astype(np.float64)) >= 0)


# --------------------------------------------------------------------------- shortlist

def test_top_targets_brute_force_with_ties():
    rng = np.random.default_rng(2)
    logits = _bf16(np.round(rng.normal(size=(2, 300)) * 2) / 2)   # heavy ties
    tokens, values = vo.top_targets(logits, 32)
    for r in range(2):
        brute = sorted(range(300), key=lambda i: (-float(logits[r, i]), i))[:32]
        assert tokens[r].tolist() == brute
        assert np.array_equal(values[r], logits[r, brute])


def test_top_targets_agrees_with_the_reference_tile_route():
    for seed in range(4):
        _, logits = _instance(seed, n=4, v=5003)
        tokens, values = vo.top_targets(logits, 128)
        tiled = vo.shortlist_tiled(logits, 128)
        for r in range(4):
            # Without a tie at the boundary both routes select the same set, values descending
            # (the tile route orders equal values by pool position, not token id).
            if values[r, -1] == np.sort(logits[r])[::-1][128]:
                continue
            assert sorted(tokens[r].tolist()) == sorted(tiled[r].tolist())
            assert np.array_equal(values[r], logits[r, tiled[r]])


def test_normaliser_is_logsumexp():
    _, logits = _instance(3, n=4, v=5003, scale=8.0)
    logits[1, :100] = -np.inf
    _, norm = vo.scan_logits(logits)
    assert np.allclose(norm, logsumexp(logits.astype(np.float64), axis=1), rtol=1e-6, atol=0)


def test_scan_tile_maxima():
    _, logits = _instance(4, n=2, v=1000)
    tile_max, _ = vo.scan_logits(logits, 64)
    assert tile_max.shape == (2, 16)
    for r in range(2):
        for t in range(16):
            assert tile_max[r, t] == logits[r, 64 * t:64 * t + 64].max()


def test_probabilities_are_the_shortlist_softmax():
    _, logits = _instance(5, n=3, v=3001, scale=3.0)
    tokens, values = vo.top_targets(logits, 64)
    _, norm = vo.scan_logits(logits)
    p = vo.probabilities(values, norm)
    exact = np.exp(values.astype(np.float64) - values.astype(np.float64).max(axis=1, keepdims=True))
    exact /= exact.sum(axis=1, keepdims=True)
    assert np.allclose(p, exact, rtol=2e-6, atol=1e-9)


def _hamilton(weights: np.ndarray, total: int) -> np.ndarray:
    """Seat-by-seat largest remainder: floors, then one seat at a time to the largest remaining
    remainder (lowest position on ties)."""
    exact = [float(np.float32(w) * np.float32(total)) for w in weights]
    seats = [int(np.floor(e)) for e in exact]
    rem = [np.float32(e) - np.float32(s) for e, s in zip(exact, seats)]
    taken = set()
    for _ in range(total - sum(seats)):
        best = max((i for i in range(len(rem)) if i not in taken), key=lambda i: (rem[i], -i))
        taken.add(best)
        seats[best] += 1
    return np.array(seats)


def test_quota_textbook_and_brute_force():
    assert vo.quota(np.array([[0.5, 0.3, 0.2]], dtype=np.float32), 10).tolist() == [[5, 3, 2]]
    assert vo.quota(np.full((1, 3), np.float32(1 / 3)), 10).tolist() == [[4, 3, 3]]
    assert vo.quota(np.full((1, 4), np.float32(0.25)), 8).tolist() == [[2, 2, 2, 2]]
    rng = np.random.default_rng(6)
    for _ in range(50):
        w = rng.dirichlet(np.ones(17) * 0.3).astype(np.float32)
        c = vo.quota(w[None], 256)[0]
        assert c.sum() == 256
        assert np.all(np.abs(c - w.astype(np.float64) * 256) < 1.0 + 1e-4)
        assert np.array_equal(c, _hamilton(w, 256))


# --------------------------------------------------------------------------- spread / prior

def test_spread_against_torch_half_arithmetic():
    table, logits = _instance(7, n=3, v=700, a=128)
    tokens, _ = vo.top_targets(logits, 32)
    for dtype, torch_dtype in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        tab = table if dtype == "bf16" else table.astype(np.float16).astype(np.float32)
        head = torch.from_numpy(tab).to(torch_dtype)[torch.from_numpy(tokens)][:, :, :64]
        ref = (head.amax(1) - head.amin(1)).double().mean(-1).float().numpy()
        assert np.array_equal(vo.spread(tab, tokens, dtype), ref)


def test_prior_closed_forms():
    counts = np.array([[256, 0, 0, 0], [64, 64, 128, 0]])
    unit = np.array([2.0, 0.5], dtype=np.float32)
    pr = vo.prior(counts, unit, 256)
    assert pr[0, 0] == 0.0 and np.all(pr[0, 1:] == np.float32(1000 * 2.0))
    assert np.isclose(pr[1, 0], -0.1 * 0.5 * np.log(0.25), rtol=1e-6)
    assert np.isclose(pr[1, 2], -0.1 * 0.5 * np.log(0.5), rtol=1e-6)
    assert pr[1, 3] == np.float32(500.0)


# --------------------------------------------------------------------------- condense

def test_condense_brute_force():
    table, logits = _instance(8, n=2, v=500, a=64)
    tokens, _ = vo.top_targets(logits, 16)
    offset = np.random.default_rng(8).normal(size=(2, 16)).astype(np.float32)
    key = vo.condense(table, tokens, offset, 4)
    assert key.shape == (2, 4, 64)
    checked = 0
    for p in range(2):
        for a in range(64):
            cost = (table[tokens[p], a] + offset[p]).astype(np.float32).astype(np.float64)
            ranked = sorted(range(16), key=lambda m: (cost[m], m))
            gaps = np.diff(cost[ranked[:5]])
            if np.any(gaps <= np.abs(cost[ranked[:5]]).max() * 2.0 ** -15):
                continue   # the key's 16-bit mantissa may order these two either way
            target, carried = vo.unpack_key(key[p, :, a])
            assert target.tolist() == ranked[:4]
            assert np.all(np.abs(carried - cost[ranked[:4]]) <= np.abs(cost[ranked[:4]]) * 2.0 ** -16)
            checked += 1
    assert checked > 100


# --------------------------------------------------------------------------- fit

def _fit_loops(key, counts, offset, unit, iterations, epsilon, relax=1.9, endpoint=0.0087, limit=0.25):
    """Independent float64 restatement with explicit per-item loops."""
    n, k, a = key.shape
    m = counts.shape[1]
    out = np.zeros((n, m))
    anneal = (endpoint / epsilon) ** (1.0 / max(iterations, 1))
    for p in range(n):
        tgt, base = vo.unpack_key(key[p])
        u = float(unit[p])
        temp, bound = epsilon * u, limit * u
        corr = np.zeros(m)
        share = np.log(np.maximum(counts[p].astype(np.float64), 1e-9))
        for _ in range(iterations):
            load = np.zeros(m)
            for item in range(a):
                c = [float(base[s, item]) + corr[tgt[s, item]] for s in range(k)]
                z = [-ci / temp for ci in c]
                zmax = max(z)
                e = [np.exp(zi - zmax) for zi in z]
                tot = sum(e)
                for s in range(k):
                    load[tgt[s, item]] += e[s] / tot
            step = temp * (np.log(np.maximum(load, 0.01)) - share)
            step = np.clip(step, -bound, bound)
            corr = np.where(counts[p] > 0, corr + relax * step, 0.0)
            temp *= anneal
        out[p] = offset[p] + corr
    return out


def _fit_case(seed: int, a: int = 64, m: int = 16, k: int = 8):
    table, logits = _instance(seed, n=2, v=400, a=a)
    tokens, counts, _, _ = vo.shortlist(logits, a, m)
    unit = vo.spread(table, tokens, "bf16")
    prior = vo.prior(counts, unit, a)
    key = vo.condense(table, tokens, prior, k)
    return table, tokens, counts, unit, prior, key


def test_fit_matches_fp64_loops():
    _, _, counts, unit, prior, key = _fit_case(9)
    ours = vo.fit(key, counts, prior, unit, 12, 0.15)
    ref = _fit_loops(key, counts, prior, unit, 12, 0.15)
    scale = unit[:, None].astype(np.float64)
    assert np.max(np.abs(ours - ref) / scale) < 2e-5


def test_fit_planted_mistakes_fail():
    _, _, counts, unit, prior, key = _fit_case(10)
    ref = _fit_loops(key, counts, prior, unit, 12, 0.15)
    scale = unit[:, None].astype(np.float64)
    for wrong in (dict(relax=1.0), dict(limit=0.01), dict(endpoint=0.02)):
        assert np.max(np.abs(_fit_loops(key, counts, prior, unit, 12, 0.15, **wrong) - ref) / scale) > 1e-3
    assert np.max(np.abs(vo.fit(key, counts, prior, unit, 11, 0.15) - ref) / scale) > 1e-3


def _transport_assignment(cost: np.ndarray, counts: np.ndarray) -> np.ndarray:
    """The optimal transport assignment: each item to one target, target m taking exactly counts[m]
    items, minimum total cost (scipy's Hungarian solver on targets expanded into seats)."""
    seats = np.repeat(np.arange(cost.shape[0]), counts)
    rows, cols = linear_sum_assignment(cost[seats].T)
    out = np.empty(cost.shape[1], dtype=np.int64)
    out[rows] = seats[cols]
    return out


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_fit_converges_to_the_transport_optimum(seed):
    # With every target condensed in (k = M) and a long, cold anneal, the fitted factors are the
    # transport problem's dual: argmin_m C + b reproduces the optimal assignment's shares and cost.
    a, m = 64, 8
    table, tokens, counts, unit, prior, _ = _fit_case(seed, a=a, m=m, k=m)
    zero = np.zeros_like(prior)
    key = vo.condense(table, tokens, zero, m)
    bias = vo.fit(key, counts, zero, unit, 600, 0.15, relax=1.0, endpoint=2e-4)
    sigma = vo.argmin(table, tokens, bias)
    for p in range(tokens.shape[0]):
        cost = vo.costs(table, tokens)[p].astype(np.float64)
        opt = _transport_assignment(cost, counts[p])
        got = np.bincount(sigma[p], minlength=m)
        assert np.abs(got - counts[p]).sum() <= 2
        ours = cost[sigma[p], np.arange(a)].sum()
        best = cost[opt, np.arange(a)].sum()
        assert ours <= best + 0.02 * abs(best) + 0.05 * unit[p]


def test_fit_sign_mistake_breaks_the_transport_shares():
    a, m = 64, 8
    table, tokens, counts, unit, prior, _ = _fit_case(11, a=a, m=m, k=m)
    zero = np.zeros_like(prior)
    key = vo.condense(table, tokens, zero, m)
    bias = vo.fit(key, counts, zero, unit, 600, 0.15, relax=1.0, endpoint=2e-4)
    flipped = -(bias - zero)
    sigma = vo.argmin(table, tokens, flipped)
    assert np.abs(np.bincount(sigma[0], minlength=m) - counts[0]).sum() > 4


# --------------------------------------------------------------------------- argmin / assign

def test_argmin_brute_force_and_ties():
    table, logits = _instance(14, n=2, v=300, a=64)
    tokens, _ = vo.top_targets(logits, 16)
    bias = np.random.default_rng(14).normal(size=(2, 16)).astype(np.float32)
    sigma = vo.argmin(table, tokens, bias)
    for p in range(2):
        for a in range(64):
            c = [np.float32(table[tokens[p, m], a]) + bias[p, m] for m in range(16)]
            assert sigma[p, a] == min(range(16), key=lambda m: (c[m], m))
    # exact ties resolve to the lowest target index
    tie = np.zeros((1, 4), dtype=np.float32)
    flat = np.zeros((8, 64), dtype=np.float32)
    assert np.all(vo.argmin(flat, np.array([[3, 1, 2, 0]]), tie) == 0)


def test_assign_shares_follow_the_quotas():
    table, logits = _instance(15, n=3, v=2003, a=256)
    st = vo.assign(table, logits, "bf16", n_targets=64, k=8)
    for p in range(3):
        assert st["counts"][p].sum() == 256
        got = np.bincount(st["sigma"][p], minlength=64)
        assert np.abs(got - st["counts"][p]).sum() <= 0.15 * 256
        # the prior alone (no fit) is much further from the quotas
    pri = vo.argmin(table, st["tokens"], st["prior"])
    far = sum(np.abs(np.bincount(pri[p], minlength=64) - st["counts"][p]).sum() for p in range(3))
    near = sum(np.abs(np.bincount(st["sigma"][p], minlength=64) - st["counts"][p]).sum() for p in range(3))
    assert near < far


def test_decode_unmasked_reads_sigma():
    table, logits = _instance(16, n=4, v=1000, a=128)
    values = np.array([0, 5, 127, 300])   # the last one clamps to 127
    st = vo.assign(table, logits, "bf16", n_targets=32, k=8)
    dec = vo.decode_unmasked(table, logits, values, "bf16", n_targets=32, k=8)
    for p, v in enumerate(np.minimum(values, 127)):
        assert dec[p] == st["tokens"][p, st["sigma"][p, v]]


def test_build_table_is_negated_transposed_scores():
    g = torch.Generator().manual_seed(0)
    vocab = torch.randn(64, 32, generator=g).to(torch.bfloat16)
    w = torch.randn(100, 32, generator=g).to(torch.bfloat16)
    t = vo.build_table(vocab, w)
    assert t.shape == (100, 64) and t.dtype == torch.bfloat16
    exact = -(w.double() @ vocab.double().T)
    assert torch.allclose(t.double(), exact, rtol=2 ** -7, atol=1e-2)
