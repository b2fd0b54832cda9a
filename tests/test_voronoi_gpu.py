"""GPU parity of the verify rows' auxiliary decode (csrc/voronoi.hip) against the oracle
(oracle/voronoi_oracle.py, restating plm/iterate.py and plm/auxiliary.py:67-75).

Bars, per stage, on the same inputs:
* shortlist tokens and values, condense keys, argmin for a given bias: bit-exact (integer and
  selection work; ties resolve by token id / shortlist position / lowest target, as the oracle's);
* quota counts: exact wherever no probability sits within 1e-3 items of a rounding boundary (the
  reference's own fp32 sums have no fixed order either); every instance here is checked for that;
* normaliser, unit, prior: within 1e-6 / 1e-6 / 2e-6 relative (fp32 reductions in another order);
* fitted factors: within 2e-4 units (``unit``: the problem's cost scale) — fp32 weights formed with
  a reciprocal multiply and the hardware exp against numpy's; the loads are exact sums on both sides;
* assignments and decoded tokens: equal on every item whose best and second-best costs differ by
  more than 1e-3 units; the rest (reported) may fall either way.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import voronoi_oracle as vo
from plm_amd.fast_gemm import hip_linear
from plm_amd.verify import LOGITS_CONFIG, AuxRoundVerify, lm_head_verify, lm_head_verify_logits
from plm_amd.voronoi import LogitVoronoiAuxiliary, Voronoi, condense

pytestmark = pytest.mark.gpu

FIT_TOL = 2e-4      # fitted factors, in units
TIE_TOL = 1e-3      # assignments closer than this (in units) to a tie may differ


def _half(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _case(seed: int, n: int, v: int, a: int, dtype=torch.bfloat16, scale: float = 2.5, kind: str = "normal"):
    g = torch.Generator().manual_seed(seed)
    table = torch.randn(v, a, generator=g).to(dtype)
    if kind == "normal":
        logits = (torch.randn(n, v, generator=g) * scale).to(dtype)
    elif kind == "ties":          # values on a 0.5 grid: thousands of equal logits near the top
        logits = (torch.round(torch.randn(n, v, generator=g) * 2) / 2).to(dtype)
    elif kind == "flat":          # every logit equal: the top targets are tokens 0..M-1
        logits = torch.full((n, v), 0.5).to(dtype)
    else:
        raise ValueError(kind)
    return table, logits


def _quota_sensitive(values: np.ndarray, norm: np.ndarray, n_items: int) -> np.ndarray:
    """Per problem: True if some quota could round either way. A share ``exact = p * A`` carries a
    relative fp32 error of a few 1e-6 (exp, the normaliser, the sum), so it is sensitive when it
    lies within 1e-5 * exact of an integer, or when the last awarded and first unawarded remainders
    (of different logits: equal logits have equal shares in any order of arithmetic) lie within
    1e-5 of the larger share of each other. A row of equal logits has exactly equal shares."""
    p = np.exp(values.astype(np.float64) - norm[:, None].astype(np.float64))
    exact = p / p.sum(axis=1, keepdims=True) * n_items
    frac = exact - np.floor(exact)
    tol = 1e-5 * exact + 1e-9
    out = np.zeros(len(values), dtype=bool)
    for r in range(len(values)):
        if np.all(values[r] == values[r, 0]):
            continue
        near_floor = np.any(np.minimum(frac[r], 1 - frac[r]) < tol[r])
        remaining = n_items - int(np.floor(exact[r]).sum())
        order = np.argsort(-frac[r], kind="stable")
        near_rank = False
        if 0 < remaining < len(order):
            i, j = order[remaining - 1], order[remaining]
            near_rank = values[r, i] != values[r, j] and frac[r, i] - frac[r, j] < max(tol[r, i], tol[r, j])
        out[r] = near_floor or near_rank
    return out


def _dtype_name(dtype) -> str:
    return "bf16" if dtype == torch.bfloat16 else "f16"


SHORTLIST_CASES = [
    # (seed, n, V, A, M, dtype, kind)
    (0, 7, 50257, 4096, 128, torch.bfloat16, "normal"),
    (1, 3, 50304, 1024, 64, torch.float16, "normal"),
    (2, 2, 1000, 64, 16, torch.bfloat16, "normal"),
    (3, 4, 50257, 4096, 128, torch.bfloat16, "ties"),
    (4, 2, 50257, 2048, 128, torch.bfloat16, "flat"),
    (5, 1, 128, 256, 128, torch.float16, "normal"),
]


@pytest.mark.parametrize("seed,n,v,a,m,dtype,kind", SHORTLIST_CASES)
def test_shortlist_matches_the_oracle(device, seed, n, v, a, m, dtype, kind):
    table, logits = _case(seed, n, v, a, dtype, kind=kind)
    print(f"shortlist case seed={seed} n={n} V={v} A={a} M={m} {dtype} {kind}", flush=True)
    eng = Voronoi.from_table(table.to(device))
    tokens, counts, unit, prior = eng._shortlist(logits.to(device), m, 0.1)
    # values and the normaliser through the C ABI's optional outputs
    from plm_amd import _lib
    values = torch.empty(n, m, dtype=torch.float32, device=device)
    norm = torch.empty(n, dtype=torch.float32, device=device)
    t2, c2 = torch.empty_like(tokens), torch.empty_like(counts)
    u2, p2 = torch.empty_like(unit), torch.empty_like(prior)
    lg = logits.to(device)
    status = _lib.lib().plm_voronoi_shortlist(_lib.DTYPE_CODES[dtype], lg.data_ptr(), lg.stride(0),
                                              eng.table.data_ptr(), n, v, a, m, 0.1, t2.data_ptr(), c2.data_ptr(),
                                              values.data_ptr(), u2.data_ptr(), p2.data_ptr(), norm.data_ptr(),
                                              _lib.stream_handle(device))
    _lib.check(status, "plm_voronoi_shortlist")
    torch.cuda.synchronize()
    assert torch.equal(t2, tokens) and torch.equal(c2, counts) and torch.equal(u2, unit) and torch.equal(p2, prior)

    lg_np, tab_np = _np(logits), _np(table)
    ref_tokens, ref_counts, ref_values, ref_norm = vo.shortlist(lg_np, a, m)
    assert np.array_equal(tokens.cpu().numpy(), ref_tokens)
    assert np.array_equal(_np(values), ref_values)
    assert np.allclose(_np(norm), ref_norm, rtol=1e-6, atol=0)
    if kind == "flat":
        assert np.array_equal(ref_tokens, np.tile(np.arange(m), (n, 1)))
    sensitive = _quota_sensitive(ref_values, ref_norm, a)
    print(f"  quota-sensitive problems: {int(sensitive.sum())} of {n}", flush=True)
    got_counts = counts.cpu().numpy()
    assert np.all(got_counts.sum(axis=1) == a)
    assert np.array_equal(got_counts[~sensitive], ref_counts[~sensitive])
    assert sensitive.sum() <= max(1, n // 4)
    ref_unit = vo.spread(tab_np, ref_tokens, _dtype_name(dtype))
    assert np.allclose(_np(unit), ref_unit, rtol=1e-6, atol=0)
    # prior from the kernel's own counts and unit (the formula, not the counts, is under test here)
    ref_prior = vo.prior(got_counts, _np(unit), a)
    assert np.allclose(_np(prior), ref_prior, rtol=2e-6, atol=0)
    # the standalone spread / prior entry points agree with the fused ones
    assert torch.equal(eng.spread(tokens)[:, 0], unit)
    assert torch.equal(eng.prior(counts, unit), prior)


def _stage_inputs(seed: int, n: int = 7, v: int = 50257, a: int = 4096, m: int = 128):
    table, logits = _case(seed, n, v, a)
    tab_np = _np(table)
    tokens, counts, _, _ = vo.shortlist(_np(logits), a, m)
    unit = vo.spread(tab_np, tokens, "bf16")
    prior = vo.prior(counts, unit, a)
    return table, logits, tab_np, tokens, counts, unit, prior


@pytest.mark.parametrize("k", [8, 4, 16])
def test_condense_is_bit_exact(device, k):
    a = 4096 if k <= 8 else 2048
    table, _, tab_np, tokens, _, _, prior = _stage_inputs(10 + k, n=5, a=a)
    key = condense(table.to(device), torch.from_numpy(tokens).to(device), torch.from_numpy(prior).to(device), k)
    ref = vo.condense(tab_np, tokens, prior, k)
    assert np.array_equal(key.cpu().numpy(), ref)


@pytest.mark.parametrize("k,a,iterations,eps", [(8, 4096, 12, 0.15), (8, 4096, 12, 0.0525), (4, 8192, 12, 0.15),
                                                (8, 512, 24, 0.15), (16, 1024, 12, 0.15)])
def test_fit_matches_the_oracle(device, k, a, iterations, eps):
    table, _, tab_np, tokens, counts, unit, prior = _stage_inputs(20 + k + a, n=5, a=a)
    key = vo.condense(tab_np, tokens, prior, k)
    eng = Voronoi.from_table(table.to(device))
    args = [torch.from_numpy(x).to(device) for x in (key, counts, prior, unit)]
    bias = eng.fit(*args, iterations, eps)
    again = eng.fit(*args, iterations, eps)
    assert torch.equal(bias, again)       # reproducible bit for bit
    ref = vo.fit(key, counts, prior, unit, iterations, eps)
    err = np.abs(_np(bias) - ref) / unit[:, None]
    print(f"fit k={k} A={a} iters={iterations} eps={eps}: max error {err.max():.3e} units", flush=True)
    assert err.max() < FIT_TOL


def test_fit_with_one_dominant_target(device):
    """One token's logit raised so that its quota is about half of the items: its loads are the
    largest the fit sums, and most lanes of an add instruction carry a weight for it."""
    a, k, m = 4096, 8, 128
    table, logits = _case(33, 5, 50257, a)
    lg = _np(logits)
    lg[:, 777] = lg.max(axis=1) + 4.0
    tab_np = _np(table)
    tokens, counts, _, _ = vo.shortlist(lg, a, m)
    assert (counts.max(axis=1) > a // 3).all()
    unit = vo.spread(tab_np, tokens, "bf16")
    prior = vo.prior(counts, unit, a)
    key = vo.condense(tab_np, tokens, prior, k)
    eng = Voronoi.from_table(table.to(device))
    args = [torch.from_numpy(x).to(device) for x in (key, counts, prior, unit)]
    bias = eng.fit(*args, 12, 0.15)
    assert torch.equal(bias, eng.fit(*args, 12, 0.15))
    ref = vo.fit(key, counts, prior, unit, 12, 0.15)
    err = np.abs(_np(bias) - ref) / unit[:, None]
    print(f"fit with one dominant target: max error {err.max():.3e} units", flush=True)
    assert err.max() < FIT_TOL


def test_argmin_for_a_given_bias(device):
    table, _, tab_np, tokens, counts, unit, prior = _stage_inputs(30, n=4, a=2048)
    bias = vo.fit(vo.condense(tab_np, tokens, prior, 8), counts, prior, unit, 12, 0.15)
    eng = Voronoi.from_table(table.to(device))
    sigma = eng.argmin(torch.from_numpy(tokens).to(device), torch.from_numpy(bias).to(device)).cpu().numpy()
    assert np.array_equal(sigma, vo.argmin(tab_np, tokens, bias))


def _compare_assign(device, table, logits, a, m=128, k=8, rounds=2, iterations=12):
    eng = Voronoi.from_table(table.to(device))
    got = eng.assign(logits.to(device), n_targets=m, k=k, rounds=rounds, iterations=iterations)
    ref = vo.assign(_np(table), _np(logits), _dtype_name(table.dtype), n_targets=m, k=k, rounds=rounds,
                    iterations=iterations)
    assert np.array_equal(got.tokens.cpu().numpy(), ref["tokens"])
    sensitive = _quota_sensitive(ref["values"], ref["normaliser"], a)
    assert not sensitive.any(), "pick another seed: this instance's quotas sit on a rounding boundary"
    assert np.array_equal(got.counts.cpu().numpy(), ref["counts"])
    err = np.abs(_np(got.bias) - ref["bias"]) / ref["unit"][:, None]
    margin = vo.argmin_margin(_np(table), ref["tokens"], ref["bias"]) / ref["unit"][:, None]
    sigma = got.sigma.cpu().numpy()
    differ = sigma != ref["sigma"]
    print(f"assign n={logits.shape[0]} A={a}: bias error {err.max():.3e} units, sigma differs on "
          f"{int(differ.sum())} of {differ.size} items (near ties: {int((margin < TIE_TOL).sum())})", flush=True)
    assert err.max() < 5 * FIT_TOL
    assert not np.any(differ & (margin >= TIE_TOL))
    assert differ.mean() < 1e-3
    return got, ref


def test_assign_end_to_end(device):
    table, logits = _case(40, 7, 50257, 4096)
    _compare_assign(device, table, logits, 4096)


def test_assign_fp16_small(device):
    table, logits = _case(41, 3, 3001, 512, torch.float16, scale=1.5)
    _compare_assign(device, table, logits, 512, m=64, k=4, rounds=3, iterations=8)


def test_decode_unmasked_through_the_scheme(device):
    """LogitVoronoiAuxiliary.decode_unmasked with the table built from an auxiliary vocabulary and
    an LM head; the oracle decodes from the same table (read back from the GPU)."""
    g = torch.Generator().manual_seed(50)
    A, H, V, n = 4096, 2048, 50257, 7
    scheme = LogitVoronoiAuxiliary(A, H, V, dtype=torch.bfloat16).to(device)
    scheme.auxiliary_vocabulary.copy_((torch.randn(A, H, generator=g) * 0.02).to(torch.bfloat16))
    w = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16).to(device)
    x = torch.randn(n, H, generator=g).to(torch.bfloat16).to(device)
    logits = hip_linear(x, w, LOGITS_CONFIG)
    values = torch.randint(0, A, (n,), generator=g)
    values[0] = A + 5                      # clamps to the last item, as the reference's clamp(max=A-1)
    tokens = scheme.decode_unmasked(logits, x, w, values.to(device))
    table = scheme._engine_for(w).table
    # The table: one plain GEMM, within a bf16 rounding step of the CPU product.
    ref_table = vo.build_table(scheme.auxiliary_vocabulary.cpu(), w.cpu())
    close = (table.cpu().float() - ref_table.float()).abs() <= ref_table.float().abs() * 2 ** -7 + 1e-6
    assert close.float().mean() > 0.999
    st = vo.assign(_np(table), _np(logits), "bf16", full_sigma=False)
    dec, margin = vo.decode_item(_np(table), st["tokens"], st["bias"], np.minimum(values.numpy(), A - 1))
    margin = margin / st["unit"]
    got = tokens.cpu().numpy()
    print(f"decode: {int((got != dec).sum())} of {n} differ, margins {np.round(margin, 4).tolist()}", flush=True)
    assert np.all((got == dec) | (margin < TIE_TOL))
    # the same engine called again (cached table) is reproducible
    assert torch.equal(scheme.decode_unmasked(logits, x, w, values.to(device)), tokens)


def test_verify_writes_the_verify_rows_logits(device):
    g = torch.Generator().manual_seed(60)
    k, V, K = 7, 50257, 2048
    W = k + k * k
    x = torch.randn(W, K, generator=g).to(torch.bfloat16).to(device)
    w = (torch.randn(V, K, generator=g) * 0.02).to(torch.bfloat16).to(device)
    pending = torch.randint(0, V, (W,), generator=g).to(device)
    logits = torch.full((k, (V + 7) // 8 * 8), float("nan"), dtype=torch.bfloat16, device=device)
    acc, am = lm_head_verify_logits(x, w, pending, k - 1, 0.94, logits, k)
    ref = hip_linear(x, w, LOGITS_CONFIG)
    assert torch.equal(logits[:, :V], ref[:k])
    ref_acc, ref_am = lm_head_verify(x, w, pending, 0.94, "bf16")
    assert torch.equal(am, ref_am)
    assert torch.equal(acc[: k - 1], ref_acc[: k - 1]) and not acc[k - 1:].any()


def test_aux_round_matches_the_oracle(device):
    import oracle

    g = torch.Generator().manual_seed(70)
    k, A, H, V = 7, 4096, 2048, 50257
    W = k + k * k
    scheme = LogitVoronoiAuxiliary(A, H, V, dtype=torch.bfloat16).to(device)
    scheme.auxiliary_vocabulary.copy_((torch.randn(A, H, generator=g) * 0.02).to(torch.bfloat16))
    w = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16).to(device)
    x = torch.randn(W, H, generator=g).to(torch.bfloat16).to(device)
    logits = hip_linear(x, w, LOGITS_CONFIG).cpu()
    pending = logits[: k - 1].float().argmax(-1)          # accepted proposals (the row maxima)...
    pending[3] = logits[3].float().argmin()                 # ...up to row 3, whose proposal is the least likely
    values = torch.randint(0, A, (k,), generator=g)
    rv = AuxRoundVerify(k, scheme, V, "nucleus", 0.05, device=device)
    state = {"pending": pending.to(device), "anchor": torch.zeros(1, dtype=torch.int64, device=device),
             "out": torch.full((64,), -1, dtype=torch.int64, device=device),
             "base_t": torch.zeros((), dtype=torch.int64, device=device),
             "offset_t": torch.zeros((), dtype=torch.int64, device=device),
             "round_sequence": torch.zeros(8, dtype=torch.int64, device=device),
             "sequence_step": torch.zeros(1, dtype=torch.int64, device=device)}
    cpu = {name: t.cpu().clone() for name, t in state.items()}
    verify_tokens = rv(x, w, values.to(device), state["pending"], state["anchor"], state["out"], state["base_t"],
                       state["offset_t"], state["round_sequence"], state["sequence_step"]).cpu()
    torch.cuda.synchronize()
    table = _np(scheme._engine_for(w).table)
    st = vo.assign(table, logits[:k].float().numpy(), "bf16", full_sigma=False)
    dec, margin = vo.decode_item(table, st["tokens"], st["bias"], values.numpy())
    near = margin / st["unit"] < TIE_TOL
    assert np.all((verify_tokens.numpy() == dec) | near)
    widened = oracle.nucleus_acceptance(logits[: k - 1].float(), pending, 0.05)
    hyp = logits[k:].float().argmax(-1)
    ref = oracle.epilogue_state(widened, hyp, verify_tokens, cpu["pending"], cpu["anchor"], cpu["out"],
                                cpu["base_t"], cpu["offset_t"], cpu["round_sequence"], cpu["sequence_step"], k, 8)
    for name in ("pending", "anchor", "out", "base_t", "offset_t", "round_sequence", "sequence_step"):
        assert torch.equal(state[name].cpu(), ref[name]), name
    assert ref["num_correct"] == 3


def test_decode_graph_replays_with_new_inputs(device):
    table, _ = _case(80, 7, 50257, 4096)
    eng = Voronoi.from_table(table.to(device))
    logits = torch.empty(7, 50257, dtype=torch.bfloat16, device=device)
    values = torch.zeros(7, dtype=torch.int64, device=device)
    out = torch.zeros(7, dtype=torch.int64, device=device)
    logits.copy_(_case(81, 7, 50257, 4096)[1])
    eng.decode(logits, values, out)          # eager call sizes the workspace
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(graph):
        eng.decode(logits, values, out)
    torch.cuda.current_stream().wait_stream(stream)
    g = torch.Generator().manual_seed(82)
    for replay in range(5):
        new = _case(83 + replay, 7, 50257, 4096)[1]
        vals = torch.randint(0, 4096, (7,), generator=g)
        logits.copy_(new)
        values.copy_(vals)
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        eager = eng.decode(new.to(device), vals.to(device))
        assert torch.equal(out, eager), replay
