"""GPU parity of the verify step's floor rule and of the round epilogue on the device.

* ``floor`` rule (floor_acceptance, plm/decoder.py:78-82): the kernel's accept bits equal the oracle's
  on the kernel's own logits on every row whose fp64 distance from the boundary exceeds 1e-4 (the
  kernel sums exp in its own order, so logsumexp may differ from torch's by a few fp32 ulps).
* ``round_epilogue`` (plm/decoder.py:351-365): every state tensor equals the oracle's restatement
  (``epilogue_state``) bit for bit, over hand-built and random rounds.
* ``RoundVerify``: the fused verify + epilogue over a 1.3B-shape round (k = 7, 56 rows, vocabulary
  50257) equals the oracle's ``epilogue`` on the same logits, eagerly and under graph replay."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import plm_oracle as po
from plm_amd import workloads
from plm_amd.fast_gemm import hip_linear_f32
from plm_amd.verify import LOGITS_CONFIG, ROWMAJOR_LOGITS_CONFIG, RoundVerify, lm_head_verify, round_epilogue

pytestmark = pytest.mark.gpu


def _rounded(logits: torch.Tensor, mode: str) -> torch.Tensor:
    if mode == "bf16":
        return logits.bfloat16().float()
    if mode == "fp16":
        return logits.half().float()
    return logits


def _floor_margin(logits: torch.Tensor, pending: torch.Tensor, eps: float) -> np.ndarray:
    """fp64 distance of ``l_own - logsumexp(l)`` from ``log(eps)``."""
    z = logits.double().numpy()
    m = z.max(axis=1)
    lse = m + np.log(np.exp(z - m[:, None]).sum(axis=1))
    own = z[np.arange(z.shape[0]), pending.numpy()]
    return np.abs(own - lse - np.log(eps)) if eps > 0 else np.full(z.shape[0], np.inf)


def _ranked_proposals(logits: torch.Tensor, stride: int = 37, span: int = 2000) -> torch.Tensor:
    """Row r proposes the id at rank (r * stride) % span of its own logits: a spread of probabilities."""
    order = logits.argsort(dim=-1, descending=True, stable=True)
    ranks = (torch.arange(logits.shape[0]) * stride) % span
    return order[torch.arange(logits.shape[0]), ranks]


def _config5(device, R=56, V=workloads.GPT2_VOCAB, K=2048, dtype=torch.bfloat16, seed=5000):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(R, K, generator=g, device=device).to(dtype)
    w = (0.02 * torch.randn(V, K, generator=g, device=device)).to(dtype)
    return x, w


# --------------------------------------------------------------------------- floor rule


@pytest.mark.parametrize("packed", [True, False], ids=["packed", "rowmajor"])
@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("eps", [1e-4, 2e-3, 1e-5])
def test_floor_rule(device, eps, mode, packed):
    x, w = _config5(device)
    logits = _rounded(hip_linear_f32(x, w, LOGITS_CONFIG if packed else ROWMAJOR_LOGITS_CONFIG).cpu(), mode)
    pending = _ranked_proposals(logits)
    acc, am = lm_head_verify(x, w, pending.to(device), eps, mode, packed=packed, rule="floor")
    acc, am = acc.cpu(), am.cpu()
    ref = oracle.floor_acceptance(logits, pending, eps)
    safe = torch.from_numpy(_floor_margin(logits, pending, eps) > 1e-4)
    assert int(safe.sum()) >= 50
    assert torch.equal(acc[safe], ref[safe]), (acc != ref).nonzero()
    assert torch.equal(am, oracle.argmax(logits))
    if eps == 1e-4:
        assert 0 < int(acc.sum()) < 56     # the ranked proposals straddle the floor
    # Against the fp64 oracle on CPU-computed logits, away from the boundary.
    cpu = _rounded(oracle.linear_fp32(x.cpu(), w.cpu()), mode)
    ref64 = torch.from_numpy(po.floor_acceptance_fp64(cpu, pending, eps))
    safe64 = torch.from_numpy(_floor_margin(cpu, pending, eps) > 1e-3)
    assert torch.equal(acc[safe64], ref64[safe64])


def test_floor_rule_special_thresholds(device):
    """eps = 0 accepts every vocabulary id (log 0 = -inf); eps < 0 accepts none (log is NaN); eps = 1
    accepts none (a probability is below 1); an id outside the vocabulary is never accepted."""
    x, w = _config5(device, R=16, V=7000)
    pending = torch.randint(0, 7000, (16,), generator=torch.Generator().manual_seed(3))
    pending[3] = -1
    pending[9] = 7000
    valid = torch.ones(16, dtype=torch.bool)
    valid[3] = valid[9] = False
    for eps, expect in ((0.0, valid), (-0.5, torch.zeros(16, dtype=torch.bool)),
                        (1.0, torch.zeros(16, dtype=torch.bool))):
        for packed in (True, False):
            acc, _ = lm_head_verify(x, w, pending.to(device), eps, packed=packed, rule="floor")
            assert torch.equal(acc.cpu(), expect), (eps, packed)


def test_floor_rule_uniform_rows(device):
    """All logits equal: every proposal has probability exactly 1/V, accepted iff 1/V > eps."""
    R, V, K = 8, 1000, 256
    x = torch.randn(R, K, device=device).bfloat16()
    w = torch.zeros(V, K, device=device).bfloat16()
    pending = torch.arange(R, device=device) * 100
    for eps, expect in ((0.9e-3, True), (1.1e-3, False)):
        acc, _ = lm_head_verify(x, w, pending, eps, rule="floor")
        assert bool((acc == expect).all()), eps


# --------------------------------------------------------------------------- round epilogue


def _state(k: int, out_len: int, base: int, seed: int, device, seq_len: int = 8, step: int = 0):
    g = torch.Generator().manual_seed(seed)
    pending = torch.randint(0, 50, (k - 1,), generator=g)
    verify = torch.randint(0, 50, (k,), generator=g)
    hyp = torch.randint(0, 50257, (k * k,), generator=g)
    cpu = {"pending": pending, "anchor": torch.tensor([7]), "out": torch.full((out_len,), -1, dtype=torch.int64),
           "base_t": torch.tensor(base), "offset_t": torch.tensor(base + 100),
           "round_sequence": torch.zeros(seq_len, dtype=torch.int64), "sequence_step": torch.tensor([step])}
    cpu["out"][::3] = 5
    gpu = {name: t.clone().to(device) for name, t in cpu.items()}
    return cpu, gpu, verify, hyp


def _run_epilogue(k, widened, hyp, verify, cpu, gpu, device, seq_len=8):
    ref = oracle.epilogue_state(widened, hyp, verify, cpu["pending"], cpu["anchor"], cpu["out"], cpu["base_t"],
                                cpu["offset_t"], cpu["round_sequence"], cpu["sequence_step"], k, seq_len)
    accepted = torch.zeros(max(k - 1, 1), dtype=torch.bool, device=device)
    nc = torch.full((), -1, dtype=torch.int64, device=device)
    round_epilogue(k, widened.to(device), hyp.to(device), verify.to(device), gpu["pending"], gpu["anchor"],
                   gpu["out"], gpu["base_t"], gpu["offset_t"], gpu["round_sequence"], gpu["sequence_step"],
                   accepted, nc)
    torch.cuda.synchronize()
    for name in ("pending", "anchor", "out", "base_t", "offset_t", "round_sequence", "sequence_step"):
        assert torch.equal(gpu[name].cpu(), ref[name]), (name, gpu[name].cpu(), ref[name])
    assert int(nc) == ref["num_correct"]
    assert torch.equal(accepted[: k - 1].cpu(), ref["accepted"])
    return ref


@pytest.mark.parametrize("k", [1, 2, 3, 7, 10, 64])
def test_epilogue_every_run_length(device, k):
    """Every num_correct from 0 to k-1, reached through the rule's bits and through equality."""
    for stop in range(k):
        for by_equality in (False, True):
            cpu, gpu, verify, hyp = _state(k, 4 * k + 16, 3, seed=100 * k + stop, device=device)
            widened = torch.zeros(k - 1, dtype=torch.bool)
            if by_equality:
                verify[: k - 1] = cpu["pending"] + 1          # no equality by default
                verify[:stop] = cpu["pending"][:stop]
            else:
                verify[: k - 1] = cpu["pending"] + 1
                widened[:stop] = True
            if stop < k - 1:                                  # later proposals accepted: must not count
                widened[stop + 1:] = True
            ref = _run_epilogue(k, widened, hyp, verify, cpu, gpu, device)
            assert ref["num_correct"] == stop


def test_epilogue_random_rounds(device):
    for seed in range(40):
        k = 1 + seed % 12
        cpu, gpu, verify, hyp = _state(k, 200, seed % 50, seed, device, step=seed % 11)
        g = torch.Generator().manual_seed(seed)
        widened = torch.rand(k - 1, generator=g) < 0.7
        eq = torch.rand(k - 1, generator=g) < 0.3
        verify[: k - 1] = torch.where(eq, cpu["pending"], verify[: k - 1])
        _run_epilogue(k, widened, hyp, verify, cpu, gpu, device)


def test_epilogue_slots_past_the_buffer_are_not_written(device):
    """A round whose slots run past ``out``: the slots inside are written, the rest dropped."""
    k = 7
    cpu, gpu, verify, hyp = _state(k, 10, 6, seed=1, device=device)
    widened = torch.ones(k - 1, dtype=torch.bool)
    accepted = torch.zeros(k - 1, dtype=torch.bool, device=device)
    round_epilogue(k, widened.to(device), hyp.to(device), verify.to(device), gpu["pending"], gpu["anchor"],
                   gpu["out"], gpu["base_t"], gpu["offset_t"], accepted=accepted)
    out = gpu["out"].cpu()
    expect = cpu["out"].clone()
    expect[6:10] = cpu["pending"][:4]
    assert torch.equal(out, expect)
    assert int(gpu["base_t"]) == 6 + k and bool(accepted.all())


def test_epilogue_sequence_capacity_clamps(device):
    k = 4
    cpu, gpu, verify, hyp = _state(k, 64, 0, seed=2, device=device, seq_len=3, step=9)
    _run_epilogue(k, torch.tensor([True, True, False]), hyp, verify, cpu, gpu, device, seq_len=3)


# --------------------------------------------------------------------------- the round's LM-head end


def _round_inputs(device, k=7, V=workloads.GPT2_VOCAB, K=2048):
    """A round whose third proposal sits at rank 1000 of its verify row (probability ~1e-4, with about
    0.12 of the mass above it) and every other proposal at rank 0; the first two verify tokens equal
    their proposals."""
    W = k + k * k
    x, w = _config5(device, R=W, V=V, K=K)
    logits = hip_linear_f32(x, w, LOGITS_CONFIG).cpu()
    order = logits[: k - 1].argsort(dim=-1, descending=True, stable=True)
    ranks = torch.zeros(k - 1, dtype=torch.int64)
    ranks[2] = 1000
    pending = order[torch.arange(k - 1), ranks]
    verify = torch.randint(0, V, (k,), generator=torch.Generator().manual_seed(11))
    verify[:2] = pending[:2]
    return x, w, logits, pending, verify


@pytest.mark.parametrize("rule,threshold,mode,accepted_bits", [
    ("nucleus", workloads.TOP_P, "fp32", [1, 1, 1, 1, 1, 1]),   # ~0.12 above the rank-1000 proposal
    ("nucleus", 0.05, "bf16", [1, 1, 0, 1, 1, 1]),
    ("nucleus", -1.0, "bf16", [1, 1, 0, 0, 0, 0]),              # exact matching: equality only
    ("floor", 2e-4, "bf16", [1, 1, 0, 1, 1, 1]),
    ("floor", 2e-4, "fp32", [1, 1, 0, 1, 1, 1])])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "separate"])
def test_round_verify_matches_the_oracle(device, rule, threshold, mode, accepted_bits, fused):
    k = 7
    x, w, logits, pending, verify = _round_inputs(device, k)
    logits = _rounded(logits, mode)
    if rule == "floor":
        assert (_floor_margin(logits[: k - 1], pending, threshold) > 1e-4).all()
    ref = oracle.epilogue(logits, verify, pending, k, rule, threshold)
    assert ref["accepted"].tolist() == [bool(b) for b in accepted_bits]
    rv = RoundVerify(k, rule, threshold, mode, device, fused=fused)
    assert rv.fused == fused
    state = {"pending": pending.to(device), "anchor": torch.zeros(1, dtype=torch.int64, device=device),
             "out": torch.full((32,), -1, dtype=torch.int64, device=device),
             "base_t": torch.zeros((), dtype=torch.int64, device=device),
             "offset_t": torch.zeros((), dtype=torch.int64, device=device)}
    accepted = torch.zeros(k - 1, dtype=torch.bool, device=device)
    nc = torch.zeros((), dtype=torch.int64, device=device)
    rv(x, w, verify.to(device), state["pending"], state["anchor"], state["out"], state["base_t"], state["offset_t"],
       accepted=accepted, num_correct=nc)
    torch.cuda.synchronize()
    n = ref["num_correct"]
    assert int(nc) == n and torch.equal(accepted.cpu(), ref["accepted"])
    assert torch.equal(state["out"].cpu()[: n + 1], ref["committed"])
    assert torch.equal(state["pending"].cpu(), ref["next_pending"])
    assert int(state["base_t"]) == n + 1 and int(state["anchor"][0]) == int(ref["committed"][-1])


def test_round_verify_graph_replays(device):
    """Captured once, replayed three rounds: each replay advances the state exactly as the oracle's
    round does from the state the previous replay left."""
    k = 7
    x, w, logits, pending, verify = _round_inputs(device, k)
    rv = RoundVerify(k, "nucleus", 0.8, "fp32", device)
    g = {"pending": pending.to(device), "anchor": torch.zeros(1, dtype=torch.int64, device=device),
         "out": torch.full((64,), -1, dtype=torch.int64, device=device),
         "base_t": torch.zeros((), dtype=torch.int64, device=device),
         "offset_t": torch.zeros((), dtype=torch.int64, device=device),
         "round_sequence": torch.zeros(16, dtype=torch.int64, device=device),
         "sequence_step": torch.zeros(1, dtype=torch.int64, device=device)}
    vt = verify.to(device)
    args = (x, w, vt, g["pending"], g["anchor"], g["out"], g["base_t"], g["offset_t"], g["round_sequence"],
            g["sequence_step"])
    rv(*args)                                   # eager warm-up (workspace, packed copy)
    torch.cuda.synchronize()
    snapshot = {n: t.clone() for n, t in g.items()}
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        rv(*args)
    for n, t in g.items():                      # capture does not run the work: restore anyway
        t.copy_(snapshot[n])
    cpu = {n: t.cpu() for n, t in snapshot.items()}
    hyp = oracle.argmax(logits[k:])
    for _ in range(3):
        widened = oracle.nucleus_acceptance(logits[: k - 1], cpu["pending"].clamp(0, logits.shape[1] - 1), 0.8)
        ref = oracle.epilogue_state(widened, hyp, verify, cpu["pending"], cpu["anchor"], cpu["out"], cpu["base_t"],
                                    cpu["offset_t"], cpu["round_sequence"], cpu["sequence_step"], k, 16)
        graph.replay()
        torch.cuda.synchronize()
        for n in g:
            assert torch.equal(g[n].cpu(), ref[n]), n
        cpu = {n: ref[n] for n in g}
        rv(x, w, vt, g["pending"].clone(), g["anchor"].clone(), g["out"].clone(), g["base_t"].clone(),
           g["offset_t"].clone())                # eager work between replays, on scratch copies
        torch.cuda.synchronize()


@pytest.mark.parametrize("k", [1, 2, 3, 5, 7])
@pytest.mark.parametrize("rule,threshold", [("nucleus", 0.3), ("floor", 1e-4)])
def test_fused_round_verify_equals_verify_then_epilogue(device, k, rule, threshold):
    """plm_round_verify_packed (epilogue in the verify's last workgroup) against lm_head_verify over
    the round's rows followed by plm_round_epilogue: every state tensor and every row's decision and
    argmax, bit for bit, over several rounds of random decoder states."""
    W = k + k * k
    x, w = _config5(device, R=W, V=20011, K=1024, seed=700 + k)
    logits = hip_linear_f32(x, w, LOGITS_CONFIG).cpu()
    g = torch.Generator().manual_seed(800 + k)
    for rnd in range(4):
        order = logits[: max(k - 1, 1)].argsort(dim=-1, descending=True, stable=True)
        ranks = torch.randint(0, 400, (k - 1,), generator=g)
        pending = order[torch.arange(k - 1), ranks] if k > 1 else torch.zeros(0, dtype=torch.int64)
        verify = torch.randint(0, 20011, (k,), generator=g)
        eq = torch.rand(k - 1, generator=g) < 0.3
        verify[: k - 1] = torch.where(eq, pending, verify[: k - 1])
        base = int(torch.randint(0, 40, (1,), generator=g))
        runs = {}
        for fused in (True, False):
            st = {"pending": pending.clone().to(device), "anchor": torch.zeros(1, dtype=torch.int64, device=device),
                  "out": torch.full((64,), -1, dtype=torch.int64, device=device),
                  "base_t": torch.tensor(base, device=device), "offset_t": torch.tensor(base + 9, device=device),
                  "round_sequence": torch.zeros(3, dtype=torch.int64, device=device),
                  "sequence_step": torch.tensor([rnd], device=device)}
            acc = torch.zeros(max(k - 1, 1), dtype=torch.bool, device=device)
            nc = torch.full((), -1, dtype=torch.int64, device=device)
            rv = RoundVerify(k, rule, threshold, "bf16", device, fused=fused)
            rv(x, w, verify.to(device), st["pending"], st["anchor"], st["out"], st["base_t"], st["offset_t"],
               st["round_sequence"], st["sequence_step"], acc, nc)
            torch.cuda.synchronize()
            runs[fused] = ({n: t.cpu() for n, t in st.items()}, acc.cpu(), int(nc), rv.accept.cpu(), rv.argmax.cpu())
        (s1, a1, n1, acc1, am1), (s2, a2, n2, acc2, am2) = runs[True], runs[False]
        for name in s1:
            assert torch.equal(s1[name], s2[name]), (rnd, name, s1[name], s2[name])
        assert n1 == n2 and torch.equal(a1[: k - 1], a2[: k - 1])
        assert torch.equal(am1, am2)
        assert torch.equal(acc1[: k - 1], acc2[: k - 1])   # rows past k-2 propose nothing in either path
