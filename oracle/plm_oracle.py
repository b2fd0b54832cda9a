"""CPU restatement of the reference's round linears and verify epilogue. TEST INFRASTRUCTURE ONLY
(imported by tests/, __graft_entry__.smoke() and bench.py's CPU baseline; never by the product).

The GEMM oracle is the reference's own ``--mode default`` path: torch ``F.linear`` on the same
half-precision operands (plm/fast_gemm.py:111), here on the CPU. The epilogue functions restate
plm/decoder.py:71-82 and 351-362 with torch CPU ops; the ``*_fp64`` helpers are independent
brute-force versions used to pin them.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


# --------------------------------------------------------------------------- GEMM

def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``x[M,K] @ w[N,K]^T`` in x's dtype via CPU ``F.linear`` (plm/fast_gemm.py:111; layout 3)."""
    return F.linear(x.cpu(), w.cpu())


def linear_fp32(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """fp32 product of the half-precision operands, without rounding the result (the accumulator the
    reference's GEMM holds before its cast, plm/fast_gemm.py:35-46)."""
    return x.cpu().float() @ w.cpu().float().T


def linear_fp64(x: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """Exact-as-possible fp64 brute force (numpy), the pin for the two functions above."""
    xa = x.cpu().float().numpy().astype(np.float64)
    wa = w.cpu().float().numpy().astype(np.float64)
    return xa @ wa.T


# --------------------------------------------------------------------------- gated LoRA

def gated_lora(x: torch.Tensor, w: torch.Tensor, lora_a: torch.Tensor, lora_bs: list[torch.Tensor],
               first_gated_row: int | None) -> torch.Tensor:
    """``GatedLoraMethod.apply`` (plm/gated_lora.py:45-57) on CPU copies in the operands' dtype: the base
    linear over every row; rows from ``first_gated_row`` add ``(x A^T) B_s^T`` into each shard's own
    output columns (one ``addmm_`` per shard, the hidden product already in the model dtype)."""
    output = linear(x, w)
    if first_gated_row is None or first_gated_row >= x.shape[0]:
        return output
    hidden = linear(x[first_gated_row:], lora_a)
    rank = hidden.shape[1] // len(lora_bs)
    gated = output[first_gated_row:]
    col = 0
    for shard, b in enumerate(lora_bs):
        b = b.cpu()
        gated[:, col:col + b.shape[0]].addmm_(hidden[:, shard * rank:(shard + 1) * rank], b.t())
        col += b.shape[0]
    return output


def silu_mul(y: torch.Tensor) -> torch.Tensor:
    """The Llama-style MLP's activation on a fused gate/up projection's output ``y[..., 2I]``.

    The rounds run the model through vLLM 0.26.0 (uv.lock:3123-3125) with ``enforce_eager=True``
    (plm/decoder.py:37), so its ``SiluAndMul`` runs the ``silu_and_mul`` custom kernel: per element,
    ``silu(g) = g / (1 + e^-g)`` computed in fp32 from the model-dtype gate ``g = y[..., :I]`` and
    rounded to the model dtype, then multiplied by ``u = y[..., I:]`` in the model dtype (exact in
    fp32, rounded once). Eager torch's ``F.silu(g) * u`` on model-dtype tensors rounds the same two
    times, which is what this computes (on the CPU)."""
    half = y.shape[-1] // 2
    g, u = y[..., :half].cpu(), y[..., half:].cpu()
    return (F.silu(g.float()).to(y.dtype).float() * u.float()).to(y.dtype)


def silu_mul_fp64(y: torch.Tensor) -> np.ndarray:
    """Independent numpy version of ``silu_mul``: ``g / (1 + e^-g)`` in fp64 rounded to the model
    dtype, times ``u`` in fp64, rounded to the model dtype (the pin for ``silu_mul``: the two agree
    except where the fp32 and fp64 silu round to neighbouring values)."""
    half = y.shape[-1] // 2
    yd = y.cpu().double().numpy()
    g, u = yd[..., :half], yd[..., half:]
    s = torch.from_numpy(g / (1.0 + np.exp(-g))).to(y.dtype).double().numpy()
    return torch.from_numpy(s * u).to(y.dtype).double().numpy()


def gated_lora_fp64(x: torch.Tensor, w: torch.Tensor, lora_a: torch.Tensor, lora_bs: list[torch.Tensor],
                    first_gated_row: int) -> np.ndarray:
    """Independent numpy version: the base and hidden products exact in fp64 and rounded to the model
    dtype, the correction added in fp64 and rounded once."""
    dt = x.dtype
    rnd = lambda a: torch.from_numpy(a).to(dt).double().numpy()
    xd, wd, ad = (t.cpu().double().numpy() for t in (x, w, lora_a))
    out = rnd(xd @ wd.T)
    g = first_gated_row
    if g >= xd.shape[0]:
        return out
    h = rnd(xd[g:] @ ad.T)
    rank = h.shape[1] // len(lora_bs)
    b_cat = np.concatenate([b.cpu().double().numpy() for b in lora_bs], axis=0)
    shard = np.repeat(np.arange(len(lora_bs)), [b.shape[0] for b in lora_bs])
    corr = np.stack([h[:, s * rank:(s + 1) * rank] @ b_cat[n] for n, s in enumerate(shard)], axis=1)
    out[g:] = rnd(out[g:] + corr)
    return out


# --------------------------------------------------------------------------- verify epilogue

def nucleus_acceptance(logits: torch.Tensor, pending: torch.Tensor, nucleus: float) -> torch.Tensor:
    """Proposal inside the top-``nucleus`` mass (plm/decoder.py:71-75): the probability mass strictly
    above the proposal's own probability is below ``nucleus``, or the proposal is the row maximum
    and ``nucleus > 0``. ``nucleus <= 0`` accepts nothing."""
    probs = torch.softmax(logits.cpu().float(), dim=-1)
    own = probs.gather(1, pending.cpu()[:, None]).squeeze(1)
    above = (probs * (probs > own[:, None])).sum(-1)
    return (above < nucleus) | ((own >= probs.amax(-1)) & (nucleus > 0))


def floor_acceptance(logits: torch.Tensor, pending: torch.Tensor, epsilon: float) -> torch.Tensor:
    """Proposal probability above ``epsilon``, in the log domain (plm/decoder.py:78-82)."""
    scores = logits.cpu().float()
    own_logit = scores.gather(1, pending.cpu()[:, None]).squeeze(1)
    return own_logit - torch.logsumexp(scores, dim=-1) > torch.log(torch.tensor(float(epsilon)))


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """Row argmax with the lowest index among equal maxima (``logits.argmax(-1)``, plm/decoder.py:362)."""
    return logits.cpu().float().argmax(dim=-1)


def verify(logits: torch.Tensor, pending: torch.Tensor, nucleus: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The fused verify step's two outputs for every row: nucleus decision and argmax."""
    return nucleus_acceptance(logits, pending, nucleus), argmax(logits)


def nucleus_margin(logits: torch.Tensor, pending: torch.Tensor, nucleus: float) -> np.ndarray:
    """fp64 distance between each row's mass-above-own and ``nucleus`` (how far a decision is from
    flipping under rounding); +inf where the proposal is the row maximum."""
    z = logits.cpu().double().numpy()
    z = z - z.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    idx = pending.cpu().numpy()
    own = p[np.arange(len(idx)), idx]
    above = np.where(p > own[:, None], p, 0.0).sum(axis=1)
    margin = np.abs(above - nucleus)
    margin[own >= p.max(axis=1)] = np.inf
    return margin


def nucleus_acceptance_fp64(logits: torch.Tensor, pending: torch.Tensor, nucleus: float) -> np.ndarray:
    """Sort-based fp64 brute force of the nucleus rule: walk each row's probabilities in descending
    order and sum everything strictly more probable than the proposal."""
    z = logits.cpu().double().numpy()
    out = np.zeros(z.shape[0], dtype=bool)
    for r in range(z.shape[0]):
        row = np.exp(z[r] - z[r].max())
        row /= row.sum()
        own = row[int(pending[r])]
        order = np.sort(row)[::-1]
        mass = 0.0
        for v in order:
            if v <= own:
                break
            mass += v
        out[r] = (mass < nucleus) or (own >= order[0] and nucleus > 0)
    return out


def floor_acceptance_fp64(logits: torch.Tensor, pending: torch.Tensor, epsilon: float) -> np.ndarray:
    z = logits.cpu().double().numpy()
    m = z.max(axis=1)
    lse = m + np.log(np.exp(z - m[:, None]).sum(axis=1))
    own = z[np.arange(z.shape[0]), pending.cpu().numpy()]
    return own - lse > np.log(epsilon)


def argmax_fp64(logits: torch.Tensor) -> np.ndarray:
    z = logits.cpu().double().numpy()
    out = np.empty(z.shape[0], dtype=np.int64)
    for r in range(z.shape[0]):
        best = 0
        for j in range(1, z.shape[1]):
            if z[r, j] > z[r, best]:
                best = j
        out[r] = best
    return out


# --------------------------------------------------------------------------- the round epilogue

def epilogue_state(widened: torch.Tensor, hypotheses: torch.Tensor, verify_tokens: torch.Tensor,
                   pending: torch.Tensor, anchor: torch.Tensor, out: torch.Tensor, base_t: torch.Tensor,
                   offset_t: torch.Tensor, round_sequence: torch.Tensor, sequence_step: torch.Tensor,
                   k: int, sequence_capacity: int) -> dict:
    """``RoundDecoder._epilogue`` (plm/decoder.py:351-365) from the rule's decisions, state writes
    included, on CPU copies: ``widened[k-1]`` is the rule over verify rows 0..k-2, ``hypotheses[k*k]``
    the argmax of the proposal rows. Returns the updated state and ``accepted``/``num_correct``."""
    pending, anchor, out = pending.cpu().clone(), anchor.cpu().clone(), out.cpu().clone()
    base_t, offset_t = base_t.cpu().clone(), offset_t.cpu().clone()
    round_sequence, sequence_step = round_sequence.cpu().clone(), sequence_step.cpu().clone()
    verify_tokens, hypotheses = verify_tokens.cpu(), hypotheses.cpu()
    kidx = torch.arange(k)
    accepted = (verify_tokens[:-1] == pending) | widened.cpu().bool()
    num_correct = accepted.to(torch.int64).cumprod(0).sum()
    confirmed_head = torch.cat([pending, verify_tokens[-1:]])
    picked = verify_tokens.index_select(0, num_correct.clamp(max=k - 1).view(1))
    slots = base_t + kidx
    out[slots] = torch.where(kidx < num_correct, confirmed_head,
                             torch.where(kidx == num_correct, picked.expand(k), out[slots]))
    round_sequence.index_copy_(0, sequence_step.clamp(max=sequence_capacity - 1), num_correct.view(1))
    sequence_step.add_(1)
    pending.copy_(hypotheses.view(k, k).index_select(0, num_correct.view(1))[0][1:k])
    anchor.copy_(picked)
    base_t.add_(num_correct + 1)
    offset_t.add_(num_correct + 1)
    return {"accepted": accepted, "num_correct": int(num_correct), "pending": pending, "anchor": anchor,
            "out": out, "base_t": base_t, "offset_t": offset_t, "round_sequence": round_sequence,
            "sequence_step": sequence_step}


def epilogue(logits: torch.Tensor, verify_tokens: torch.Tensor, pending: torch.Tensor, k: int, rule: str,
             threshold: float) -> dict:
    """One round's bookkeeping after the LM head (plm/decoder.py:351-365) from the round's logits.

    ``logits`` is ``[k + k*k, V]`` (verify rows first, then ``k`` proposal blocks of ``k``),
    ``verify_tokens[k]`` the verify rows' own decodes, ``pending[k-1]`` last round's proposals.
    Returns ``accepted[k-1]``, ``num_correct``, the ``num_correct + 1`` committed tokens (the slots
    the round writes, from a fresh state at position 0) and the next round's ``pending[k-1]``."""
    widened = floor_acceptance if rule == "floor" else nucleus_acceptance
    decisions = widened(logits[: k - 1], pending, threshold)
    state = epilogue_state(decisions, argmax(logits[k:]), verify_tokens, pending,
                           torch.zeros(1, dtype=torch.int64), torch.full((k,), -1, dtype=torch.int64),
                           torch.zeros((), dtype=torch.int64), torch.zeros((), dtype=torch.int64),
                           torch.zeros(1, dtype=torch.int64), torch.zeros(1, dtype=torch.int64), k, 1)
    n = state["num_correct"]
    return {"accepted": state["accepted"], "num_correct": n, "committed": state["out"][: n + 1],
            "next_pending": state["pending"]}
