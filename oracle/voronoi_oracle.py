"""CPU restatement of the verify row's auxiliary decode (the logit-Voronoi ``iterate`` engine).
TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU baseline.

Follows plm/iterate.py and plm/auxiliary.py:56-75 step by step, in numpy float32 where the reference
computes in float32, so that every intermediate has the reference's dtype:

* ``scan_logits``  — iterate.py:54-80, 176-192: per-tile maxima and the softmax normaliser.
* ``shortlist``    — iterate.py:248-273: the ``n_targets`` largest logits and their quotas.
* ``quota``        — iterate.py:214-223: largest-remainder apportionment.
* ``spread``       — iterate.py:275-284: the cost unit.
* ``prior``        — iterate.py:286-290: the factor before any geometry.
* ``condense``     — iterate.py:83-107, 195-211: each item's ``k`` cheapest candidates, packed keys.
* ``fit``          — iterate.py:110-159, 292-312: the annealed Sinkhorn sweeps.
* ``argmin``       — iterate.py:314-320, 345-346.
* ``assign``       — iterate.py:322-342.
* ``decode_unmasked`` — auxiliary.py:67-75.
* ``build_table``  — auxiliary.py:56-65 (the ``(V, A)`` cost table from the auxiliary vocabulary).

Where the reference leaves a choice to a library, the oracle fixes it (and the HIP path makes the
same choice):

* Ties. ``torch.topk`` and the unstable ``argsort`` in ``quota`` leave the order of equal values
  open. Here the shortlist is the ``n_targets`` largest logits by (value descending, token id
  ascending) and equal remainders in ``quota`` rank by shortlist position.
* Sums. The reference's normaliser is an online fp32 scan, ``spread``'s mean and ``quota``'s
  renormalising sum are torch reductions, and the fit's per-token loads are fp32 ``atomic_add``s
  in arrival order (iterate.py:8-9, 146): none has a fixed summation order. The oracle sums in
  float64 and rounds once to float32, the value every order approximates.

Pinning (tests/test_voronoi_oracle.py): ``shortlist`` against a full-vocabulary sort and the
reference's tile route; ``quota`` against a seat-by-seat Hamilton count and textbook cases;
``condense`` against a per-item sort and the key's bit layout; ``fit`` against an fp64
per-item loop restatement, a hand-computed first sweep, and, run to convergence, the optimal
transport assignment of ``scipy.optimize.linear_sum_assignment``; ``argmin`` against brute force;
``assign`` against its purpose (token shares follow the quotas). Planted mistakes in each fail.
"""

from __future__ import annotations

import numpy as np

# iterate.py:21-26
STEP_LIMIT = 0.25
LOAD_FLOOR = 1e-2
BLOCKED = 1e3
EMPTY = -1e30

f32 = np.float32


# --------------------------------------------------------------------------- bit helpers

def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def to_model_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to the model dtype ("bf16" or "f16"), as float32."""
    if dtype == "bf16":
        return bf16_round(np.asarray(x, dtype=np.float32))
    if dtype == "f16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


def pack_key(cost: np.ndarray, target: np.ndarray) -> np.ndarray:
    """iterate.py:102-103: float32 cost -> order-preserving int32 with the low 7 bits replaced by the
    target index."""
    bits = np.ascontiguousarray(cost, dtype=np.float32).view(np.int32)
    ordered = np.where(bits >= 0, bits, bits ^ np.int32(0x7FFFFFFF))
    return (ordered & np.int32(~0x7F)) | np.asarray(target, dtype=np.int32)


def unpack_key(key: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """iterate.py:132-134: packed key -> (target, carried cost as float32)."""
    key = np.asarray(key, dtype=np.int32)
    target = key & np.int32(0x7F)
    carried = key & np.int32(~0x7F)
    bits = np.where(carried >= 0, carried, carried ^ np.int32(0x7FFFFFFF)).astype(np.int32)
    return target, bits.view(np.float32)


# --------------------------------------------------------------------------- shortlist

def scan_logits(logits: np.ndarray, tile: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """iterate.py:176-192 (kernel 54-80): per-tile maxima (ragged tail padded with -inf, an all -inf
    tile reads -inf) and the normaliser ``max + log(sum exp(l - max))`` of each row."""
    logits = np.asarray(logits, dtype=np.float32)
    n, v = logits.shape
    tiles = -(-v // tile)
    padded = np.full((n, tiles * tile), -np.inf, dtype=np.float32)
    padded[:, :v] = logits
    tile_max = padded.reshape(n, tiles, tile).max(axis=2)
    l64 = np.maximum(logits.astype(np.float64), EMPTY)
    mx = l64.max(axis=1)
    normaliser = mx + np.log(np.exp(l64 - mx[:, None]).sum(axis=1))
    return tile_max, normaliser.astype(np.float32)


def top_targets(logits: np.ndarray, n_targets: int) -> tuple[np.ndarray, np.ndarray]:
    """The ``n_targets`` largest logits of each row by (value descending, token id ascending):
    (tokens int64, values float32), in that order."""
    logits = np.asarray(logits, dtype=np.float32)
    n, v = logits.shape
    tokens = np.empty((n, n_targets), dtype=np.int64)
    for r in range(n):
        order = np.lexsort((np.arange(v), -logits[r].astype(np.float64)))
        tokens[r] = order[:n_targets]
    return tokens, np.take_along_axis(logits, tokens, axis=1)


def quota(weights: np.ndarray, total: int) -> np.ndarray:
    """iterate.py:214-223: floor of ``weights * total`` plus one for the largest remainders, summing to
    ``total``; equal remainders rank by position."""
    exact = np.asarray(weights, dtype=np.float32) * f32(total)
    counts = np.floor(exact).astype(np.int64)
    remaining = total - counts.sum(axis=-1, keepdims=True)
    remainder = (exact - counts.astype(np.float32)).astype(np.float32)
    order = np.argsort(-remainder, axis=-1, kind="stable")
    rank = np.argsort(order, axis=-1, kind="stable")
    return counts + (rank < remaining).astype(np.int64)


def probabilities(values: np.ndarray, normaliser: np.ndarray) -> np.ndarray:
    """iterate.py:272-273: ``exp(value - normaliser)`` renormalised over the shortlist (float32)."""
    p = np.exp((np.asarray(values, dtype=np.float32) - normaliser[:, None].astype(np.float32)).astype(np.float32))
    p = p.astype(np.float32)
    total = p.astype(np.float64).sum(axis=-1, keepdims=True).astype(np.float32)
    return (p / total).astype(np.float32)


def shortlist(logits: np.ndarray, n_items: int, n_targets: int = 128, tile: int = 64):
    """iterate.py:248-273: (tokens int64, counts int64, values float32, normaliser float32)."""
    _, normaliser = scan_logits(logits, tile)
    tokens, values = top_targets(logits, n_targets)
    counts = quota(probabilities(values, normaliser), n_items)
    return tokens, counts, values, normaliser


def shortlist_tiled(logits: np.ndarray, n_targets: int = 128, tile: int = 64) -> np.ndarray:
    """The reference's own route (iterate.py:259-267): top tiles by tile maximum, then the top logits
    of their pool. Token sets agree with ``top_targets`` whenever the ``n_targets``-th value is not
    tied; used only to pin ``top_targets``."""
    logits = np.asarray(logits, dtype=np.float32)
    n, v = logits.shape
    tile_max, _ = scan_logits(logits, tile)
    tiles = tile_max.shape[1]
    padded = np.full((n, tiles * tile), -np.inf, dtype=np.float32)
    padded[:, :v] = logits
    out = np.empty((n, n_targets), dtype=np.int64)
    for r in range(n):
        cand = np.argsort(-tile_max[r].astype(np.float64), kind="stable")[:min(n_targets, tiles)]
        pool_tokens = (cand[:, None] * tile + np.arange(tile)[None, :]).reshape(-1)
        pool = padded[r, pool_tokens]
        best = np.argsort(-pool.astype(np.float64), kind="stable")[:n_targets]
        out[r] = pool_tokens[best]
    return out


# --------------------------------------------------------------------------- spread / prior

def spread(table: np.ndarray, tokens: np.ndarray, dtype: str, sample: int = 64) -> np.ndarray:
    """iterate.py:275-284: per problem, the mean over the first ``sample`` items of the gap between
    the worst and best target, ``(N,)`` float32. ``table`` holds model-dtype values as float32 and
    ``dtype`` names that dtype ("bf16" or "f16"): the reference subtracts in it, so the float32
    difference is rounded to it before the float32 mean."""
    head = np.asarray(table, dtype=np.float32)[np.asarray(tokens), :sample]    # (N, M, sample)
    gap = (head.max(axis=1) - head.min(axis=1)).astype(np.float32)
    gap = to_model_dtype(gap, dtype)
    return gap.astype(np.float64).mean(axis=-1).astype(np.float32)


def prior(counts: np.ndarray, unit: np.ndarray, n_items: int, weight: float = 0.1) -> np.ndarray:
    """iterate.py:286-290, in the reference's float32 operation order."""
    counts = np.asarray(counts)
    unit = np.asarray(unit, dtype=np.float32).reshape(-1, 1)
    share = np.maximum(counts.astype(np.float32) / f32(n_items), f32(1e-9)).astype(np.float32)
    scale = (f32(-weight) * unit).astype(np.float32)
    inside = (scale * np.log(share).astype(np.float32)).astype(np.float32)
    blocked = np.broadcast_to((f32(BLOCKED) * unit).astype(np.float32), share.shape)
    return np.where(counts > 0, inside, blocked).astype(np.float32)


# --------------------------------------------------------------------------- condense / fit / argmin

def costs(table: np.ndarray, tokens: np.ndarray) -> np.ndarray:
    """``table[tokens]`` as float32: ``(N, M, A)``."""
    return np.asarray(table, dtype=np.float32)[np.asarray(tokens)]


def condense(table: np.ndarray, tokens: np.ndarray, offset: np.ndarray, k: int) -> np.ndarray:
    """iterate.py:195-211 (kernel 87-107): ``(N, k, A)`` int32 — for each item its ``k`` smallest
    packed keys of ``cost + offset``, ascending."""
    c = (costs(table, tokens) + np.asarray(offset, dtype=np.float32)[:, :, None]).astype(np.float32)
    n, m, a = c.shape
    target = np.broadcast_to(np.arange(m, dtype=np.int32)[None, :, None], c.shape)
    key = pack_key(c, target)
    return np.sort(key, axis=1)[:, :k, :].astype(np.int32)


def fit(key: np.ndarray, counts: np.ndarray, offset: np.ndarray, unit: np.ndarray, iterations: int,
        epsilon: float, relax: float = 1.9, endpoint: float = 0.0087, limit: float = STEP_LIMIT) -> np.ndarray:
    """iterate.py:292-312 (kernel 110-159): the annealed Sinkhorn fit; ``(N, M)`` float32 factors.

    Scalars reach the kernel as float32 (the anneal factor is formed in double first, 308); loads
    are float64 sums rounded to float32 (the reference's fp32 atomics approximate this)."""
    key = np.asarray(key, dtype=np.int32)
    n, k, a = key.shape
    counts = np.asarray(counts)
    m = counts.shape[1]
    anneal = f32((endpoint / epsilon) ** (1.0 / max(iterations, 1)))
    out = np.empty((n, m), dtype=np.float32)
    for p in range(n):
        u = f32(np.asarray(unit, dtype=np.float32).reshape(-1)[p])
        share = np.log(np.maximum(counts[p].astype(np.float32), f32(1e-9))).astype(np.float32)
        temperature = f32(f32(epsilon) * u)
        bound = f32(f32(limit) * u)
        correction = np.zeros(m, dtype=np.float32)
        target, base = unpack_key(key[p])
        for _ in range(iterations):
            cost = (base + correction[target]).astype(np.float32)
            w = (-cost / temperature).astype(np.float32)
            w = np.exp((w - w.max(axis=0, keepdims=True)).astype(np.float32)).astype(np.float32)
            w = (w / w.sum(axis=0, keepdims=True, dtype=np.float32)).astype(np.float32)
            load = np.bincount(target.reshape(-1), weights=w.reshape(-1).astype(np.float64),
                               minlength=m).astype(np.float32)
            step = (temperature * (np.log(np.maximum(load, f32(LOAD_FLOOR))).astype(np.float32) - share)).astype(np.float32)
            step = np.minimum(np.maximum(step, -bound), bound)
            correction = (correction + f32(relax) * step).astype(np.float32)
            correction = np.where(counts[p] > 0, correction, f32(0.0)).astype(np.float32)
            temperature = f32(temperature * anneal)
        out[p] = (np.asarray(offset, dtype=np.float32)[p] + correction).astype(np.float32)
    return out


def argmin(table: np.ndarray, tokens: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """iterate.py:314-320, 345-346: ``sigma[a] = argmin_m (C[m, a] + b[m])``, lowest m on ties."""
    c = (costs(table, tokens) + np.asarray(bias, dtype=np.float32)[:, :, None]).astype(np.float32)
    return c.argmin(axis=1).astype(np.int64)


def argmin_margin(table: np.ndarray, tokens: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """Gap between the best and second-best ``C[m, a] + b[m]`` per item (float64): how far an item's
    assignment is from a tie."""
    c = costs(table, tokens).astype(np.float64) + np.asarray(bias, dtype=np.float64)[:, :, None]
    part = np.partition(c, 1, axis=1)
    return part[:, 1, :] - part[:, 0, :]


# --------------------------------------------------------------------------- pipeline

def assign(table: np.ndarray, logits: np.ndarray, dtype: str, *, n_targets: int = 128, k: int = 8,
           rounds: int = 2, iterations: int = 12, weight: float = 0.1, epsilon: float = 0.15,
           refocus: float = 0.35, full_sigma: bool = True) -> dict:
    """iterate.py:322-342: shortlist, spread, prior, then ``rounds`` of condense + fit, then argmin.
    Returns the stages too (tokens, counts, unit, prior, keys and bias of each round)."""
    n_items = table.shape[1]
    tokens, counts, values, normaliser = shortlist(logits, n_items, n_targets)
    unit = spread(table, tokens, dtype)
    bias = prior(counts, unit, n_items, weight)
    stages = {"tokens": tokens, "counts": counts, "values": values, "normaliser": normaliser,
              "unit": unit, "prior": bias, "keys": [], "biases": []}
    for index in range(rounds):
        offset = bias
        key = condense(table, tokens, offset, k)
        bias = fit(key, counts, offset, unit, iterations, epsilon if index == 0 else epsilon * refocus)
        stages["keys"].append(key)
        stages["biases"].append(bias)
    stages["bias"] = bias
    if full_sigma:
        stages["sigma"] = argmin(table, tokens, bias)
    return stages


def decode_item(table: np.ndarray, tokens: np.ndarray, bias: np.ndarray, values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """auxiliary.py:70-75 for the one item each problem reads: (token, argmin margin)."""
    n_items = table.shape[1]
    items = np.clip(np.asarray(values, dtype=np.int64).reshape(-1), 0, n_items - 1)
    out = np.empty(len(items), dtype=np.int64)
    margin = np.empty(len(items), dtype=np.float64)
    tab = np.asarray(table, dtype=np.float32)
    for p, a in enumerate(items):
        c = (tab[tokens[p], a] + bias[p]).astype(np.float32)
        s = int(np.argmin(c))
        out[p] = tokens[p, s]
        srt = np.sort(c.astype(np.float64))
        margin[p] = srt[1] - srt[0] if len(srt) > 1 else np.inf
    return out, margin


def decode_unmasked(table: np.ndarray, logits: np.ndarray, values: np.ndarray, dtype: str, **kwargs) -> np.ndarray:
    """auxiliary.py:67-75: the token each problem's auxiliary value decodes to."""
    stages = assign(table, logits, dtype, full_sigma=False, **kwargs)
    return decode_item(table, stages["tokens"], stages["bias"], values)[0]


def build_table(vocabulary, output_weight):
    """auxiliary.py:56-65: ``-(vocabulary @ output_weight^T)^T`` in the model dtype, ``(V, A)``.
    Takes and returns CPU torch tensors (torch ``F.linear`` in the operands' dtype)."""
    import torch.nn.functional as F
    scores = F.linear(vocabulary.cpu(), output_weight.cpu())
    return scores.t().contiguous().neg()
