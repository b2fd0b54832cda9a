"""Writes the golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no tests or result vectors for its GEMM or verify path, so these fixtures are
this build's own: seeded inputs plus expected outputs computed by fp64 brute force with numpy
(independent of torch's CPU matmul, which the oracle wraps), following the reference's formulas:

* GEMM ``y = x @ w.T`` rounded once to the output dtype (plm/fast_gemm.py:35-46, 111);
* the nucleus rule (plm/decoder.py:71-75) by a descending sort walk, and argmax with the lowest
  index winning ties (plm/decoder.py:362).

Half-precision tensors are stored as their uint16 bit patterns. Files are .npz without pickles.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_round(v: np.ndarray) -> np.ndarray:
    """Round fp64 values to bf16 (nearest, ties to even) through fp32, returned as uint16 bits.
    The fp64 -> fp32 step is exact enough here: an fp32 rounding can only move a value across a
    bf16 midpoint if it lies within 2^-24 relative of it, which the generator checks never happens."""
    f32 = v.astype(np.float32)
    u = f32.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def midpoint_clearance(v: np.ndarray) -> float:
    """Smallest relative distance of any value to a bf16 rounding midpoint."""
    f = np.abs(v[v != 0])
    e = np.floor(np.log2(f))
    step = 2.0 ** (e - 7)
    frac = (f / step) % 1.0
    return float(np.min(np.abs(frac - 0.5) * step / f))


def gemm_case(name: str, M: int, N: int, K: int, seed: int, ints: bool = False) -> None:
    g = torch.Generator().manual_seed(seed)
    if ints:
        x = torch.randint(-2, 3, (M, K), generator=g).bfloat16()
        w = torch.randint(-1, 2, (N, K), generator=g).bfloat16()
    else:
        x = torch.randn(M, K, generator=g).bfloat16()
        w = (0.02 * torch.randn(N, K, generator=g)).bfloat16()
    exact = x.double().numpy() @ w.double().numpy().T
    assert midpoint_clearance(exact) > 2.0 ** -24, name
    np.savez(HERE / f"{name}.npz", x=bits(x), w=bits(w), y_fp64=exact, y_bf16=bf16_round(exact),
             seed=np.int64(seed))
    print(f"{name}: x{tuple(x.shape)} w{tuple(w.shape)}")


def nucleus_fp64(z: np.ndarray, pending: np.ndarray, p: float) -> tuple[np.ndarray, np.ndarray]:
    """Decision and distance to the threshold for every row, by a sorted walk in fp64."""
    acc = np.zeros(z.shape[0], dtype=bool)
    margin = np.full(z.shape[0], np.inf)
    for r in range(z.shape[0]):
        row = np.exp(z[r] - z[r].max())
        row /= row.sum()
        own = row[pending[r]]
        mass = 0.0
        for v in np.sort(row)[::-1]:
            if v <= own:
                break
            mass += v
        top = own >= row.max()
        acc[r] = mass < p or (top and p > 0)
        if not top:
            margin[r] = abs(mass - p)
    return acc, margin


def argmax_lowest(z: np.ndarray) -> np.ndarray:
    out = np.empty(z.shape[0], dtype=np.int64)
    for r in range(z.shape[0]):
        best = 0
        for j in range(1, z.shape[1]):
            if z[r, j] > z[r, best]:
                best = j
        out[r] = best
    return out


def verify_case(name: str, R: int, V: int, K: int, p: float, seed: int) -> None:
    """Fused LM-head verify on fp32 logits of X @ W^T: expected accept bits and argmax ids. Rows
    whose decision is within 1e-4 of the threshold, or whose top-2 logits are within 1e-3, are
    marked unsafe (fp32 accumulation order could flip them)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(R, K, generator=g).bfloat16()
    w = (0.15 * torch.randn(V, K, generator=g)).bfloat16()
    z = x.double().numpy() @ w.double().numpy().T
    # Half the proposals are near the top of their row (so some are accepted), half uniform.
    order = np.argsort(-z, axis=1, kind="stable")
    pick = torch.randint(0, 8, (R,), generator=g).numpy()
    uniform = torch.randint(0, V, (R,), generator=g).numpy()
    pending = np.where(np.arange(R) % 2 == 0, order[np.arange(R), pick], uniform).astype(np.int64)
    acc, margin = nucleus_fp64(z, pending, p)
    am = argmax_lowest(z)
    top2 = np.sort(z, axis=1)[:, -2:]
    safe_acc = margin > 1e-4
    safe_am = (top2[:, 1] - top2[:, 0]) > 1e-3
    np.savez(HERE / f"{name}.npz", x=bits(x), w=bits(w), pending=pending, p=np.float64(p), accept=acc,
             argmax=am, safe_accept=safe_acc, safe_argmax=safe_am, seed=np.int64(seed))
    print(f"{name}: R={R} V={V} K={K} accepted {int(acc.sum())}/{R}, safe {int(safe_acc.sum())}/{int(safe_am.sum())}")


def main() -> None:
    gemm_case("gemm_m42_n96_k1024", 42, 96, 1024, seed=101)      # the 350M-shape k=6 width, K of the MLP up
    gemm_case("gemm_m56_n48_k2048", 56, 48, 2048, seed=102)      # the 1.3B-shape k=7 width
    gemm_case("gemm_m7_n33_k1416", 7, 33, 1416, seed=103)        # a partial round, ragged N and K
    gemm_case("gemm_m56_n64_k512_int", 56, 64, 512, seed=104, ints=True)  # exactly representable
    verify_case("verify_r24_v2003_k128", 24, 2003, 128, 0.94, seed=105)


if __name__ == "__main__":
    main()
