"""The round workloads the MI355X kernels are measured and checked on, and their seeded inputs.

A PLM round runs its linears at ``M = k + k^2`` rows (plm/rounds.py:62-64): 42 at k=6, 56 at k=7.
The measured shapes are GPT-style blocks (QKV ``H -> 3H``, attention-out ``H -> H``, MLP up
``H -> 4H``, MLP down ``4H -> H``) plus a GPT-2-vocabulary LM head ``H -> 50257``. Weights are
``[N, K]`` row-major (the layout ``fast_gemm`` receives, plm/fast_gemm.py:84,108).

Seeds: X ~ N(0,1) with seed ``1000*cfg``; the weight of GEMM ``i`` ~ 0.02*N(0,1) with seed
``1 + 1000*cfg + i``; the verify step's proposals ~ U[0, 50257) with seed ``2 + 1000*5``.
Tensors are drawn in fp32 on the CPU with ``torch.Generator`` and rounded to the dtype
(round-to-nearest-even), so a CPU check and the GPU see the same bits.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

GPT2_VOCAB = 50257
TOP_P = 0.94
M_SWEEP = (7, 14, 28, 42, 56)


@dataclass(frozen=True)
class Gemm:
    name: str
    N: int
    K: int

    def bytes(self, M: int, elem: int = 2) -> int:
        """Algorithmic HBM bytes of one call: read W and X once, write Y once."""
        return elem * (self.N * self.K + M * self.K + M * self.N)

    def flops(self, M: int) -> int:
        return 2 * M * self.N * self.K


def gpt_block(hidden: int, mlp: int) -> list[Gemm]:
    return [Gemm("qkv", 3 * hidden, hidden), Gemm("attn_out", hidden, hidden), Gemm("mlp_up", mlp, hidden),
            Gemm("mlp_down", hidden, mlp)]


def llama_block(hidden: int, qkv: int, intermediate: int) -> list[Gemm]:
    """The reference's per-layer linears (plm/gemm_tables.py:22-27): fused QKV with grouped KV heads,
    attention-out, fused gate/up, down."""
    return [Gemm("qkv", qkv, hidden), Gemm("o", hidden, hidden), Gemm("gate_up", 2 * intermediate, hidden),
            Gemm("down", hidden, intermediate)]


# The reference's released Llama-style linear sets at hidden 2048 and 3072 (the shapes its tile tables
# key, plm/gpu_tuning/tiles_hidden{2048,3072}.json; vocabulary padded to 50304, plm/gemm_tables.py:16,
# 26). The reference reads the layer counts from its checkpoints; these are the build's choice for
# the 1.3B and 3B classes.
LLAMA_SETS = {
    "1.3B": {"hidden": 2048, "qkv": 3072, "intermediate": 5632, "layers": 24, "vocab": 50304},
    "3B": {"hidden": 3072, "qkv": 4608, "intermediate": 8192, "layers": 28, "vocab": 50304},
}


def llama_round(name: str) -> list[Gemm]:
    s = LLAMA_SETS[name]
    gemms = [g for _ in range(s["layers"]) for g in llama_block(s["hidden"], s["qkv"], s["intermediate"])]
    return gemms + [Gemm("lm_head", s["vocab"], s["hidden"])]


def round_linears(hidden: int, mlp: int, layers: int, vocab: int = GPT2_VOCAB) -> list[Gemm]:
    gemms = [g for _ in range(layers) for g in gpt_block(hidden, mlp)]
    return gemms + [Gemm("lm_head", vocab, hidden)]


@dataclass(frozen=True)
class Workload:
    name: str
    cfg: int          # index used in the seeds
    M: int
    gemms: tuple[Gemm, ...]

    @property
    def bytes(self) -> int:
        return sum(g.bytes(self.M) for g in self.gemms)

    @property
    def flops(self) -> int:
        return sum(g.flops(self.M) for g in self.gemms)

    def at(self, M: int) -> "Workload":
        return Workload(f"{self.name}@M{M}", self.cfg, M, self.gemms)


# The measured configurations, smallest first.
SINGLE_GEMM = Workload("350M-shape MLP up, k=6", 1, 42, (Gemm("mlp_up", 4096, 1024),))
BLOCK_1P3B = Workload("1.3B-shape block, k=7", 2, 56, tuple(gpt_block(2048, 8192)))
ROUND_1P3B = Workload("1.3B-shape round (24 blocks + LM head), k=7", 3, 56, tuple(round_linears(2048, 8192, 24)))
ROUND_3B = Workload("3B-shape round (32 blocks + LM head), k=7", 4, 56, tuple(round_linears(2560, 10240, 32)))
VERIFY_1P3B = Workload("fused LM-head verify, 1.3B shape", 5, 56, (Gemm("lm_head", GPT2_VOCAB, 2048),))

WORKLOADS = {w.cfg: w for w in (SINGLE_GEMM, BLOCK_1P3B, ROUND_1P3B, ROUND_3B, VERIFY_1P3B)}


def x_seed(cfg: int) -> int:
    return 1000 * cfg


def w_seed(cfg: int, index: int) -> int:
    return 1 + 1000 * cfg + index


def proposal_seed() -> int:
    return 2 + 1000 * 5


def normal(shape: tuple[int, ...], seed: int, std: float = 1.0, dtype: torch.dtype = torch.bfloat16,
           device: str | torch.device = "cpu") -> torch.Tensor:
    """``std * N(0,1)`` drawn in fp32 from a seeded generator on ``device``, then rounded to ``dtype``."""
    gen = torch.Generator(device=device).manual_seed(seed)
    t = torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
    if std != 1.0:
        t.mul_(std)
    return t.to(dtype)


def activations(cfg: int, M: int, K: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    return normal((M, K), x_seed(cfg), 1.0, dtype)


def weight(cfg: int, index: int, N: int, K: int, dtype: torch.dtype = torch.bfloat16,
           device: str | torch.device = "cpu") -> torch.Tensor:
    return normal((N, K), w_seed(cfg, index), 0.02, dtype, device)


def proposals(R: int, vocab: int = GPT2_VOCAB) -> torch.Tensor:
    gen = torch.Generator().manual_seed(proposal_seed())
    return torch.randint(0, vocab, (R,), generator=gen, dtype=torch.int64)
