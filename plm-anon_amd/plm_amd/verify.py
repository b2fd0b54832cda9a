"""Fused LM-head verify step on the HIP kernel: the LM-head GEMM with the round's acceptance
epilogue folded in, so the ``[R, V]`` logits are never written to memory.

Per row ``r`` it returns the acceptance rule's decision for ``pending[r]`` (``nucleus_acceptance``,
plm/decoder.py:71-75, or ``floor_acceptance``, 78-82) and the row argmax with lowest-index ties
(``logits.argmax(-1)``, plm/decoder.py:362). ``round_epilogue`` is the rest of the round's
bookkeeping (``RoundDecoder._epilogue``, plm/decoder.py:351-365) on the device. ``round_to`` fixes which logits the decision reads: ``"fp32"`` is the fp32
accumulator; ``"bf16"``/``"fp16"`` round it to the model dtype first, which is what the reference's
decoder sees (the GEMM output cast at plm/fast_gemm.py:46, upcast again at plm/decoder.py:73).
"""

from __future__ import annotations

import torch

from . import _lib
from .fast_gemm import HALF_DTYPES, Config, packed_weight, row_major_weight, workspace

ROUND_MODES = {"fp32": _lib.PLM_ROUND_F32, "bf16": _lib.PLM_ROUND_BF16, "fp16": _lib.PLM_ROUND_F16}
RULES = {"nucleus": _lib.PLM_RULE_NUCLEUS, "floor": _lib.PLM_RULE_FLOOR}

# Verify tile over packed weights (plm_lm_head_verify_packed): the row-split layout, 128-row tiles.
VERIFY_CONFIG: Config = {"wave_frags": 4, "k_waves": 1, "split_k": 1, "unroll": 4}

# A GEMM tile with the packed verify's accumulation order (every logit one MFMA chain over the K
# steps in order): ``hip_linear_f32`` with it (or any row-split tile with split_k 1) returns, bit for
# bit, the logits the packed verify decides on.
LOGITS_CONFIG: Config = {"wave_frags": 2, "k_waves": 1, "split_k": 1, "unroll": 2}

# The same pair for the verify kernel over row-major weights (``packed=False``): its workgroup's
# four wavefronts each take a quarter of K, summed in wavefront order, as the packed GEMM's
# 4-wavefront K split does.
ROWMAJOR_VERIFY_CONFIG: Config = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 4}
ROWMAJOR_LOGITS_CONFIG: Config = {"wave_frags": 2, "k_waves": 4, "split_k": 1, "unroll": 2}


def verify_workspace_bytes(R: int, V: int, K: int, cfg: Config = VERIFY_CONFIG) -> int:
    return int(_lib.lib().plm_lm_head_verify_workspace_bytes(R, V, K, _lib.Tile.from_config(cfg)))


def lm_head_verify(x: torch.Tensor, w: torch.Tensor, pending: torch.Tensor, p: float, round_to: str = "fp32",
                   cfg: Config | None = None, accept: torch.Tensor | None = None,
                   argmax: torch.Tensor | None = None, packed: bool = True,
                   rule: str = "nucleus") -> tuple[torch.Tensor, torch.Tensor]:
    """``(accept[R] bool, argmax[R] int64)`` for ``logits = x[R,K] @ w[V,K]^T``.

    ``pending[R]`` (int64, on the GPU) are the proposed ids; an id outside ``[0, V)`` is never
    accepted. ``rule`` is the decoder's ``accept_rule``: ``"nucleus"`` reads ``p`` as top-p
    (``p <= 0`` accepts nothing: exact matching, plm/decoder.py:115), ``"floor"`` as epsilon.
    With ``packed``
    (the default) W is read through its packed copy (``fast_gemm.packed_weight``, made once per
    weight) on the packed GEMM's pipeline; ``packed=False`` reads W row-major."""
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"lm_head_verify expects x[R,K] and w[V,K], got {tuple(x.shape)} and {tuple(w.shape)}")
    if x.dtype not in HALF_DTYPES or w.dtype != x.dtype:
        raise TypeError(f"lm_head_verify needs matching bf16/fp16 operands, got {x.dtype} and {w.dtype}")
    if round_to not in ROUND_MODES:
        raise ValueError(f"round_to must be one of {sorted(ROUND_MODES)}")
    if rule not in RULES:
        raise ValueError(f"rule must be one of {sorted(RULES)}")
    R, K = x.shape
    V = w.shape[0]
    if pending.shape != (R,) or pending.dtype != torch.int64 or pending.device != x.device:
        raise ValueError(f"pending must be an int64 [{R}] tensor on {x.device}")
    if not (x.is_cuda and w.is_cuda):
        raise RuntimeError("lm_head_verify runs on the GPU only; got a CPU tensor")
    cfg = (VERIFY_CONFIG if packed else ROWMAJOR_VERIFY_CONFIG) if cfg is None else cfg
    tile = _lib.Tile.from_config(cfg)
    x = x if (x.stride(1) == 1 and x.stride(0) % 8 == 0) else x.contiguous()
    if not packed:  # the packed path reads packed_weight(w), which handles any layout of w itself
        w = row_major_weight(w)
        w = w if (w.stride(1) == 1 and w.stride(0) % 8 == 0) else w.contiguous()
    pending = pending.contiguous()
    # The kernel writes one byte 0/1 per row: a bool tensor's storage directly.
    direct = accept is not None and accept.dtype == torch.bool and accept.is_contiguous() and accept.shape == (R,)
    accept_out = accept if direct else torch.empty(R, dtype=torch.bool, device=x.device)
    if argmax is None:
        argmax = torch.empty(R, dtype=torch.int64, device=x.device)
    lib = _lib.lib()
    need = int(lib.plm_lm_head_verify_workspace_bytes(R, V, K, tile))
    ws = workspace(x.device, need)
    common = (pending.data_ptr(), RULES[rule], float(p), ROUND_MODES[round_to], accept_out.data_ptr(), argmax.data_ptr(), tile,
              ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device))
    if packed:
        status = lib.plm_lm_head_verify_packed(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0),
                                               packed_weight(w).data_ptr(), R, V, K, *common)
        _lib.check(status, f"plm_lm_head_verify_packed(R={R}, V={V}, K={K}, cfg={cfg})")
    else:
        status = lib.plm_lm_head_verify(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0), w.data_ptr(),
                                        w.stride(0), R, V, K, *common)
        _lib.check(status, f"plm_lm_head_verify(R={R}, V={V}, K={K}, cfg={cfg})")
    if accept is not None and not direct:
        accept.copy_(accept_out)
        return accept, argmax
    return accept_out, argmax


_I64, _U8 = (torch.int64,), (torch.bool, torch.uint8)


def _ptr(t: torch.Tensor | None, name: str, n: int, dtypes: tuple, dev: torch.device) -> int:
    """Device pointer of a contiguous tensor of at least ``n`` entries on ``dev`` (0 for None)."""
    if t is None:
        return 0
    if t.device != dev or t.dtype not in dtypes or not t.is_contiguous() or t.numel() < n:
        raise ValueError(f"{name} must be a contiguous {dtypes[0]} tensor of >= {n} entries on {dev}")
    return t.data_ptr()


def _state_args(k, verify, pending, anchor, out, base_t, offset_t, round_sequence, sequence_step, dev) -> tuple:
    """The decoder-state arguments shared by plm_round_epilogue and plm_round_verify_packed, from
    ``verify`` to ``sequence_step``."""
    return (_ptr(verify, "verify", k, _I64, dev), _ptr(pending, "pending", k - 1, _I64, dev) if k > 1 else 0,
            _ptr(anchor, "anchor", 1, _I64, dev), _ptr(out, "out", 0, _I64, dev), out.numel(),
            _ptr(base_t, "base_t", 1, _I64, dev), _ptr(offset_t, "offset_t", 1, _I64, dev),
            _ptr(round_sequence, "round_sequence", 1, _I64, dev),
            0 if round_sequence is None else round_sequence.numel(), _ptr(sequence_step, "sequence_step", 1, _I64, dev))


def round_epilogue(k: int, widened: torch.Tensor, hypotheses: torch.Tensor, verify: torch.Tensor,
                   pending: torch.Tensor, anchor: torch.Tensor, out: torch.Tensor, base_t: torch.Tensor,
                   offset_t: torch.Tensor, round_sequence: torch.Tensor | None = None,
                   sequence_step: torch.Tensor | None = None, accepted: torch.Tensor | None = None,
                   num_correct: torch.Tensor | None = None) -> None:
    """``RoundDecoder._epilogue`` (plm/decoder.py:351-365) after the fused verify, in one launch.

    ``widened[k-1]`` (bool/uint8) is ``lm_head_verify``'s ``accept`` for verify rows ``0..k-2``
    with ``pending`` as the proposed ids; ``hypotheses[k*k]`` its ``argmax`` for the proposal rows
    ``k..k+k*k-1``; ``verify[k]`` the verify rows' decoded tokens. Updates ``pending``, ``anchor``,
    ``out``, ``base_t``, ``offset_t`` and (if given) ``round_sequence``/``sequence_step`` in place, as
    the reference does; ``accepted[k-1]`` and ``num_correct`` (0-dim or [1] int64) are optional
    outputs. Every tensor is a contiguous int64 (``widened``/``accepted``: one byte per entry)
    tensor on the GPU."""
    if not 1 <= k <= 64:
        raise ValueError(f"k must be in [1, 64], got {k}")
    dev = verify.device
    if not verify.is_cuda:
        raise RuntimeError("round_epilogue runs on the GPU only; got a CPU tensor")

    if (round_sequence is None) != (sequence_step is None):
        raise ValueError("round_sequence and sequence_step go together")
    args = (_ptr(widened, "widened", k - 1, _U8, dev) if k > 1 else 0, _ptr(hypotheses, "hypotheses", k * k, _I64, dev),
            *_state_args(k, verify, pending, anchor, out, base_t, offset_t, round_sequence, sequence_step, dev),
            _ptr(accepted, "accepted", k - 1, _U8, dev), _ptr(num_correct, "num_correct", 1, _I64, dev))
    status = _lib.lib().plm_round_epilogue(k, *args, _lib.stream_handle(dev))
    _lib.check(status, f"plm_round_epilogue(k={k})")


class RoundVerify:
    """The LM-head end of one round on the device (plm/decoder.py:351-365): one fused verify pass over
    the round's ``k + k*k`` rows (the rule's decisions for verify rows ``0..k-2`` against the pending
    proposals, the argmax of every row) and the epilogue. With ``fused`` (the default, for rounds of
    at most 64 rows: k <= 7) both are one launch pair, ``plm_round_verify_packed``, whose last
    workgroup runs the epilogue; otherwise rows go to the verify kernel in chunks of at most 64 and
    ``round_epilogue`` follows. Buffers are allocated once, so calls can be captured in a HIP graph."""

    def __init__(self, k: int, rule: str = "nucleus", threshold: float = -1.0, round_to: str = "fp32",
                 device: torch.device | str = "cuda", cfg: Config | None = None, fused: bool = True):
        if rule not in RULES or round_to not in ROUND_MODES:
            raise ValueError(f"rule must be one of {sorted(RULES)} and round_to one of {sorted(ROUND_MODES)}")
        if not 1 <= k <= 64:
            raise ValueError(f"k must be in [1, 64], got {k}")
        self.k, self.width = k, k + k * k
        self.rule, self.threshold, self.round_to, self.cfg = rule, float(threshold), round_to, cfg
        self.rows_pending = torch.full((self.width,), -1, dtype=torch.int64, device=device)
        self.accept = torch.zeros(self.width, dtype=torch.bool, device=device)
        self.argmax = torch.zeros(self.width, dtype=torch.int64, device=device)
        self.fused = fused and self.width <= 64

    def __call__(self, hidden: torch.Tensor, w: torch.Tensor, verify_tokens: torch.Tensor, pending: torch.Tensor,
                 anchor: torch.Tensor, out: torch.Tensor, base_t: torch.Tensor, offset_t: torch.Tensor,
                 round_sequence: torch.Tensor | None = None, sequence_step: torch.Tensor | None = None,
                 accepted: torch.Tensor | None = None, num_correct: torch.Tensor | None = None) -> None:
        k, W = self.k, self.width
        if hidden.dim() != 2 or hidden.shape[0] != W:
            raise ValueError(f"hidden must be [{W}, K] for k={k}, got {tuple(hidden.shape)}")
        if self.fused:
            self._fused(hidden, w, verify_tokens, pending, anchor, out, base_t, offset_t, round_sequence,
                        sequence_step, accepted, num_correct)
            return
        if k > 1:
            self.rows_pending[: k - 1].copy_(pending)
        for r0 in range(0, W, 64):
            r1 = min(W, r0 + 64)
            lm_head_verify(hidden[r0:r1], w, self.rows_pending[r0:r1], self.threshold, self.round_to, self.cfg,
                           accept=self.accept[r0:r1], argmax=self.argmax[r0:r1], rule=self.rule)
        round_epilogue(k, self.accept[: max(k - 1, 0)], self.argmax[k:], verify_tokens, pending, anchor, out, base_t,
                       offset_t, round_sequence, sequence_step, accepted, num_correct)

    def _fused(self, hidden, w, verify_tokens, pending, anchor, out, base_t, offset_t, round_sequence, sequence_step,
               accepted, num_correct) -> None:
        k, W = self.k, self.width
        if hidden.dtype not in HALF_DTYPES or w.dtype != hidden.dtype or hidden.shape[1] != w.shape[1]:
            raise TypeError(f"RoundVerify needs matching bf16/fp16 operands, got {hidden.dtype} and {w.dtype}")
        if not (hidden.is_cuda and w.is_cuda):
            raise RuntimeError("RoundVerify runs on the GPU only; got a CPU tensor")
        if (round_sequence is None) != (sequence_step is None):
            raise ValueError("round_sequence and sequence_step go together")
        dev = hidden.device
        x = hidden if (hidden.stride(1) == 1 and hidden.stride(0) % 8 == 0) else hidden.contiguous()
        V, K = w.shape
        tile = _lib.Tile.from_config(VERIFY_CONFIG if self.cfg is None else self.cfg)
        lib = _lib.lib()
        ws = workspace(dev, int(lib.plm_lm_head_verify_workspace_bytes(W, V, K, tile)))
        status = lib.plm_round_verify_packed(
            _lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0), packed_weight(w).data_ptr(), k, V, K,
            RULES[self.rule], self.threshold, ROUND_MODES[self.round_to],
            *_state_args(k, verify_tokens, pending, anchor, out, base_t, offset_t, round_sequence, sequence_step, dev),
            self.accept.data_ptr(), self.argmax.data_ptr(), _ptr(accepted, "accepted", k - 1, _U8, dev),
            _ptr(num_correct, "num_correct", 1, _I64, dev), tile, ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
        _lib.check(status, f"plm_round_verify_packed(k={k}, V={V}, K={K})")


def lm_head_verify_logits(x: torch.Tensor, w: torch.Tensor, pending: torch.Tensor, pending_rows: int, p: float,
                          logits: torch.Tensor, logit_rows: int, rule: str = "nucleus", cfg: Config | None = None,
                          accept: torch.Tensor | None = None,
                          argmax: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``lm_head_verify`` over the packed weight for a round whose verify rows decode through the
    auxiliary scheme: rows ``r < pending_rows`` decide on ``pending[r]`` (the rest are never
    accepted) and the logits of rows ``[0, logit_rows)`` land in ``logits`` (model dtype, rounded as
    the decision reads them) — the reference's ``logits[:K]`` (plm/decoder.py:318-320) without the
    other rows' logits ever being written. The decision reads model-dtype logits."""
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"lm_head_verify_logits expects x[R,K] and w[V,K], got {tuple(x.shape)} and {tuple(w.shape)}")
    if x.dtype not in HALF_DTYPES or w.dtype != x.dtype or logits.dtype != x.dtype:
        raise TypeError(f"lm_head_verify_logits needs matching bf16/fp16 operands, got {x.dtype}, {w.dtype}, "
                        f"{logits.dtype}")
    if rule not in RULES:
        raise ValueError(f"rule must be one of {sorted(RULES)}")
    R, K = x.shape
    V = w.shape[0]
    if not 0 <= pending_rows <= R or not 0 <= logit_rows <= R:
        raise ValueError(f"pending_rows and logit_rows must be in [0, {R}]")
    if pending.dtype != torch.int64 or pending.numel() < pending_rows or not pending.is_contiguous():
        raise ValueError(f"pending must be a contiguous int64 tensor of >= {pending_rows} entries")
    if logits.dim() != 2 or logits.shape[0] < logit_rows or logits.shape[1] < V or logits.stride(1) != 1:
        raise ValueError(f"logits must be a row-major [>= {logit_rows}, >= {V}] tensor, got {tuple(logits.shape)}")
    if not (x.is_cuda and w.is_cuda and logits.is_cuda):
        raise RuntimeError("lm_head_verify_logits runs on the GPU only; got a CPU tensor")
    cfg = VERIFY_CONFIG if cfg is None else cfg
    tile = _lib.Tile.from_config(cfg)
    x = x if (x.stride(1) == 1 and x.stride(0) % 8 == 0) else x.contiguous()
    accept = torch.empty(R, dtype=torch.bool, device=x.device) if accept is None else accept
    argmax = torch.empty(R, dtype=torch.int64, device=x.device) if argmax is None else argmax
    _ptr(accept, "accept", R, _U8, x.device)
    _ptr(argmax, "argmax", R, _I64, x.device)
    lib = _lib.lib()
    ws = workspace(x.device, int(lib.plm_lm_head_verify_workspace_bytes(R, V, K, tile)))
    mode = _lib.PLM_ROUND_BF16 if x.dtype == torch.bfloat16 else _lib.PLM_ROUND_F16
    status = lib.plm_lm_head_verify_packed_logits(
        _lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0), packed_weight(w).data_ptr(), R, V, K,
        pending.data_ptr() if pending_rows > 0 else 0, pending_rows, RULES[rule], float(p), mode, accept.data_ptr(),
        argmax.data_ptr(), logits.data_ptr(), logits.stride(0), logit_rows, tile, ws.data_ptr(), ws.numel(),
        _lib.stream_handle(x.device))
    _lib.check(status, f"plm_lm_head_verify_packed_logits(R={R}, V={V}, K={K}, logit_rows={logit_rows})")
    return accept, argmax


class AuxRoundVerify:
    """The LM-head end of a steady round whose verify rows decode through the logit-Voronoi scheme
    (RoundDecoder._steady_round, plm/decoder.py:316-322): one verify launch pair over the round's
    ``k + k*k`` rows that also writes the ``k`` verify rows' logits, the scheme's decode of those rows
    (``LogitVoronoiAuxiliary.decode_unmasked``), and the epilogue (plm/decoder.py:351-365). Buffers
    are allocated once, so a call can be captured in a HIP graph after one eager call."""

    def __init__(self, k: int, scheme, vocab: int, rule: str = "nucleus", threshold: float = -1.0,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda", cfg: Config | None = None):
        if not 1 <= k <= 7:
            raise ValueError(f"k must be in [1, 7] (a round of at most 64 rows), got {k}")
        if rule not in RULES:
            raise ValueError(f"rule must be one of {sorted(RULES)}")
        self.k, self.width, self.scheme = k, k + k * k, scheme
        self.rule, self.threshold, self.cfg = rule, float(threshold), cfg
        ld = (vocab + 7) // 8 * 8
        self.logits = torch.empty(k, ld, dtype=dtype, device=device)
        self.verify_tokens = torch.zeros(k, dtype=torch.int64, device=device)
        self.accept = torch.zeros(self.width, dtype=torch.bool, device=device)
        self.argmax = torch.zeros(self.width, dtype=torch.int64, device=device)
        self.vocab = vocab

    def __call__(self, hidden: torch.Tensor, w: torch.Tensor, values: torch.Tensor, pending: torch.Tensor,
                 anchor: torch.Tensor, out: torch.Tensor, base_t: torch.Tensor, offset_t: torch.Tensor,
                 round_sequence: torch.Tensor | None = None, sequence_step: torch.Tensor | None = None,
                 accepted: torch.Tensor | None = None, num_correct: torch.Tensor | None = None) -> torch.Tensor:
        """``values[k]``: the verify rows' auxiliary values. Returns the decoded verify tokens."""
        k, W = self.k, self.width
        if hidden.dim() != 2 or hidden.shape[0] != W or w.shape[0] != self.vocab:
            raise ValueError(f"hidden must be [{W}, K] and w [{self.vocab}, K]")
        lm_head_verify_logits(hidden, w, pending, k - 1, self.threshold, self.logits, k, self.rule, self.cfg,
                              accept=self.accept, argmax=self.argmax)
        self.scheme.decode_unmasked(self.logits[:, : self.vocab], None, w, values, out=self.verify_tokens)
        round_epilogue(k, self.accept[: max(k - 1, 0)], self.argmax[k:], self.verify_tokens, pending, anchor, out,
                       base_t, offset_t, round_sequence, sequence_step, accepted, num_correct)
        return self.verify_tokens
