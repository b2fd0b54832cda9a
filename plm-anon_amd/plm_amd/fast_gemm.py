"""HIP skinny GEMM for the decode-width shapes of a PLM round, as a drop-in for the reference's
``plm.fast_gemm`` (plm/fast_gemm.py).

``C[M,N] = A[M,K] @ W[N,K]^T`` with fp32 accumulation on gfx950 MFMA, output in the input dtype.
The kernel reads W in a packed fragment layout (``plm_pack_weight``); each weight tensor is packed
once, on its first use, and the packed copy is kept while the tensor lives and is unchanged.
Split-K partials are combined inside the same launch in a fixed order, so results are bitwise
reproducible run to run (plm/fast_gemm.py:3-4). ``install`` routes eligible calls through the
kernel: the build's own dispatch slot always, and vLLM's ``default_unquantized_gemm`` when vLLM is
importable (plm/fast_gemm.py:100-113). Tile configs are keyed on ``(M, N, K)``; shapes without a
config go to ``F.linear``, exactly as in the reference.

``release(weight)`` keeps one copy of a weight: its row-major storage is freed and every product with
it runs from the packed copy: widths up to 128 rows (the round widths) on the packed kernel with
their tuned tiles or ``default_config``'s; wider calls (prefill chunks, plm/rounds.py:16, which the
reference hands to ``F.linear``) as ``F.linear`` on the weight unpacked into a transient buffer
(``unpacked``, bit for bit), which measured faster than ``plm_gemm_packed``'s own wide kernel
(1.3B block at M = 640: 134.5 against 190.7 µs), so they are the reference's own products.
"""

from __future__ import annotations

import threading

import torch
import torch.nn.functional as F
from torch.utils.weak import WeakTensorKeyDictionary

from . import _lib

# {"wave_frags", "k_waves", "split_k", "unroll"}: the MI355X counterpart of the reference's
# {BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K, num_warps, num_stages} (plm/fast_gemm.py:64).
Config = dict[str, int]

HALF_DTYPES = (torch.bfloat16, torch.float16)

CONFIGS: dict[tuple[int, int, int], Config] = {}
# Tiles for the fused gate/up projection with its SiLU-and-multiply (gate_up_silu), keyed like
# CONFIGS: the fastest tile with an even wave_frags (gemm_tables.install fills it).
ACT_CONFIGS: dict[tuple[int, int, int], Config] = {}

_tiles: dict[tuple[int, int, int, int], _lib.Tile] = {}
# weight tensor -> ((data_ptr, shape, row stride, version counter), packed copy); entries go with
# the tensor
_packed = WeakTensorKeyDictionary()
# released weight tensor -> its packed copy (the tensor itself then holds no data)
_released = WeakTensorKeyDictionary()
# fused gate/up weight tensor -> ((data_ptr, shape, row stride, version counter), packed copy with the
# gate and up halves interleaved by 16-row fragment)
_packed_gate_up = WeakTensorKeyDictionary()
_pack_lock = threading.Lock()
_workspaces: dict[int, torch.Tensor] = {}
_ws_lock = threading.Lock()


def _tile(cfg: Config) -> _lib.Tile:
    key = (int(cfg["wave_frags"]), int(cfg["k_waves"]), int(cfg.get("split_k", 1)), int(cfg["unroll"]))
    t = _tiles.get(key)
    if t is None:
        t = _tiles[key] = _lib.Tile(*key)
    return t


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device zero-filled byte workspace of at least ``nbytes`` (the reference's ``_partials``,
    plm/fast_gemm.py:70-79). Kernels leave it zeroed. It grows only outside HIP-graph capture:
    size it with an eager call (or ``reserve_workspace``) before capturing."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(index)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"plm_amd workspace needs {nbytes} bytes on cuda:{index} during graph capture; "
                               "run the shape eagerly (or call reserve_workspace) before capturing")
        with _ws_lock:
            buf = _workspaces.get(index)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 2 * buf.numel() if buf is not None else 0, 1 << 20)
                buf = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", index))
                _workspaces[index] = buf
    return buf


def reset_counters(buf: torch.Tensor) -> None:
    """Zeroes the counter area at the start of workspace ``buf`` (a uint8 tensor): every arrival
    counter, flag, epoch and the error int. After a bounded wait gave up, a late workgroup of the
    failed launch can have counted itself in after the counter's owner reset it; only a whole reset
    leaves every counter ready for the next launch."""
    buf[: _lib.COUNTER_BYTES].zero_()


def check_workspace(device: torch.device) -> None:
    """Raises if a launch on ``device``'s workspace reported a bounded wait that gave up (the int at
    ``PLM_WORKSPACE_ERROR_INDEX``: chained launches, the gated-LoRA launch, the fused verify), whose
    results are then invalid; the counter area is zeroed first, so the workspace is usable again.
    Synchronizes with the device: call it where the serving loop syncs anyway, with no launch on
    the workspace in flight."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(index)
    if buf is None:
        return
    flag = int(buf[: 4 * (_lib.ERROR_INDEX + 1)].view(torch.int32)[_lib.ERROR_INDEX].item())
    if flag:
        reset_counters(buf)
        raise RuntimeError(f"a launch on cuda:{index}'s workspace gave up a bounded wait (another process "
                           "holding CUs?): its results are invalid; the counter area was reset")


def gemm_workspace_bytes(M: int, N: int, K: int, cfg: Config) -> int:
    return int(_lib.lib().plm_gemm_packed_workspace_bytes(M, N, K, _tile(cfg)))


def tile_supported(M: int, K: int, cfg: Config, dtype: torch.dtype = torch.bfloat16) -> bool:
    return bool(_lib.lib().plm_gemm_packed_tile_supported(_lib.DTYPE_CODES[dtype], M, K, _tile(cfg)))


def pack_weight(w: torch.Tensor) -> torch.Tensor:
    """``w[N,K]`` rearranged into the kernel's fragment layout (a new uint8 device tensor of
    ``plm_packed_weight_bytes(N, K)`` bytes)."""
    if w.dim() != 2 or w.dtype not in HALF_DTYPES or not w.is_cuda:
        raise ValueError(f"pack_weight expects a 2-D bf16/fp16 GPU tensor, got {tuple(w.shape)} {w.dtype}")
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("a weight is packed on its first use, which cannot happen during graph capture; "
                           "run the shape eagerly (or call packed_weight) before capturing")
    w = _row_major(w)
    N, K = w.shape
    lib = _lib.lib()
    nbytes = int(lib.plm_packed_weight_bytes(N, K))
    out = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    status = lib.plm_pack_weight(_lib.DTYPE_CODES[w.dtype], w.data_ptr(), w.stride(0), N, K, out.data_ptr(), nbytes,
                                 _lib.stream_handle(w.device))
    _lib.check(status, f"plm_pack_weight(N={N}, K={K})")
    return out


def packed_weight(w: torch.Tensor) -> torch.Tensor:
    """The packed copy of ``w``, made on first use and reused while ``w`` lives unchanged (same
    storage, shape, stride and version counter); for a released weight, the copy it keeps."""
    released = _released.get(w)
    if released is not None:
        return released
    key = (w.data_ptr(), tuple(w.shape), w.stride(0), w._version)
    hit = _packed.get(w)
    if hit is not None and hit[0] == key:
        return hit[1]
    with _pack_lock:
        hit = _packed.get(w)
        if hit is not None and hit[0] == key:
            return hit[1]
        p = pack_weight(w)
        _packed[w] = (key, p)
        return p


def release(w: torch.Tensor) -> torch.Tensor:
    """Keep one copy of ``w``: pack it (if not yet) and free its row-major storage. ``w`` keeps its
    shape, dtype and device, but holds no data any more (a one-element view expanded to its shape):
    afterwards only the packed kernels may read it (``hip_linear``, ``fast_gemm`` at every width,
    the packed verify and chain); the row-major paths raise. The storage is returned to the caching
    allocator once nothing else refers to it. Returns ``w``."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("release() packs and frees memory, which cannot happen during graph capture")
    if w in _released:
        return w
    p = packed_weight(w)
    with _pack_lock:
        N, K = w.shape
        w.data = torch.empty(1, dtype=w.dtype, device=w.device).expand(N, K)
        _released[w] = p
        _packed.pop(w, None)
    return w


def is_released(w: torch.Tensor) -> bool:
    """Whether ``w``'s row-major data was freed by ``release``."""
    return w in _released


def unpack_weight(p: torch.Tensor, N: int, K: int, dtype: torch.dtype) -> torch.Tensor:
    """The row-major ``[N, K]`` weight rebuilt from its packed copy ``p`` (``plm_unpack_weight``), bit
    for bit: a new tensor on ``p``'s device."""
    out = torch.empty(N, K, dtype=dtype, device=p.device)
    status = _lib.lib().plm_unpack_weight(_lib.DTYPE_CODES[dtype], p.data_ptr(), p.numel(), N, K, out.data_ptr(), K,
                                          _lib.stream_handle(p.device))
    _lib.check(status, f"plm_unpack_weight(N={N}, K={K})")
    return out


def unpacked(w: torch.Tensor) -> torch.Tensor:
    """A transient row-major copy of a released weight, rebuilt from the packed copy it keeps."""
    p = _released.get(w)
    if p is None:
        raise ValueError("unpacked() takes a released weight")
    return unpack_weight(p, w.shape[0], w.shape[1], w.dtype)


def row_major_weight(w: torch.Tensor) -> torch.Tensor:
    """``w`` for a kernel that reads it row-major; raises for a released weight."""
    if w in _released:
        raise RuntimeError(f"weight {tuple(w.shape)} was released (only its packed copy exists); "
                           "use the packed kernels")
    return w


def default_config(M: int, N: int, K: int) -> Config:
    """The tile for a width the tables do not tune: round widths (M <= 128) take
    ``tiles.heuristic_tile``; wider calls run on the wide kernel, which has its own fixed tiling
    (any valid tile is accepted and not used)."""
    from .tiles import heuristic_tile

    if M <= 128:
        return heuristic_tile(M, N, K, supported=lambda cfg: tile_supported(M, K, cfg))
    return {"wave_frags": 2, "k_waves": 8, "split_k": 1, "unroll": 2}  # unused: the wide kernel runs


def gate_up_order(w: torch.Tensor) -> torch.Tensor:
    """A fused gate/up weight ``[2I, K]`` (gate rows first) with its halves interleaved by 16-row
    fragment — gate rows [16j, 16j+16), then up rows [16j, 16j+16), for j = 0, 1, ... — the row
    order ``plm_gemm_packed_silu_mul`` reads packed. A new tensor."""
    N, K = w.shape
    if N % 32:
        raise ValueError(f"a fused gate/up weight needs a multiple of 32 rows, got {N}")
    return w.reshape(2, N // 32, 16, K).transpose(0, 1).reshape(N, K).contiguous()


def packed_gate_up(w: torch.Tensor) -> torch.Tensor:
    """The interleaved packed copy of a fused gate/up weight, made on first use and kept while ``w``
    lives unchanged (for a released weight, rebuilt from its packed copy)."""
    key = (w.data_ptr(), tuple(w.shape), w.stride(0), w._version)
    hit = _packed_gate_up.get(w)
    if hit is not None and hit[0] == key:
        return hit[1]
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("a gate/up weight is packed on its first use, which cannot happen during graph capture")
    with _pack_lock:
        src = unpack_weight(_released[w], w.shape[0], w.shape[1], w.dtype) if w in _released else w
        p = pack_weight(gate_up_order(src))
        _packed_gate_up[w] = (key, p)
        return p


def gate_up_silu(x: torch.Tensor, w: torch.Tensor, cfg: Config | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(g) * u`` of the fused gate/up projection ``x @ w^T`` (``w = [gate; up]``, ``[2I, K]``),
    ``[M, I]`` in x's dtype, in one launch (``plm_gemm_packed_silu_mul``): the Llama-style MLP's
    gate_up_proj GEMM (routed through plm/fast_gemm.py:104-110) and the ``SiluAndMul`` vLLM runs on
    its output as a second launch, with the same roundings (the projection's output rounded to the
    model dtype, silu rounded, then the product). ``cfg``: the tile, by default ``ACT_CONFIGS``'
    (the fastest even-wave_frags tile the tuner found) or the projection's; a tile with
    wave_frags 1 runs with 2. Widths above 128 rows run as the
    projection then the activation, each as its own launch."""
    _check_operands(x, w)
    M, K = x.shape
    N = w.shape[0]
    half = N // 2
    if M > 128:
        y = released_linear(x, w) if w in _released else F.linear(x, w)
        act = F.silu(y[:, :half]) * y[:, half:]
        if out is not None:
            out.copy_(act)
            return out
        return act
    if cfg is None:
        cfg = ACT_CONFIGS.get((M, N, K)) or CONFIGS.get((M, N, K)) or default_config(M, N, K)
    if cfg["wave_frags"] % 2:
        cfg = dict(cfg, wave_frags=2)   # gate and up fragments pair up in a wavefront's or a tile's
    if out is None:
        out = torch.empty(M, half, device=x.device, dtype=x.dtype)
    elif out.shape != (M, half) or out.dtype != x.dtype or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major [{M},{half}] {x.dtype} tensor")
    x = _row_major(x)
    tile = _tile(cfg)
    lib = _lib.lib()
    need = int(lib.plm_gemm_packed_workspace_bytes(M, N, K, tile))
    ws_ptr, ws_bytes = None, 0
    if need:
        ws = workspace(x.device, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    status = lib.plm_gemm_packed_silu_mul(_lib.DTYPE_CODES[x.dtype], x.data_ptr(), x.stride(0),
                                          packed_gate_up(w).data_ptr(), out.data_ptr(), out.stride(0), M, N, K,
                                          tile, ws_ptr, ws_bytes, _lib.stream_handle(x.device))
    _lib.check(status, f"plm_gemm_packed_silu_mul(M={M}, N={N}, K={K}, cfg={cfg})")
    return out


def llama_mlp(x: torch.Tensor, gate_up_weight: torch.Tensor, down_weight: torch.Tensor,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """The Llama-style MLP's linears as the reference's rounds run them through vLLM:
    ``down_proj(SiluAndMul(gate_up_proj(x)))``, both projections routed through ``fast_gemm``
    (plm/fast_gemm.py:104-110; the model forward at plm/decoder.py:250-259). A drop-in for the MLP
    forward of one layer: ``gate_up_weight`` is the fused ``[2I, K]`` projection (gate rows first),
    ``down_weight`` ``[K, I]``; the result is ``[M, K]`` in x's dtype with the reference's three
    roundings (projection output, silu, product) and the down projection's.

    Up to 128 rows it is two launches: the gate/up projection with its SiLU-and-multiply
    (``gate_up_silu``, one launch, tile from ``ACT_CONFIGS``), then down (the tuned tile, or
    ``default_config``). One chained launch of the two (``LinearChain`` with ``Link(act=True)``)
    computes the same values bit for bit with matching tiles, but measured no faster on MI355X
    (hidden 2048, M = 56: 31.75 against 31.74 us; hidden 3072: 48.81 against 47.63 us). Wider
    calls (prefill chunks) run the projection, the activation and down through ``fast_gemm``'s own
    routing."""
    _check_operands(x, gate_up_weight)
    M, K = x.shape
    I = gate_up_weight.shape[0] // 2
    if gate_up_weight.shape[0] != 2 * I or down_weight.shape != (K, I) or down_weight.dtype != x.dtype:
        raise ValueError(f"llama_mlp expects gate_up [2I, {K}] and down [{K}, I], got "
                         f"{tuple(gate_up_weight.shape)} and {tuple(down_weight.shape)} {down_weight.dtype}")
    act = gate_up_silu(x, gate_up_weight)
    if M > 128:
        y = fast_gemm(None, act, down_weight)
        if out is None:
            return y
        out.copy_(y)
        return out
    cfg = CONFIGS.get((M, K, I)) or default_config(M, K, I)
    return hip_linear(act, down_weight, cfg, out)


def reserve_workspace(device: torch.device, shapes: dict[tuple[int, int, int], Config] | None = None) -> None:
    """Size the device workspace for every configured shape, so later calls can be graph-captured."""
    shapes = CONFIGS if shapes is None else shapes
    need = max((gemm_workspace_bytes(M, N, K, cfg) for (M, N, K), cfg in shapes.items()), default=0)
    if need:
        workspace(device, need)


def _row_major(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself if the kernel can read it in place (unit inner stride, 16-byte aligned rows)."""
    if t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0 and t.stride(0) >= t.shape[1]:
        return t
    return t.contiguous()


def launch_packed(a: torch.Tensor, wp: torch.Tensor, N: int, cfg: Config, out: torch.Tensor,
                  f32_out: bool = False) -> torch.Tensor:
    """``out = a @ W^T`` for a packed W (``pack_weight``) of N rows; ``out`` row-major."""
    M, K = a.shape
    a = _row_major(a)
    tile = _tile(cfg)
    lib = _lib.lib()
    need = int(lib.plm_gemm_packed_workspace_bytes(M, N, K, tile))
    ws_ptr, ws_bytes = None, 0
    if need:
        ws = workspace(a.device, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    entry = lib.plm_gemm_packed_f32out if f32_out else lib.plm_gemm_packed
    status = entry(_lib.DTYPE_CODES[a.dtype], a.data_ptr(), a.stride(0), wp.data_ptr(), out.data_ptr(), out.stride(0),
                   M, N, K, tile, ws_ptr, ws_bytes, _lib.stream_handle(a.device))
    _lib.check(status, f"plm_gemm_packed(M={M}, N={N}, K={K}, cfg={cfg})")
    return out


def _launch(a: torch.Tensor, w: torch.Tensor, cfg: Config, out: torch.Tensor, f32_out: bool) -> torch.Tensor:
    return launch_packed(a, packed_weight(w), w.shape[0], cfg, out, f32_out)


def hip_linear_rowmajor(a: torch.Tensor, w: torch.Tensor, cfg: Config, out: torch.Tensor | None = None,
                        f32_out: bool = False) -> torch.Tensor:
    """``a @ w.T`` on the streaming kernel that reads W row-major (``plm_gemm``; no packed copy).
    Its tiles: ``64*wave_frags`` rows, ``unroll`` = 2 (``tiles.stream_compiled``)."""
    _check_operands(a, w)
    row_major_weight(w)
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, N, device=a.device, dtype=torch.float32 if f32_out else a.dtype)
    a, w = _row_major(a), _row_major(w)
    tile = _tile(cfg)
    lib = _lib.lib()
    need = int(lib.plm_gemm_workspace_bytes(M, N, K, tile))
    ws_ptr, ws_bytes = None, 0
    if need:
        ws = workspace(a.device, need)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    entry = lib.plm_gemm_f32out if f32_out else lib.plm_gemm
    status = entry(_lib.DTYPE_CODES[a.dtype], a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                   out.stride(0), M, N, K, tile, ws_ptr, ws_bytes, _lib.stream_handle(a.device))
    _lib.check(status, f"plm_gemm(M={M}, N={N}, K={K}, cfg={cfg})")
    return out


def _check_operands(a: torch.Tensor, w: torch.Tensor) -> None:
    if a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise ValueError(f"hip_linear expects a[M,K] and w[N,K], got {tuple(a.shape)} and {tuple(w.shape)}")
    if a.dtype not in HALF_DTYPES or w.dtype != a.dtype:
        raise TypeError(f"hip_linear needs matching bf16/fp16 operands, got {a.dtype} and {w.dtype}")
    if not (a.is_cuda and w.is_cuda):
        raise RuntimeError("hip_linear runs on the GPU only; got a CPU tensor")


def hip_linear(a: torch.Tensor, w: torch.Tensor, cfg: Config, out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[M,N] = a[M,K] @ w[N,K]^T`` on the HIP kernel (the reference's ``triton_linear``,
    plm/fast_gemm.py:82-97). ``out`` is allocated as ``empty(M, N)`` in ``a``'s dtype if None."""
    _check_operands(a, w)
    M, N = a.shape[0], w.shape[0]
    if out is None:
        out = torch.empty(M, N, device=a.device, dtype=a.dtype)
    elif out.shape != (M, N) or out.dtype != a.dtype or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major [{M},{N}] {a.dtype} tensor")
    return _launch(a, w, cfg, out, False)


def hip_linear_f32(a: torch.Tensor, w: torch.Tensor, cfg: Config, out: torch.Tensor | None = None) -> torch.Tensor:
    """As ``hip_linear`` but returns the fp32 accumulator (no cast to the input dtype)."""
    _check_operands(a, w)
    M, N = a.shape[0], w.shape[0]
    if out is None:
        out = torch.empty(M, N, device=a.device, dtype=torch.float32)
    elif out.shape != (M, N) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError(f"out must be a row-major [{M},{N}] float32 tensor")
    return _launch(a, w, cfg, out, True)


# Widths above this run as F.linear on the unpacked weight (plm_gemm_packed's wide kernel, which
# takes them too, measured slower over the 1.3B block's linears from 256 rows on).
WIDE_ROWS = 128


def released_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` for a released weight, any leading shape of ``x``: up to
    ``WIDE_ROWS`` rows on the packed kernel (the tuned tile where the tables have one for
    ``(M, N, K)``, else ``default_config``; a bias added after), wider as ``F.linear`` on the weight
    unpacked into a transient buffer."""
    if x.dtype != weight.dtype:
        raise TypeError(f"released weight is {weight.dtype}, input is {x.dtype}")
    N, K = weight.shape
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if M > WIDE_ROWS:
        return F.linear(x, unpacked(weight), bias)
    if M == 0:
        out = x2.new_empty(0, N)
    else:
        cfg = CONFIGS.get((M, N, K)) or default_config(M, N, K)
        out = hip_linear(x2, weight, cfg)
    if bias is not None:
        out += bias
    return out.reshape(*lead, N)


def fast_gemm(layer, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """vLLM ``default_unquantized_gemm`` signature; tuned 2-D half-precision calls without bias go to
    the HIP kernel, everything else to ``F.linear`` (plm/fast_gemm.py:106-111). A released weight
    has no row-major data: every call with it runs on its packed copy (``released_linear``)."""
    if weight in _released:
        return released_linear(x, weight, bias)
    if bias is None and x.dim() == 2 and x.dtype in HALF_DTYPES:
        cfg = CONFIGS.get((x.shape[0], weight.shape[0], weight.shape[1]))
        if cfg is not None:
            return hip_linear(x, weight, cfg)
    return F.linear(x, weight, bias)


def _default_gemm(layer, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    if weight in _released:
        return released_linear(x, weight, bias)
    return F.linear(x, weight, bias)


# The build's own dispatch slot, standing in for vLLM's where vLLM is absent.
default_unquantized_gemm = _default_gemm


def dispatch_unquantized_gemm():
    """The GEMM currently installed in the build's slot (vLLM's ``dispatch_unquantized_gemm()``)."""
    return default_unquantized_gemm


def install(configs: dict[tuple[int, int, int], Config]) -> None:
    """Route unquantized GEMMs with a configured ``(M, N, K)`` through the HIP kernel.

    Loads the kernel library first (raising if it is not built) and rejects tiles the library has
    no kernel for, so a bad table fails here rather than at the first call."""
    global default_unquantized_gemm
    lib = _lib.lib()
    for (M, N, K), cfg in configs.items():
        if not lib.plm_gemm_packed_tile_supported(_lib.PLM_BF16, M, K, _tile(cfg)):
            raise ValueError(f"no compiled MI355X kernel for tile {cfg} at (M={M}, N={N}, K={K})")
    CONFIGS.update(configs)
    default_unquantized_gemm = fast_gemm
    try:
        import vllm.model_executor.layers.utils as vllm_utils
    except ImportError:
        return
    vllm_utils.default_unquantized_gemm = fast_gemm


def uninstall() -> None:
    """Restore ``F.linear`` in the build's slot and forget every configured shape."""
    global default_unquantized_gemm
    CONFIGS.clear()
    ACT_CONFIGS.clear()
    default_unquantized_gemm = _default_gemm
