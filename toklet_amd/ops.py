"""Device attention operators with the reference's operator interface.

Each function mirrors one toklet operator (same names, shape structs,
argument meaning and error behaviour) and calls libtokhip through its C ABI.
Tensors are torch tensors in device memory; torch supplies allocation and
the stream, the kernels are the library's.

    toklet                                   this module
    cpu::attention_cached (attention.rs:201)  attention_cached
    cpu::attention        (attention.rs:85)   attention
    cpu::window_attention (window_attention.rs:36)  window_attention
    cpu::span_attention   (span_attention.rs:42)    span_attention
    cpu::logit_softcap    (softcap.rs:16)     logit_softcap

Errors raise :class:`TkhError` carrying the code of the matching
``toklet::cpu::Error`` variant.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


class TkhError(Exception):
    def __init__(self, err: _lib.Error):
        self.code = int(err.code)
        self.name = _lib.CODE_NAMES.get(self.code, str(self.code))
        self.tensor = err.tensor.decode(errors="replace")
        self.index = int(err.index)
        self.expected = int(err.expected)
        self.actual = int(err.actual)
        self.message = err.message.decode(errors="replace")
        super().__init__(f"{self.name}: {self.message}")


def _check(rc: int, err: _lib.Error):
    if rc != _lib.OK:
        raise TkhError(err)


class Context:
    """One device stream, workspace and status word (tkh_context)."""

    def __init__(self, device: int = 0, stream: Optional[torch.cuda.Stream] = None,
                 workspace_bytes: int = 0, synchronous: bool = True):
        lib = _lib.load()
        if stream is None:
            stream = torch.cuda.current_stream(device)
        self.device = device
        self.torch_stream = stream
        handle = ctypes.c_void_p()
        err = _lib.Error()
        _check(lib.tkh_context_create(device, ctypes.c_void_p(stream.cuda_stream), workspace_bytes,
                                      int(synchronous), ctypes.byref(handle), ctypes.byref(err)), err)
        self.handle = handle
        _lib.track(self, _lib.CONTEXT)

    def synchronize(self):
        err = _lib.Error()
        _check(_lib.load().tkh_context_synchronize(self.handle, ctypes.byref(err)), err)

    def profile(self, enable: bool = True):
        """Start (and zero) or stop per-launch HIP-event timing of the kernels."""
        err = _lib.Error()
        _check(_lib.load().tkh_context_profile(self.handle, int(enable), ctypes.byref(err)), err)

    def profile_read(self) -> dict:
        """{'launches', 'attention_ms', 'combine_ms'} summed since profile(True)."""
        out = _lib.Profile()
        err = _lib.Error()
        _check(_lib.load().tkh_context_profile_read(self.handle, ctypes.byref(out),
                                                    ctypes.byref(err)), err)
        return {"launches": int(out.launches), "attention_ms": float(out.attention_ms),
                "combine_ms": float(out.combine_ms)}

    def close(self):
        if getattr(self, "handle", None):
            _lib.load().tkh_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- shape structs (reference field names) ----

@dataclass
class CachedAttentionShape:
    """src/cpu/attention.rs:180-189"""
    tokens: int
    query_heads: int
    kv_heads: int
    head_dim: int
    capacity: int
    offset: int


@dataclass
class AttentionShape:
    """src/cpu/attention.rs:67-72"""
    tokens: int
    query_heads: int
    kv_heads: int
    head_dim: int


@dataclass
class WindowAttentionShape:
    """src/cpu/window_attention.rs:6-17, plus the score softcap (0 disables)."""
    queries: int
    keys: int
    capacity: int
    query_heads: int
    kv_heads: int
    head_dim: int
    query_start: int
    key_start: int
    window: Optional[int]
    scale: float
    softcap: float = 0.0


@dataclass
class AttentionKvSegment:
    """src/cpu/span_attention.rs:9-16 (k/v are device tensors or None when keys == 0)."""
    k: Optional[torch.Tensor]
    v: Optional[torch.Tensor]
    keys: int
    head_stride: int
    key_start: int


@dataclass
class SpanAttentionShape:
    """src/cpu/span_attention.rs:18-28, plus the score softcap."""
    queries: int
    keys: int
    query_heads: int
    kv_heads: int
    head_dim: int
    query_start: int
    key_start: int
    window: Optional[int]
    scale: float
    softcap: float = 0.0


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p()


def _fptr(t: Optional[torch.Tensor]):
    if t is None:
        return ctypes.cast(None, _lib.fptr)
    if t.dtype != torch.float32:
        raise TypeError("outputs are float32 tensors")
    return ctypes.cast(t.data_ptr(), _lib.fptr)


def _n(t: Optional[torch.Tensor]) -> int:
    return t.numel() if t is not None else 0


def dtype_of(*tensors: torch.Tensor) -> int:
    dts = {t.dtype for t in tensors if t is not None}
    if len(dts) != 1:
        raise TypeError(f"q/k/v must share one dtype, got {dts}")
    (dt,) = dts
    if dt not in _DTYPES:
        raise TypeError(f"unsupported dtype {dt}")
    return _DTYPES[dt]


def _window(window):
    return (0, 0) if window is None else (1, int(window))


def attention_cached(ctx: Context, q, k, v, context, scores, probabilities,
                     shape: CachedAttentionShape):
    """Chunk queries over a head-major cache (reference: attention_cached)."""
    err = _lib.Error()
    s = _lib.CachedShape(shape.tokens, shape.query_heads, shape.kv_heads, shape.head_dim,
                         shape.capacity, shape.offset)
    rc = _lib.load().tkh_attention_cached(
        ctx.handle, ctypes.byref(s), dtype_of(q, k, v), _ptr(q), _n(q), _ptr(k), _n(k), _ptr(v),
        _n(v), _fptr(context), _n(context), _fptr(scores), _n(scores), _fptr(probabilities),
        _n(probabilities), ctypes.byref(err))
    _check(rc, err)


def attention_cached_static(device: int, q, k, v, context, shape: CachedAttentionShape,
                            stream: Optional[torch.cuda.Stream] = None,
                            status: Optional[torch.Tensor] = None):
    """attention_cached without a context or any allocation: split-K partials in
    the library's fixed per-GPU scratch (tkh_attention_cached_static).  `status`:
    an int32 device tensor of one element the kernels OR their status bits into
    (the call then returns once queued), or None to wait and raise on failure."""
    err = _lib.Error()
    s = _lib.CachedShape(shape.tokens, shape.query_heads, shape.kv_heads, shape.head_dim,
                         shape.capacity, shape.offset)
    if stream is None:
        stream = torch.cuda.current_stream(device)
    st = ctypes.cast(status.data_ptr(), ctypes.POINTER(ctypes.c_uint32)) if status is not None else None
    rc = _lib.load().tkh_attention_cached_static(
        device, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(s), dtype_of(q, k, v), _ptr(q),
        _n(q), _ptr(k), _n(k), _ptr(v), _n(v), _fptr(context), _n(context), st, ctypes.byref(err))
    _check(rc, err)


def attention(ctx: Context, q, k, v, context, scores, probabilities, shape: AttentionShape):
    """Full-prefix causal GQA with token-major K/V (reference: attention)."""
    err = _lib.Error()
    s = _lib.AttentionShape(shape.tokens, shape.query_heads, shape.kv_heads, shape.head_dim)
    rc = _lib.load().tkh_attention(
        ctx.handle, ctypes.byref(s), dtype_of(q, k, v), _ptr(q), _n(q), _ptr(k), _n(k), _ptr(v),
        _n(v), _fptr(context), _n(context), _fptr(scores), _n(scores), _fptr(probabilities),
        _n(probabilities), ctypes.byref(err))
    _check(rc, err)


def window_attention(ctx: Context, q, k, v, context, scores, probabilities,
                     shape: WindowAttentionShape):
    """Causal/sliding GQA with explicit scale (reference: window_attention)."""
    err = _lib.Error()
    hw, w = _window(shape.window)
    s = _lib.WindowShape(shape.queries, shape.keys, shape.capacity, shape.query_heads,
                         shape.kv_heads, shape.head_dim, shape.query_start, shape.key_start, hw, w,
                         shape.scale, shape.softcap)
    rc = _lib.load().tkh_window_attention(
        ctx.handle, ctypes.byref(s), dtype_of(q, k, v), _ptr(q), _n(q), _ptr(k), _n(k), _ptr(v),
        _n(v), _fptr(context), _n(context), _fptr(scores), _n(scores), _fptr(probabilities),
        _n(probabilities), ctypes.byref(err))
    _check(rc, err)


def span_attention(ctx: Context, q, segments: Sequence[AttentionKvSegment], context, scores,
                   probabilities, shape: SpanAttentionShape):
    """GQA over <=2 old ring spans plus the staged chunk (reference: span_attention)."""
    err = _lib.Error()
    segs = (_lib.Segment * 3)()
    tensors = [q] + [t for sg in segments for t in (sg.k, sg.v) if t is not None]
    for i, sg in enumerate(segments):
        segs[i] = _lib.Segment(_ptr(sg.k).value, _n(sg.k), _ptr(sg.v).value, _n(sg.v), sg.keys,
                               sg.head_stride, sg.key_start)
    hw, w = _window(shape.window)
    s = _lib.SpanShape(shape.queries, shape.keys, shape.query_heads, shape.kv_heads,
                       shape.head_dim, shape.query_start, shape.key_start, hw, w, shape.scale,
                       shape.softcap)
    rc = _lib.load().tkh_span_attention(
        ctx.handle, ctypes.byref(s), dtype_of(*tensors), _ptr(q), _n(q), segs, _fptr(context),
        _n(context), _fptr(scores), _n(scores), _fptr(probabilities), _n(probabilities),
        ctypes.byref(err))
    _check(rc, err)


def project_greedy(ctx: Context, context: torch.Tensor, weights: torch.Tensor,
                   tokens: torch.Tensor, logits: Optional[torch.Tensor] = None):
    """The o-projection of FP32 context rows [rows, hidden] by weights [vocab, hidden]
    in the reference matmul's FP32 order, then the greedy token of each row
    (reference: cpu::matmul + sampling::greedy).  tokens: int32 device tensor
    [rows] (holding the uint32 ids); logits: optional FP32 [rows, vocab]."""
    err = _lib.Error()
    rows, hidden = context.shape[0], context.shape[-1]
    vocab = weights.shape[0]
    if tokens.dtype != torch.int32:
        raise TypeError("tokens is an int32 tensor (uint32 ids)")
    tok = ctypes.cast(tokens.data_ptr(), ctypes.POINTER(ctypes.c_uint32))
    rc = _lib.load().tkh_project_greedy(
        ctx.handle, rows, hidden, vocab, _fptr(context), _n(context), _fptr(weights), _n(weights),
        _fptr(logits), _n(logits), tok, _n(tokens), ctypes.byref(err))
    _check(rc, err)


def logit_softcap(ctx: Context, logits: torch.Tensor, cap: float):
    """In-place cap*tanh(x/cap) in FP64 rounded to FP32 (reference: logit_softcap)."""
    err = _lib.Error()
    rc = _lib.load().tkh_logit_softcap(ctx.handle, _fptr(logits), _n(logits), cap,
                                       ctypes.byref(err))
    _check(rc, err)


def _u64s(values):
    arr = (ctypes.c_uint64 * len(values))(*[int(x) for x in values])
    return arr


def decode_batch(ctx: Context, q, k_base, v_base, offsets, head_strides, lengths, context, *,
                 query_heads: int, kv_heads: int, head_dim: int, scale: float):
    """One query token per session over its own head-major cache (tkh_decode_batch)."""
    err = _lib.Error()
    batch = len(lengths)
    rc = _lib.load().tkh_decode_batch(
        ctx.handle, batch, query_heads, kv_heads, head_dim, dtype_of(q, k_base, v_base), _ptr(q),
        _ptr(k_base), _ptr(v_base), _u64s(offsets), _u64s(head_strides), _u64s(lengths), scale,
        _fptr(context), ctypes.byref(err))
    _check(rc, err)


def prefill_batch(ctx: Context, q, k_base, v_base, offsets, head_strides, positions, context, *,
                  tokens: int, query_heads: int, kv_heads: int, head_dim: int, scale: float):
    """A causal chunk of `tokens` queries per session at cache offset positions[b]."""
    err = _lib.Error()
    batch = len(positions)
    rc = _lib.load().tkh_prefill_batch(
        ctx.handle, batch, tokens, query_heads, kv_heads, head_dim, dtype_of(q, k_base, v_base),
        _ptr(q), _ptr(k_base), _ptr(v_base), _u64s(offsets), _u64s(head_strides),
        _u64s(positions), scale, _fptr(context), ctypes.byref(err))
    _check(rc, err)


# ---- producer: the step before attention (Model::run, src/model/mod.rs:611-662) ----

ROTARY_NONE, ROTARY_SPLIT_HALF, ROTARY_PROPORTIONAL, ROTARY_LLAMA3 = 0, 1, 2, 3


@dataclass
class ProducerShape:
    """Per-layer producer geometry: norm epsilon, rotary kind and its parameters
    (split-half theta; proportional base / rotated_dims / factor; Llama 3 theta,
    factor, low/high frequency factors and original context length, as
    Llama3Scaling::new takes them, src/cpu/llama3_rotary.rs:14-37)."""
    tokens: int
    query_heads: int
    kv_heads: int
    head_dim: int
    position: int
    norm_epsilon: float = 1e-6
    rotary: int = ROTARY_SPLIT_HALF
    theta: float = 1e6
    rotated_dims: int = 0
    factor: float = 1.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_positions: int = 8192

    def c(self):
        return _lib.ProducerShape(self.tokens, self.query_heads, self.kv_heads, self.head_dim,
                                  self.position, self.norm_epsilon, self.rotary, self.theta,
                                  self.rotated_dims, self.factor, self.low_freq_factor,
                                  self.high_freq_factor, self.original_max_positions)


def produce_qkv(ctx: Context, shape: ProducerShape, q_proj, k_proj, v_proj, q_norm, k_norm,
                q_out, k_out, v_out, out_head_stride: int):
    """rmsnorm (optional) -> rotary -> rounding of Q, and the K/V append into head-major
    rows, in one launch.  k_out/v_out may be views into a cache at a row offset."""
    err = _lib.Error()
    s = shape.c()
    rc = _lib.load().tkh_produce_qkv(
        ctx.handle, ctypes.byref(s), dtype_of(q_out, k_out, v_out), _ptr(q_proj), _ptr(k_proj),
        _ptr(v_proj), _ptr(q_norm), _ptr(k_norm), _ptr(q_out), _ptr(k_out), _ptr(v_out),
        out_head_stride, ctypes.byref(err))
    _check(rc, err)
