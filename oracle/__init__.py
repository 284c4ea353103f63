"""ctypes view of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY.  This module is imported by tests/, by
``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of ``bench.py`` as
the parity checker.  The product package ``toklet_amd`` never imports it.

Each wrapper takes float32 numpy arrays (slices carry their own lengths, as
the reference's Rust slices do) and either returns the outputs or raises
:class:`OracleError` with the code and payload of the matching
``toklet::cpu::Error`` variant (src/cpu/mod.rs:47-68).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

OK, ZERO_DIMENSION, SIZE_OVERFLOW, LENGTH, TOKEN, NON_FINITE, INVALID_PARAMETER, FULLY_MASKED = range(8)
CODE_NAMES = {
    0: "Ok", 1: "ZeroDimension", 2: "SizeOverflow", 3: "Length", 4: "Token",
    5: "NonFinite", 6: "InvalidParameter", 7: "FullyMasked",
}

_size = ctypes.c_size_t
_fp = ctypes.POINTER(ctypes.c_float)


class _Error(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint32), ("tensor", ctypes.c_char_p), ("index", _size),
                ("expected", _size), ("actual", _size)]


class _AttentionShape(ctypes.Structure):
    _fields_ = [(n, _size) for n in ("tokens", "query_heads", "kv_heads", "head_dim")]


class _CachedShape(ctypes.Structure):
    _fields_ = [(n, _size) for n in ("tokens", "query_heads", "kv_heads", "head_dim", "capacity", "offset")]


class _WindowShape(ctypes.Structure):
    _fields_ = [(n, _size) for n in ("queries", "keys", "capacity", "query_heads", "kv_heads",
                                     "head_dim", "query_start", "key_start")] + [
        ("has_window", ctypes.c_int), ("window", _size), ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float)]


class _Segment(ctypes.Structure):
    _fields_ = [("k", _fp), ("k_len", _size), ("v", _fp), ("v_len", _size), ("keys", _size),
                ("head_stride", _size), ("key_start", _size)]


class _SpanShape(ctypes.Structure):
    _fields_ = [(n, _size) for n in ("queries", "keys", "query_heads", "kv_heads", "head_dim",
                                     "query_start", "key_start")] + [
        ("has_window", ctypes.c_int), ("window", _size), ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float)]


class OracleError(Exception):
    def __init__(self, err: _Error):
        self.code = err.code
        self.name = CODE_NAMES.get(err.code, str(err.code))
        self.tensor = err.tensor.decode() if err.tensor else None
        self.index = err.index
        self.expected = err.expected
        self.actual = err.actual
        super().__init__(f"{self.name}(tensor={self.tensor}, index={self.index}, "
                         f"expected={self.expected}, actual={self.actual})")


def build() -> str:
    """Compile liboracle.so from oracle.c (gcc, -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_view_start.restype = _size
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_fp) if a.size else ctypes.cast(None, _fp)


def _check(rc: int, err: _Error):
    if rc != OK:
        raise OracleError(err)


def rotary(x, tokens, heads, head_dim, offset, theta):
    x = _f32(x)
    out = np.zeros_like(x)
    err = _Error()
    rc = lib().orc_rotary(_ptr(x), _size(x.size), _ptr(out), _size(out.size), _size(tokens),
                          _size(heads), _size(head_dim), _size(offset), ctypes.c_float(theta),
                          ctypes.byref(err))
    _check(rc, err)
    return out


def proportional_rotary(x, tokens, heads, head_dim, rotated_dims, offset, base, factor):
    x = _f32(x)
    out = np.zeros_like(x)
    err = _Error()
    rc = lib().orc_proportional_rotary(
        _ptr(x), _size(x.size), _ptr(out), _size(out.size), _size(tokens), _size(heads),
        _size(head_dim), _size(rotated_dims), _size(offset), ctypes.c_float(base),
        ctypes.c_float(factor), ctypes.byref(err))
    _check(rc, err)
    return out


class _Llama3(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("factor", "low", "high", "original")]


def llama3_scaling(factor, low, high, original):
    """Llama3Scaling::new (src/cpu/llama3_rotary.rs:14-37)."""
    s, err = _Llama3(), _Error()
    rc = lib().orc_llama3_scaling(ctypes.c_float(factor), ctypes.c_float(low), ctypes.c_float(high),
                                  _size(original), ctypes.byref(s), ctypes.byref(err))
    _check(rc, err)
    return s


def llama3_inverse_frequency(scaling, ordinary):
    """Llama3Scaling::inverse_frequency (src/cpu/llama3_rotary.rs:44-61), FP64."""
    out, err = ctypes.c_double(), _Error()
    rc = lib().orc_llama3_inverse_frequency(ctypes.byref(scaling), ctypes.c_double(ordinary),
                                            ctypes.byref(out), ctypes.byref(err))
    _check(rc, err)
    return out.value


def llama3_rotary(x, tokens, heads, head_dim, offset, theta, factor, low, high, original):
    """llama3_rotary (src/cpu/llama3_rotary.rs:87-146)."""
    s = llama3_scaling(factor, low, high, original)
    x = _f32(x)
    out = np.zeros_like(x)
    err = _Error()
    rc = lib().orc_llama3_rotary(
        _ptr(x), _size(x.size), _ptr(out), _size(out.size), _size(tokens), _size(heads),
        _size(head_dim), _size(offset), ctypes.c_float(theta), ctypes.byref(s), ctypes.byref(err))
    _check(rc, err)
    return out


def rmsnorm(x, weight, tokens, hidden, epsilon):
    x, weight = _f32(x), _f32(weight)
    out = np.zeros_like(x)
    err = _Error()
    rc = lib().orc_rmsnorm(_ptr(x), _size(x.size), _ptr(weight), _size(weight.size), _ptr(out),
                           _size(out.size), _size(tokens), _size(hidden), ctypes.c_float(epsilon),
                           ctypes.byref(err))
    _check(rc, err)
    return out


def softmax(scores, rows, columns, mask=None):
    scores = _f32(scores)
    out = np.zeros_like(scores)
    err = _Error()
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        mp, ml = m.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), _size(m.size)
    else:
        mp, ml = ctypes.cast(None, ctypes.POINTER(ctypes.c_uint8)), _size(0)
    rc = lib().orc_softmax(_ptr(scores), _size(scores.size), mp, ml, _ptr(out), _size(out.size),
                           _size(rows), _size(columns), ctypes.byref(err))
    _check(rc, err)
    return out


def attention(q, k, v, tokens, query_heads, kv_heads, head_dim, out=None):
    """Full-prefix causal GQA (src/cpu/attention.rs:85-178).

    Returns (context, scores, probabilities) with the reference layouts.
    ``out`` may pass preallocated (context, scores, probabilities) buffers, to
    observe that nothing is written on a validation error.
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    if out is None:
        out = (np.zeros(tokens * query_heads * head_dim, np.float32),
               np.zeros(query_heads * tokens * tokens, np.float32),
               np.zeros(query_heads * tokens * tokens, np.float32))
    ctx, sc, pr = out
    shape = _AttentionShape(tokens, query_heads, kv_heads, head_dim)
    err = _Error()
    rc = lib().orc_attention(_ptr(q), _size(q.size), _ptr(k), _size(k.size), _ptr(v),
                             _size(v.size), _ptr(ctx), _size(ctx.size), _ptr(sc), _size(sc.size),
                             _ptr(pr), _size(pr.size), ctypes.byref(shape), ctypes.byref(err))
    _check(rc, err)
    return ctx, sc, pr


def attention_cached(q, k, v, tokens, query_heads, kv_heads, head_dim, capacity, offset,
                     out=None):
    """Chunk attention over a head-major cache (src/cpu/attention.rs:201-296).

    Returns (context, scores, probabilities); scores/probabilities are the
    reusable ``[capacity]`` rows left by the last (head, query).
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    if out is None:
        out = (np.zeros(tokens * query_heads * head_dim, np.float32),
               np.zeros(capacity, np.float32), np.zeros(capacity, np.float32))
    ctx, sc, pr = out
    shape = _CachedShape(tokens, query_heads, kv_heads, head_dim, capacity, offset)
    err = _Error()
    rc = lib().orc_attention_cached(_ptr(q), _size(q.size), _ptr(k), _size(k.size), _ptr(v),
                                    _size(v.size), _ptr(ctx), _size(ctx.size), _ptr(sc),
                                    _size(sc.size), _ptr(pr), _size(pr.size), ctypes.byref(shape),
                                    ctypes.byref(err))
    _check(rc, err)
    return ctx, sc, pr


def _window(window):
    return (0, 0) if window is None else (1, int(window))


def window_attention(q, k, v, queries, keys, capacity, query_heads, kv_heads, head_dim,
                     query_start, key_start, window, scale, softcap=0.0, out=None):
    """Causal/sliding GQA with explicit scale (src/cpu/window_attention.rs:36-168)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    n = query_heads * queries * keys
    if out is None:
        out = (np.zeros(queries * query_heads * head_dim, np.float32), np.zeros(n, np.float32),
               np.zeros(n, np.float32))
    ctx, sc, pr = out
    hw, w = _window(window)
    shape = _WindowShape(queries, keys, capacity, query_heads, kv_heads, head_dim, query_start,
                         key_start, hw, w, scale, softcap)
    err = _Error()
    rc = lib().orc_window_attention(_ptr(q), _size(q.size), _ptr(k), _size(k.size), _ptr(v),
                                    _size(v.size), _ptr(ctx), _size(ctx.size), _ptr(sc),
                                    _size(sc.size), _ptr(pr), _size(pr.size), ctypes.byref(shape),
                                    ctypes.byref(err))
    _check(rc, err)
    return ctx, sc, pr


@dataclass
class Segment:
    """One logical key interval (src/cpu/span_attention.rs:9-16)."""
    k: np.ndarray
    v: np.ndarray
    keys: int
    head_stride: int
    key_start: int


def span_attention(q, segments, queries, keys, query_heads, kv_heads, head_dim, query_start,
                   key_start, window, scale, softcap=0.0, out=None):
    """GQA over <=2 old ring spans plus a new chunk (src/cpu/span_attention.rs:42-220)."""
    q = _f32(q)
    n = query_heads * queries * keys
    if out is None:
        out = (np.zeros(queries * query_heads * head_dim, np.float32), np.zeros(n, np.float32),
               np.zeros(n, np.float32))
    ctx, sc, pr = out
    segs = (_Segment * 3)()
    keep = []
    for i, seg in enumerate(segments):
        sk, sv = _f32(seg.k), _f32(seg.v)
        keep += [sk, sv]
        segs[i] = _Segment(_ptr(sk), sk.size, _ptr(sv), sv.size, seg.keys, seg.head_stride,
                           seg.key_start)
    hw, w = _window(window)
    shape = _SpanShape(queries, keys, query_heads, kv_heads, head_dim, query_start, key_start,
                       hw, w, scale, softcap)
    err = _Error()
    rc = lib().orc_span_attention(_ptr(q), _size(q.size), segs, _ptr(ctx), _size(ctx.size),
                                  _ptr(sc), _size(sc.size), _ptr(pr), _size(pr.size),
                                  ctypes.byref(shape), ctypes.byref(err))
    _check(rc, err)
    return ctx, sc, pr


def logit_softcap(logits, cap):
    x = _f32(logits).copy()
    err = _Error()
    rc = lib().orc_logit_softcap(_ptr(x), _size(x.size), ctypes.c_float(cap), ctypes.byref(err))
    _check(rc, err)
    return x


def view_start(offset, window):
    hw, w = _window(window)
    return int(lib().orc_view_start(_size(offset), ctypes.c_int(hw), _size(w)))


def old_spans(capacity, offset, window):
    out = (_size * 6)()
    hw, w = _window(window)
    lib().orc_old_spans(_size(capacity), _size(offset), ctypes.c_int(hw), _size(w), out)
    return [(out[0], out[1], out[2]), (out[3], out[4], out[5])]


def copy_runs(capacity, offset, tokens, sliding):
    out = (_size * 6)()
    lib().orc_copy_runs(_size(capacity), _size(offset), _size(tokens), ctypes.c_int(int(sliding)),
                        out)
    return [(out[0], out[1], out[2]), (out[3], out[4], out[5])]


def matmul(x, weights, tokens, in_features, out_features, bias=None, out=None):
    """FP32 projection [tokens, in] x [out, in]^T (+ bias) (src/cpu/mod.rs:183-247)."""
    x, w = _f32(x), _f32(weights)
    b = _f32(bias) if bias is not None else None
    if out is None:
        out = np.zeros(tokens * out_features, np.float32)
    err = _Error()
    rc = lib().orc_matmul(_ptr(x), _size(x.size), _ptr(w), _size(w.size),
                          _ptr(b) if b is not None else None, _size(b.size if b is not None else 0),
                          _ptr(out), _size(out.size), _size(tokens), _size(in_features),
                          _size(out_features), ctypes.byref(err))
    _check(rc, err)
    return out


def greedy(logits):
    x = _f32(logits)
    token = ctypes.c_uint32()
    err = _Error()
    rc = lib().orc_greedy(_ptr(x), _size(x.size), ctypes.byref(token), ctypes.byref(err))
    _check(rc, err)
    return int(token.value)
