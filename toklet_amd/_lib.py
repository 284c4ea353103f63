"""ctypes declarations of libtokhip.so (include/tokhip.h).

The library is loaded from this package directory only.  A missing library is
an error: there is no CPU fallback behind these bindings.
"""

from __future__ import annotations

import atexit
import ctypes
import os
import weakref

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtokhip.so")

u32, u64, f32, vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
fptr = ctypes.POINTER(ctypes.c_float)

CODE_NAMES = {
    0: "Ok", 1: "ZeroDimension", 2: "SizeOverflow", 3: "Length", 4: "Token", 5: "NonFinite",
    6: "InvalidParameter", 7: "FullyMasked", 8: "Capacity", 9: "InvalidConfig", 10: "Device",
    11: "Unsupported",
}
OK, ZERO_DIMENSION, SIZE_OVERFLOW, LENGTH, TOKEN, NON_FINITE, INVALID_PARAMETER, FULLY_MASKED, \
    CAPACITY, INVALID_CONFIG, DEVICE, UNSUPPORTED = range(12)
F32, F16, BF16 = 0, 1, 2


class Error(ctypes.Structure):
    _fields_ = [("code", u32), ("index", u64), ("expected", u64), ("actual", u64),
                ("tensor", ctypes.c_char * 64), ("message", ctypes.c_char * 256)]


class CachedShape(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("tokens", "query_heads", "kv_heads", "head_dim", "capacity", "offset")]


class AttentionShape(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("tokens", "query_heads", "kv_heads", "head_dim")]


class WindowShape(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("queries", "keys", "capacity", "query_heads", "kv_heads",
                                   "head_dim", "query_start", "key_start")] + [
        ("has_window", u32), ("window", u64), ("scale", f32), ("softcap", f32)]


class Segment(ctypes.Structure):
    _fields_ = [("k", vp), ("k_len", u64), ("v", vp), ("v_len", u64), ("keys", u64),
                ("head_stride", u64), ("key_start", u64)]


class SpanShape(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("queries", "keys", "query_heads", "kv_heads", "head_dim",
                                   "query_start", "key_start")] + [
        ("has_window", u32), ("window", u64), ("scale", f32), ("softcap", f32)]


class KvInfo(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("heads", "dims", "capacity", "max_positions", "window",
                                   "offset", "generation", "owner")] + [
        ("has_window", u32), ("storage", ctypes.c_int), ("k", vp), ("v", vp),
        ("allocated_bytes", u64)]


class Profile(ctypes.Structure):
    _fields_ = [("launches", u64), ("attention_ms", ctypes.c_double), ("combine_ms", ctypes.c_double)]


class KvFrame(ctypes.Structure):
    _fields_ = [("k", vp), ("v", vp), ("owner", u64), ("generation", u64), ("offset", u64),
                ("tokens", u64)]


# TKH_ABI_VERSION of include/tokhip.h that the structures below mirror.
ABI_VERSION = 2


class ProducerShape(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("tokens", "query_heads", "kv_heads", "head_dim", "position")] + [
        ("norm_epsilon", f32), ("rotary", u32), ("theta", f32), ("rotated_dims", u64),
        ("factor", f32), ("low_freq_factor", f32), ("high_freq_factor", f32),
        ("original_max_positions", u64)]


class SessionOptions(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("capacity", "prefill_chunk_size", "position_offset",
                                   "vocab_size", "layers", "query_heads", "kv_heads",
                                   "head_dim")] + [
        ("storage", ctypes.c_int), ("score_scale", f32), ("softcap", f32), ("norm_epsilon", f32),
        ("rotary", u32), ("theta", f32), ("rotated_dims", u64), ("factor", f32),
        ("low_freq_factor", f32), ("high_freq_factor", f32), ("original_max_positions", u64),
        ("shared_layers", u64)]


class SessionState(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("history_len", "evaluated_len", "pending_len", "capacity")] + [
        ("distribution_valid", u32), ("kv_bytes", u64), ("scratch_bytes", u64)]


class LayerIo(ctypes.Structure):
    _fields_ = [(n, vp) for n in ("q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "context")]


P = ctypes.POINTER
E = P(Error)

SIGNATURES = {
    "tkh_abi_version": (u32, []),
    "tkh_context_create": (u32, [ctypes.c_int, vp, ctypes.c_size_t, ctypes.c_int, P(vp), E]),
    "tkh_context_destroy": (None, [vp]),
    "tkh_context_synchronize": (u32, [vp, E]),
    "tkh_context_stream": (vp, [vp]),
    "tkh_context_profile": (u32, [vp, ctypes.c_int, E]),
    "tkh_context_profile_read": (u32, [vp, P(Profile), E]),
    "tkh_attention_cached": (u32, [vp, P(CachedShape), ctypes.c_int, vp, u64, vp, u64, vp, u64,
                                   fptr, u64, fptr, u64, fptr, u64, E]),
    "tkh_attention_cached_static": (u32, [ctypes.c_int, vp, P(CachedShape), ctypes.c_int, vp, u64,
                                          vp, u64, vp, u64, fptr, u64, P(u32), E]),
    "tkh_attention": (u32, [vp, P(AttentionShape), ctypes.c_int, vp, u64, vp, u64, vp, u64, fptr,
                            u64, fptr, u64, fptr, u64, E]),
    "tkh_window_attention": (u32, [vp, P(WindowShape), ctypes.c_int, vp, u64, vp, u64, vp, u64,
                                   fptr, u64, fptr, u64, fptr, u64, E]),
    "tkh_span_attention": (u32, [vp, P(SpanShape), ctypes.c_int, vp, u64, P(Segment), fptr, u64,
                                 fptr, u64, fptr, u64, E]),
    "tkh_project_greedy": (u32, [vp, u64, u64, u64, fptr, u64, fptr, u64, fptr, u64, P(u32), u64,
                                 E]),
    "tkh_logit_softcap": (u32, [vp, fptr, u64, f32, E]),
    "tkh_decode_batch": (u32, [vp, u64, u64, u64, u64, ctypes.c_int, vp, vp, vp, P(u64), P(u64),
                               P(u64), f32, fptr, E]),
    "tkh_prefill_batch": (u32, [vp, u64, u64, u64, u64, u64, ctypes.c_int, vp, vp, vp, P(u64),
                                P(u64), P(u64), f32, fptr, E]),
    "tkh_kv_planned_bytes": (u32, [u64, u64, u64, u32, u64, ctypes.c_int, u64, P(u64), E]),
    "tkh_kv_create": (u32, [vp, u64, u64, u64, u64, u32, u64, ctypes.c_int, P(vp), E]),
    "tkh_kv_destroy": (None, [vp]),
    "tkh_kv_info_get": (u32, [vp, P(KvInfo)]),
    "tkh_kv_append": (u32, [vp, u64, u64, ctypes.c_int, vp, vp, E]),
    "tkh_kv_prepare": (u32, [vp, vp, u64, vp, u64, u64, P(KvFrame), E]),
    "tkh_kv_view": (u32, [vp, P(KvFrame), u64, f32, P(Segment), P(SpanShape), E]),
    "tkh_kv_commit_batch": (u32, [P(vp), P(KvFrame), u64, E]),
    "tkh_kv_reset_batch": (u32, [P(vp), u64, E]),
    "tkh_produce_qkv": (u32, [vp, P(ProducerShape), ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp,
                              u64, E]),
    "tkh_session_create": (u32, [vp, P(SessionOptions), P(u64), P(vp), E]),
    "tkh_session_destroy": (None, [vp]),
    "tkh_session_append": (u32, [vp, P(u32), u64, E]),
    "tkh_session_set_tokens": (u32, [vp, P(u32), u64, E]),
    "tkh_session_discard_pending": (None, [vp]),
    "tkh_session_reset": (None, [vp]),
    "tkh_session_state_get": (u32, [vp, P(SessionState)]),
    "tkh_session_history": (u64, [vp, P(u32), u64]),
    "tkh_session_kv_producer": (u32, [vp, u64, P(u64)]),
    "tkh_session_chunk_begin": (u32, [vp, u64, P(u64), P(u64), E]),
    "tkh_session_chunk_layer": (u32, [vp, u64, P(LayerIo), E]),
    "tkh_session_chunk_commit": (u32, [vp, P(u64), E]),
    "tkh_session_chunk_abort": (None, [vp]),
    "tkh_session_next_chunk": (u32, [vp, P(u64), P(u64)]),
    "tkh_session_evaluate_next_chunk": (u32, [vp, P(LayerIo), P(u64), E]),
    "tkh_session_evaluate": (u32, [vp, P(LayerIo), u64, P(u64), E]),
    "tkh_session_synchronize": (u32, [vp, E]),
}

_lib = None


def load():
    """Load libtokhip.so from this package (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m toklet_amd.build` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.tkh_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {lib.tkh_abi_version()}, these "
                               f"bindings expect {ABI_VERSION}: rebuild it")
        _lib = lib
    return _lib


# Handles still open when the interpreter exits are closed here, before the
# HIP runtime's own teardown: sessions, then KV owners, then contexts (an
# object kept alive only by a reference cycle would otherwise be finalised
# after the runtime is gone).
_live = {0: weakref.WeakSet(), 1: weakref.WeakSet(), 2: weakref.WeakSet()}
SESSION, KV_OWNER, CONTEXT = 0, 1, 2


def track(obj, order: int):
    _live[order].add(obj)


@atexit.register
def _close_all():
    for order in (SESSION, KV_OWNER, CONTEXT):
        for obj in list(_live[order]):
            try:
                obj.close()
            except Exception:
                pass
