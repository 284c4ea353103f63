"""Session over device KV: toklet's Session / InferenceSession for the attention path.

Mirrors ``src/session.rs``: the same method names and state transitions
(``append``, ``set_tokens`` with longest-prefix reuse, ``evaluate_next_chunk``,
``evaluate``, ``discard_pending``, ``reset``, ``history``, ``evaluated_len``,
``pending_len``).  What the reference's model computes around attention stays
with the caller: evaluating a chunk takes, per layer, the Q/K/V projections of
the chunk's tokens and returns the attention context.  The state machine and
the per-chunk driver (producer, KV append or ring staging, attention, joint
commit) are native code in libtokhip (``tkh_session_*``).

``Session(None, ...)`` builds a host-only session: its token state machine
runs without a GPU, and evaluation commits state without computing anything.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _lib
from .ops import ROTARY_SPLIT_HALF, Context, TkhError, _check

_STORAGE = {"f32": _lib.F32, "f16": _lib.F16, "bf16": _lib.BF16}


@dataclass
class Options:
    """session::Options (src/session.rs:38-62) plus the attention geometry."""
    capacity: int
    prefill_chunk_size: int = 128
    position_offset: int = 0
    vocab_size: int = 1 << 20
    layers: int = 1
    query_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    storage: str = "bf16"
    score_scale: float = 0.0      # 0: attention_cached semantics (dot / sqrt(D))
    softcap: float = 0.0
    norm_epsilon: float = 1e-6
    rotary: int = ROTARY_SPLIT_HALF
    theta: float = 1e6
    rotated_dims: int = 0
    factor: float = 1.0
    low_freq_factor: float = 1.0       # Llama 3 rotary only
    high_freq_factor: float = 4.0
    original_max_positions: int = 8192
    layer_windows: Optional[Sequence[int]] = None   # per layer, 0 = full
    shared_layers: int = 0   # trailing layers attending over an earlier layer's KV

    def c(self):
        return _lib.SessionOptions(self.capacity, self.prefill_chunk_size, self.position_offset,
                                   self.vocab_size, self.layers, self.query_heads, self.kv_heads,
                                   self.head_dim, _STORAGE[self.storage], self.score_scale,
                                   self.softcap, self.norm_epsilon, self.rotary, self.theta,
                                   self.rotated_dims, self.factor, self.low_freq_factor,
                                   self.high_freq_factor, self.original_max_positions,
                                   self.shared_layers)


@dataclass
class LayerIo:
    """One layer's chunk inputs (FP32 device tensors [rows, H, D]) and context output."""
    q_proj: object
    k_proj: object
    v_proj: object
    context: object
    q_norm: object = None
    k_norm: object = None


def _tokens(tokens):
    arr = (ctypes.c_uint32 * max(1, len(tokens)))(*[int(t) for t in tokens])
    return arr, len(tokens)


def _layers(layers: Sequence[LayerIo]):
    arr = (_lib.LayerIo * len(layers))()
    for i, io in enumerate(layers):
        for name in ("q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "context"):
            t = getattr(io, name)
            setattr(arr[i], name, t.data_ptr() if t is not None else None)
    return arr


class Session:
    def __init__(self, ctx: Optional[Context], options: Options):
        lib = _lib.load()
        self.ctx = ctx
        self.options = options
        handle = ctypes.c_void_p()
        err = _lib.Error()
        o = options.c()
        windows = None
        if options.layer_windows is not None:
            if len(options.layer_windows) != options.layers:
                raise ValueError("layer_windows needs one entry per layer")
            windows = (ctypes.c_uint64 * options.layers)(*[int(w) for w in options.layer_windows])
        _check(lib.tkh_session_create(ctx.handle if ctx is not None else None, ctypes.byref(o),
                                      windows, ctypes.byref(handle), ctypes.byref(err)), err)
        self.handle = handle
        _lib.track(self, _lib.SESSION)

    # ---- state (InferenceSession accessors)
    def _state(self):
        st = _lib.SessionState()
        _lib.load().tkh_session_state_get(self.handle, ctypes.byref(st))
        return st

    def history(self):
        lib = _lib.load()
        n = lib.tkh_session_history(self.handle, None, 0)
        buf = (ctypes.c_uint32 * max(1, n))()
        lib.tkh_session_history(self.handle, buf, n)
        return [int(buf[i]) for i in range(n)]

    def evaluated_len(self) -> int:
        return int(self._state().evaluated_len)

    def pending_len(self) -> int:
        return int(self._state().pending_len)

    def capacity(self) -> int:
        return int(self._state().capacity)

    def distribution_valid(self) -> bool:
        """Session::logits().is_some(): a fully evaluated, nonempty history."""
        return bool(self._state().distribution_valid)

    def memory(self) -> dict:
        st = self._state()
        return {"kv_bytes": int(st.kv_bytes), "scratch_bytes": int(st.scratch_bytes)}

    def kv_producer(self, layer: int) -> int:
        """SharedKvPlan::producer_for (src/model/shared_kv.rs:141-146)."""
        out = ctypes.c_uint64()
        if _lib.load().tkh_session_kv_producer(self.handle, layer, ctypes.byref(out)) != 0:
            raise IndexError(f"layer {layer}")
        return int(out.value)

    def next_chunk(self):
        start, count = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.load().tkh_session_next_chunk(self.handle, ctypes.byref(start), ctypes.byref(count))
        return int(start.value), int(count.value)

    # ---- transitions
    def append(self, tokens):
        err = _lib.Error()
        arr, n = _tokens(tokens)
        _check(_lib.load().tkh_session_append(self.handle, arr, n, ctypes.byref(err)), err)

    def set_tokens(self, tokens):
        err = _lib.Error()
        arr, n = _tokens(tokens)
        _check(_lib.load().tkh_session_set_tokens(self.handle, arr, n, ctypes.byref(err)), err)

    def discard_pending(self):
        _lib.load().tkh_session_discard_pending(self.handle)

    def reset(self):
        _lib.load().tkh_session_reset(self.handle)

    def evaluate_next_chunk(self, layers: Sequence[LayerIo]) -> int:
        """Evaluate the next chunk; `layers` hold chunk-relative rows."""
        err = _lib.Error()
        count = ctypes.c_uint64()
        arr = _layers(layers) if layers is not None else None
        _check(_lib.load().tkh_session_evaluate_next_chunk(self.handle, arr, ctypes.byref(count),
                                                           ctypes.byref(err)), err)
        return int(count.value)

    def evaluate(self, layers: Sequence[LayerIo], chunk_limit: Optional[int] = None) -> int:
        """Evaluate every pending token; `layers` hold rows indexed by session position.
        chunk_limit 1 evaluates them as single-token decode steps."""
        err = _lib.Error()
        done = ctypes.c_uint64()
        limit = chunk_limit or self.options.prefill_chunk_size
        arr = _layers(layers) if layers is not None else None
        _check(_lib.load().tkh_session_evaluate(self.handle, arr, limit, ctypes.byref(done),
                                                ctypes.byref(err)), err)
        return int(done.value)

    # ---- layer-by-layer chunks (the host's model runs between the layers)
    def chunk_begin(self, chunk_limit: Optional[int] = None):
        """Fix the next chunk: (start, count); count 0 when nothing is pending."""
        err = _lib.Error()
        start, count = ctypes.c_uint64(), ctypes.c_uint64()
        limit = chunk_limit or self.options.prefill_chunk_size
        _check(_lib.load().tkh_session_chunk_begin(self.handle, limit, ctypes.byref(start),
                                                   ctypes.byref(count), ctypes.byref(err)), err)
        return int(start.value), int(count.value)

    def chunk_layer(self, layer: int, io: Optional[LayerIo]):
        """Evaluate one layer of the chunk (in order); inputs chunk-relative."""
        err = _lib.Error()
        arr = _layers([io]) if io is not None else (_lib.LayerIo * 1)()
        _check(_lib.load().tkh_session_chunk_layer(self.handle, layer, arr, ctypes.byref(err)), err)

    def chunk_commit(self) -> int:
        err = _lib.Error()
        count = ctypes.c_uint64()
        _check(_lib.load().tkh_session_chunk_commit(self.handle, ctypes.byref(count),
                                                    ctypes.byref(err)), err)
        return int(count.value)

    def chunk_abort(self):
        _lib.load().tkh_session_chunk_abort(self.handle)

    def synchronize(self):
        err = _lib.Error()
        _check(_lib.load().tkh_session_synchronize(self.handle, ctypes.byref(err)), err)

    def close(self):
        if getattr(self, "handle", None):
            _lib.load().tkh_session_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["Options", "LayerIo", "Session", "TkhError"]
