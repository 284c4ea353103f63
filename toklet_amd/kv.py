"""Device-resident KV owners with the reference's KV interfaces.

    toklet                                         this module
    model::KvCache / LayerKv (cache.rs:1-97)       KvCache, LayerKv
    model::WindowKvCache (window_cache.rs:21-350)   WindowKvCache, PreparedKv, KvView
    window_cache::commit_batch / reset_batch         commit_batch, reset_batch
    capacity::KvOwner::at_capacity (capacity.rs:49) planned_bytes

K/V live in HBM as separate head-major [heads, capacity, head_dim] arrays in
the storage dtype (f32, f16 or bf16), allocated once by tkh_kv_create.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional

import torch

from . import _lib
from .ops import (AttentionKvSegment, CachedAttentionShape, Context, SpanAttentionShape,
                  TkhError, _check, _ptr, attention_cached)

_TORCH = {_lib.F32: torch.float32, _lib.F16: torch.float16, _lib.BF16: torch.bfloat16}
_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


class _DeviceView:
    """__cuda_array_interface__ over library-owned device memory."""

    def __init__(self, ptr: int, shape, dtype: torch.dtype):
        typestr = {torch.float32: "<f4", torch.float16: "<f2", torch.bfloat16: "<f2"}[dtype]
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (ptr, False), "version": 2}


def device_tensor(ptr: int, shape, dtype: torch.dtype, device: int) -> torch.Tensor:
    """A torch view (no copy) of `shape` elements at device address `ptr`."""
    if dtype == torch.bfloat16:
        t = torch.as_tensor(_DeviceView(ptr, shape, torch.float16), device=f"cuda:{device}")
        return t.view(torch.bfloat16)
    return torch.as_tensor(_DeviceView(ptr, shape, dtype), device=f"cuda:{device}")


def planned_bytes(heads: int, head_dim: int, capacity: int, window: Optional[int],
                  storage: torch.dtype, copies: int = 1) -> int:
    out = ctypes.c_uint64()
    err = _lib.Error()
    hw, w = (0, 0) if window is None else (1, window)
    _check(_lib.load().tkh_kv_planned_bytes(heads, head_dim, capacity, hw, w, _CODE[storage],
                                            copies, ctypes.byref(out), ctypes.byref(err)), err)
    return int(out.value)


class _Owner:
    def __init__(self, ctx: Context, heads: int, dims: int, capacity: int, max_positions: int,
                 window: Optional[int], storage: torch.dtype):
        self.ctx = ctx
        handle = ctypes.c_void_p()
        err = _lib.Error()
        hw, w = (0, 0) if window is None else (1, window)
        _check(_lib.load().tkh_kv_create(ctx.handle, heads, dims, capacity, max_positions, hw, w,
                                         _CODE[storage], ctypes.byref(handle), ctypes.byref(err)),
               err)
        self.handle = handle
        self.storage = storage
        _lib.track(self, _lib.KV_OWNER)

    def info(self) -> _lib.KvInfo:
        info = _lib.KvInfo()
        _lib.load().tkh_kv_info_get(self.handle, ctypes.byref(info))
        return info

    def committed(self):
        """(k, v) torch views of the physical [heads, capacity, dims] storage."""
        i = self.info()
        shape = (i.heads, i.capacity, i.dims)
        return (device_tensor(i.k, shape, self.storage, self.ctx.device),
                device_tensor(i.v, shape, self.storage, self.ctx.device))

    @property
    def offset(self) -> int:
        return int(self.info().offset)

    @property
    def generation(self) -> int:
        return int(self.info().generation)

    @property
    def allocated_bytes(self) -> int:
        return int(self.info().allocated_bytes)

    def close(self):
        if getattr(self, "handle", None):
            _lib.load().tkh_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LayerKv(_Owner):
    """One layer's full-retention K/V (model::LayerKv, src/model/cache.rs:4-97)."""

    def __init__(self, ctx: Context, kv_heads: int, head_dim: int, capacity: int,
                 storage: torch.dtype):
        super().__init__(ctx, kv_heads, head_dim, capacity, capacity, None, storage)
        self.kv_heads, self.head_dim, self.capacity = kv_heads, head_dim, capacity

    def append(self, k: torch.Tensor, v: torch.Tensor, offset: int):
        """Token-major new rows [tokens, kv_heads, head_dim] into rows [offset, offset+tokens)."""
        tokens = k.numel() // (self.kv_heads * self.head_dim)
        if k.numel() != tokens * self.kv_heads * self.head_dim or v.numel() != k.numel():
            raise TkhError(_err(_lib.LENGTH, "new KV rows"))
        err = _lib.Error()
        _check(_lib.load().tkh_kv_append(self.handle, offset, tokens, _CODE[k.dtype], _ptr(k),
                                         _ptr(v), ctypes.byref(err)), err)

    def attend(self, q, context, scores, probabilities, shape: CachedAttentionShape):
        k, v = self.committed()
        attention_cached(self.ctx, q, k, v, context, scores, probabilities, shape)


def _err(code: int, tensor: str) -> _lib.Error:
    e = _lib.Error()
    e.code = code
    e.tensor = tensor.encode()
    e.message = f"{tensor} has the wrong length".encode()
    return e


class KvCache:
    """Per-layer separate K/V allocated at session creation (model::KvCache)."""

    def __init__(self, ctx: Context, num_layers: int, kv_heads: int, head_dim: int,
                 capacity: int, storage: torch.dtype):
        self.capacity = capacity
        self.layers: List[LayerKv] = [LayerKv(ctx, kv_heads, head_dim, capacity, storage)
                                      for _ in range(num_layers)]

    @staticmethod
    def planned_bytes(num_layers, kv_heads, head_dim, capacity, storage) -> int:
        return planned_bytes(kv_heads, head_dim, capacity, None, storage, num_layers)

    @property
    def allocated_bytes(self) -> int:
        return sum(layer.allocated_bytes for layer in self.layers)


@dataclass
class PreparedKv:
    """Opaque proposal (window_cache.rs:36-43); k/v must stay alive and unchanged."""
    frame: _lib.KvFrame
    k: torch.Tensor
    v: torch.Tensor


class WindowKvCache(_Owner):
    """Global (window None) or ring (window W == capacity) owner (window_cache.rs:21-350)."""

    def __init__(self, ctx: Context, heads: int, dims: int, capacity: int, max_positions: int,
                 window: Optional[int], storage: torch.dtype):
        super().__init__(ctx, heads, dims, capacity, max_positions, window, storage)
        self.heads, self.dims, self.capacity, self.window = heads, dims, capacity, window

    def prepare(self, k: torch.Tensor, v: torch.Tensor, tokens: int) -> PreparedKv:
        """New rows [heads, tokens, dims] in the storage dtype (device)."""
        frame = _lib.KvFrame()
        err = _lib.Error()
        _check(_lib.load().tkh_kv_prepare(self.handle, _ptr(k), k.numel(), _ptr(v), v.numel(),
                                          tokens, ctypes.byref(frame), ctypes.byref(err)), err)
        return PreparedKv(frame, k, v)

    def view(self, prepared: PreparedKv) -> "KvView":
        return KvView(self, prepared)

    def commit(self, prepared: PreparedKv):
        commit_batch([self], [prepared])


class KvView:
    """Checked attention union of old ring spans and the staged chunk (window_cache.rs:45-52)."""

    def __init__(self, cache: WindowKvCache, prepared: PreparedKv):
        self.cache, self.prepared = cache, prepared

    def _raw(self, query_heads: int, scale: float):
        segs = (_lib.Segment * 3)()
        shape = _lib.SpanShape()
        err = _lib.Error()
        _check(_lib.load().tkh_kv_view(self.cache.handle, ctypes.byref(self.prepared.frame),
                                       query_heads, scale, segs, ctypes.byref(shape),
                                       ctypes.byref(err)), err)
        return segs, shape

    def segments(self) -> List[AttentionKvSegment]:
        segs, _ = self._raw(1, 1.0)
        out = []
        dt = self.cache.storage
        for s in segs:
            if s.keys == 0:
                out.append(AttentionKvSegment(None, None, 0, 0, int(s.key_start)))
                continue
            k = device_tensor(s.k, (s.k_len,), dt, self.cache.ctx.device)
            v = device_tensor(s.v, (s.v_len,), dt, self.cache.ctx.device)
            out.append(AttentionKvSegment(k, v, int(s.keys), int(s.head_stride), int(s.key_start)))
        return out

    def attention_shape(self, query_heads: int, scale: float) -> SpanAttentionShape:
        _, s = self._raw(query_heads, scale)
        return SpanAttentionShape(int(s.queries), int(s.keys), int(s.query_heads),
                                  int(s.kv_heads), int(s.head_dim), int(s.query_start),
                                  int(s.key_start), int(s.window) if s.has_window else None,
                                  float(s.scale))


def commit_batch(caches: List[WindowKvCache], frames: List[PreparedKv]):
    if len(caches) != len(frames):
        raise TkhError(_err(_lib.LENGTH, "KV commit frames"))
    n = len(caches)
    handles = (ctypes.c_void_p * n)(*[c.handle.value for c in caches])
    raw = (_lib.KvFrame * n)(*[f.frame for f in frames])
    err = _lib.Error()
    _check(_lib.load().tkh_kv_commit_batch(handles, raw, n, ctypes.byref(err)), err)


def reset_batch(caches: List[WindowKvCache]):
    n = len(caches)
    handles = (ctypes.c_void_p * n)(*[c.handle.value for c in caches])
    err = _lib.Error()
    _check(_lib.load().tkh_kv_reset_batch(handles, n, ctypes.byref(err)), err)
