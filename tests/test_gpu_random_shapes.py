"""Seeded random shapes through attention_cached and window_attention against the
CPU oracle: head sizes 64/128/256, GQA groups 1/2/4/7/8, bf16/f16/f32 storage,
1..130 queries at offsets to 6000, windows from 1 key to none, score softcaps and
scales.  The combinations the fixed cases leave out (a group of 7 at head_dim 256,
a softcap at head_dim 64, an offset past every split boundary) go through the
same planner, kernels and merge.  Bar: max abs error 2e-3 for half storage; the
reference's gate 1e-5 + 1e-4|e| for FP32 (tests/cpu_attention.rs:6-14)."""

import numpy as np
import pytest

from gpu_util import TOL_HALF, dev, host, log, stored

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch


@pytest.fixture(scope="module")
def ops():
    from toklet_amd import ops

    return ops


def _case(rng):
    D = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 7, 8]))
    return dict(D=D, hkv=hkv, hq=hkv * G, dt=str(rng.choice(["bf16", "f16", "f32"])),
                Q=int(rng.choice([1, 1, 2, 5, 17, 64, 130])), start=int(rng.integers(0, 6000)),
                kind=str(rng.choice(["cached", "window"])), pad=int(rng.integers(0, 7)),
                W=int(rng.choice([0, 1, 7, 64, 300, 1024, 5000])),
                softcap=float(rng.choice([0.0, 0.0, 30.0, 50.0])), scale_pick=int(rng.integers(0, 3)))


@pytest.mark.parametrize("seed", [7, 11])
def test_random_shapes_match_oracle(torch_mod, ops, orc, seed):
    torch = torch_mod
    rng = np.random.default_rng(seed)
    ctx = ops.Context(0)
    for n in range(30):
        c = _case(rng)
        D, hkv, hq, dt, Q, start = c["D"], c["hkv"], c["hq"], c["dt"], c["Q"], c["start"]
        keys = start + Q
        cap = keys + c["pad"]
        k = stored(rng.standard_normal((hkv, cap, D)).astype(np.float32), dt)
        v = stored(rng.standard_normal((hkv, cap, D)).astype(np.float32), dt)
        q = stored(rng.standard_normal((Q, hq, D)).astype(np.float32), dt).reshape(-1)
        out = torch.full((Q * hq * D,), np.nan, dtype=torch.float32, device="cuda")
        log(f"seed {seed} case {n}: {c}")
        if c["kind"] == "cached":
            ops.attention_cached(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None,
                                 ops.CachedAttentionShape(Q, hq, hkv, D, cap, start))
            ref, _, _ = orc.attention_cached(q, k, v, Q, hq, hkv, D, cap, start)
        else:
            scale = [1.0 / np.sqrt(D), 1.0 / 16.0, 0.3][c["scale_pick"]]
            W = c["W"] or None
            shape = ops.WindowAttentionShape(Q, keys, cap, hq, hkv, D, start, 0, W, scale, c["softcap"])
            ops.window_attention(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None, shape)
            ref, _, _ = orc.window_attention(q, k.reshape(-1), v.reshape(-1), Q, keys, cap, hq, hkv, D,
                                             start, 0, W, scale, softcap=c["softcap"])
        got = host(out).astype(np.float64)
        ref = np.asarray(ref, np.float64)
        assert np.all(np.isfinite(got))
        if dt == "f32":
            assert np.all(np.abs(got - ref) <= 1e-5 + 1e-4 * np.abs(ref)), c
        else:
            assert np.max(np.abs(got - ref)) <= TOL_HALF, c


@pytest.mark.parametrize("seed", [3, 5])
def test_random_ring_chunks_match_window_attention(torch_mod, ops, orc, seed):
    """A ring owner (WindowKvCache, src/model/window_cache.rs:21-350) fed random chunk
    sizes (single tokens, chunks shorter and longer than the window): each chunk's
    prepare -> view -> span_attention -> commit gives the contexts of window_attention
    over the whole history, which the ring no longer holds."""
    from toklet_amd import kv as kvmod

    torch = torch_mod
    rng = np.random.default_rng(seed)
    ctx = ops.Context(0)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}
    for trial in range(3):
        D = int(rng.choice([64, 128, 256]))
        hkv = int(rng.choice([1, 2, 4]))
        hq = hkv * int(rng.choice([1, 2, 4]))
        dt = str(rng.choice(["bf16", "f16"]))
        W = int(rng.choice([8, 33, 64, 200]))
        T = int(rng.integers(W, 3 * W + 50))
        scale = float(1.0 / np.sqrt(D))
        softcap = float(rng.choice([0.0, 50.0]))
        cache = kvmod.WindowKvCache(ctx, hkv, D, W, T, W, tdt[dt])
        k_all = stored(rng.standard_normal((hkv, T, D)).astype(np.float32), dt)
        v_all = stored(rng.standard_normal((hkv, T, D)).astype(np.float32), dt)
        q_all = stored(rng.standard_normal((T, hq, D)).astype(np.float32), dt)
        pos = 0
        while pos < T:
            n = int(min(T - pos, rng.choice([1, 1, 3, 17, W, W + 5])))
            log(f"seed {seed} trial {trial}: {hq}/{hkv}/{D} {dt} W={W} softcap {softcap}, chunk {pos}+{n}")
            kn = dev(np.ascontiguousarray(k_all[:, pos:pos + n]), dt)
            vn = dev(np.ascontiguousarray(v_all[:, pos:pos + n]), dt)
            prepared = cache.prepare(kn, vn, n)
            view = cache.view(prepared)
            s = view.attention_shape(hq, scale)
            shape = ops.SpanAttentionShape(s.queries, s.keys, s.query_heads, s.kv_heads, s.head_dim,
                                           s.query_start, s.key_start, s.window, s.scale, softcap)
            q = q_all[pos:pos + n].reshape(-1)
            out = torch.full((n * hq * D,), np.nan, dtype=torch.float32, device="cuda")
            ops.span_attention(ctx, dev(q, dt), view.segments(), out, None, None, shape)
            keys = pos + n
            kh = np.ascontiguousarray(k_all[:, :keys]).reshape(-1)
            vh = np.ascontiguousarray(v_all[:, :keys]).reshape(-1)
            ref, _, _ = orc.window_attention(q, kh, vh, n, keys, keys, hq, hkv, D, pos, 0, W, scale,
                                             softcap=softcap)
            assert np.max(np.abs(host(out).astype(np.float64) - ref)) <= TOL_HALF
            cache.commit(prepared)
            pos += n
        cache.close()


@pytest.mark.parametrize("seed", [13, 17])
def test_random_batches_match_per_session_attention(torch_mod, ops, orc, seed):
    """tkh_decode_batch and tkh_prefill_batch over random batches (1 to 70 sessions,
    past the 64 that travel in the kernel arguments), lengths, head sizes, GQA
    groups, dtypes, scales and per-session cache strides: every session's context
    equals window attention over its own cache (no window)."""
    torch = torch_mod
    rng = np.random.default_rng(seed)
    ctx = ops.Context(0)
    for trial in range(4):
        D = int(rng.choice([64, 128, 256]))
        hkv = int(rng.choice([1, 2, 8]))
        hq = hkv * int(rng.choice([1, 2, 4]))
        dt = str(rng.choice(["bf16", "f16"]))
        B = int(rng.choice([1, 3, 17, 64, 70]))
        scale = float(rng.choice([1.0 / np.sqrt(D), 0.05]))
        decode = trial % 2 == 0
        tokens = 1 if decode else int(rng.choice([1, 16, 64, 128]))
        if decode:
            lengths = [int(x) for x in rng.integers(1, 3000, B)]
            positions = [n - 1 for n in lengths]
        else:
            positions = [int(x) for x in rng.integers(0, 1500, B)]
            lengths = [p + tokens for p in positions]
        caps = [n + int(rng.integers(0, 5)) for n in lengths]
        log(f"seed {seed} trial {trial}: {'decode' if decode else 'prefill'} B={B} tokens={tokens} "
            f"{hq}/{hkv}/{D} {dt} scale {scale:.4f}")
        offsets, pool_k, pool_v, total = [], [], [], 0
        for b in range(B):
            n = hkv * caps[b] * D
            offsets.append(total)
            pool_k.append(stored(rng.standard_normal(n).astype(np.float32), dt))
            pool_v.append(stored(rng.standard_normal(n).astype(np.float32), dt))
            total += n
        kpool, vpool = np.concatenate(pool_k), np.concatenate(pool_v)
        q = stored(rng.standard_normal((B, tokens, hq, D)).astype(np.float32), dt)
        out = torch.full((B * tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
        strides = [c * D for c in caps]
        if decode:
            ops.decode_batch(ctx, dev(q, dt), dev(kpool, dt), dev(vpool, dt), offsets, strides, lengths,
                             out, query_heads=hq, kv_heads=hkv, head_dim=D, scale=scale)
        else:
            ops.prefill_batch(ctx, dev(q, dt), dev(kpool, dt), dev(vpool, dt), offsets, strides,
                              positions, out, tokens=tokens, query_heads=hq, kv_heads=hkv, head_dim=D,
                              scale=scale)
        got = host(out).reshape(B, -1).astype(np.float64)
        for b in range(B):
            kb = kpool[offsets[b]:offsets[b] + hkv * caps[b] * D]
            vb = vpool[offsets[b]:offsets[b] + hkv * caps[b] * D]
            ref, _, _ = orc.window_attention(q[b].reshape(-1), kb, vb, tokens, lengths[b], caps[b], hq,
                                             hkv, D, positions[b] if not decode else lengths[b] - 1, 0,
                                             None, scale)
            assert np.max(np.abs(got[b] - ref)) <= TOL_HALF, (trial, b)
