"""GPU parity: the HIP path through the C ABI against the CPU oracle and frozen vectors.

Bar: FP32 storage within 1e-5 of the oracle (and the reference gate against the
frozen fixtures); bf16/f16 storage within 2e-3 max abs of the oracle run on the
same stored (rounded) Q/K/V, with identical greedy tokens.
"""

import os

import numpy as np
import pytest

from goldens import TINY_CASES, Golden, close, head_major_to_token_major
from gpu_util import (TOL_F32, TOL_HALF, assert_tokens_agree, dev, head_major_cache, host, log,
                      max_err, stored)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch


@pytest.fixture(scope="module")
def ctx(torch_mod):
    from toklet_amd import ops

    return ops.Context(0)


@pytest.fixture(scope="module")
def ops():
    from toklet_amd import ops

    return ops


def _zeros(torch, n):
    return torch.zeros(n, dtype=torch.float32, device="cuda")


# ---------------------------------------------------------------- frozen fixtures, FP32

def test_tiny_cached_f32_with_stale_nan_tails(torch_mod, ctx, ops, orc):
    torch = torch_mod
    tiny = Golden("tiny_v1")
    for case in TINY_CASES:
        for layer in range(2):
            p = f"cases.{case}.layers.{layer}"
            q = tiny.arrays[f"{p}.q_rotary"].reshape(-1)
            tokens = q.size // 32
            cap = tokens + 3
            kc = head_major_cache(tiny.arrays[f"{p}.k_rotary"], 2, cap, 8)
            vc = head_major_cache(tiny.arrays[f"{p}.v_projection"], 2, cap, 8)
            expected = tiny.arrays[f"{p}.attention_context"].reshape(-1)
            kd, vd = dev(kc, "f32"), dev(vc, "f32")
            for offset in range(tokens):
                n = tokens - offset
                log(f"tiny cached {case} layer {layer} offset {offset}")
                out = _zeros(torch, n * 32)
                ops.attention_cached(ctx, dev(q[offset * 32:], "f32"), kd, vd, out, None, None,
                                     ops.CachedAttentionShape(n, 4, 2, 8, cap, offset))
                got = host(out)
                close(got, expected[offset * 32:])
                ref, _, _ = orc.attention_cached(q[offset * 32:], kc, vc, n, 4, 2, 8, cap, offset)
                assert max_err(got, ref) <= TOL_F32


def test_tiny_full_attention_with_diagnostics(torch_mod, ctx, ops):
    torch = torch_mod
    tiny = Golden("tiny_v1")
    for case in TINY_CASES:
        for layer in range(2):
            p = f"cases.{case}.layers.{layer}"
            q = tiny.arrays[f"{p}.q_rotary"].reshape(-1)
            tokens = q.size // 32
            log(f"tiny full {case} layer {layer}")
            out = _zeros(torch, tokens * 32)
            sc = _zeros(torch, 4 * tokens * tokens)
            pr = _zeros(torch, 4 * tokens * tokens)
            ops.attention(ctx, dev(q, "f32"), dev(tiny.arrays[f"{p}.k_rotary"], "f32"),
                          dev(tiny.arrays[f"{p}.v_projection"], "f32"), out, sc, pr,
                          ops.AttentionShape(tokens, 4, 2, 8))
            close(host(out), tiny.arrays[f"{p}.attention_context"])
            close(host(sc), tiny.arrays[f"{p}.attention_scores"])
            close(host(pr), tiny.arrays[f"{p}.attention_probabilities"])
            probs = host(pr).reshape(4, tokens, tokens)
            for t in range(tokens):
                assert np.all(probs[:, t, t + 1:].view(np.uint32) == 0)


def test_grouped_heads_share_value_head(torch_mod, ctx, ops):
    torch = torch_mod
    out = _zeros(torch, 8)
    ops.attention(ctx, dev(np.zeros(8), "f32"), dev(np.zeros(4), "f32"),
                  dev(np.array([1.0, 2.0, 3.0, 4.0]), "f32"), out, None, None,
                  ops.AttentionShape(1, 4, 2, 2))
    assert host(out).tolist() == [1, 2, 1, 2, 3, 4, 3, 4]


def test_gemma_local_fixture_window_attention(torch_mod, ctx, ops):
    torch = torch_mod
    g = Golden("gemma_local_attention_v1")
    for case in g.meta["cases"]:
        if case["queries"] == 0:
            continue
        Q, K, hq, hkv, D = case["queries"], case["keys"], case["q_heads"], case["kv_heads"], case["dims"]
        log(f"gemma local {case['name']}")
        cap = K + 2
        arr = {n: g[case["arrays"][n]] for n in case["arrays"]}
        k = np.full((hkv, cap, D), np.nan, np.float32)
        v = k.copy()
        k[:, :K] = arr["k"]
        v[:, :K] = arr["v"]
        out = _zeros(torch, Q * hq * D)
        sc = _zeros(torch, hq * Q * K)
        pr = _zeros(torch, hq * Q * K)
        shape = ops.WindowAttentionShape(Q, K, cap, hq, hkv, D, case["origin"] + K - Q,
                                         case["origin"], case["window"], case["scale"])
        ops.window_attention(ctx, dev(head_major_to_token_major(arr["q"], hq, Q, D), "f32"),
                             dev(k, "f32"), dev(v, "f32"), out, sc, pr, shape)
        close(host(out), head_major_to_token_major(arr["output"], hq, Q, D))
        close(host(sc), arr["scores"])
        close(host(pr), arr["probabilities"])


def test_fp16_fixture_half_storage(torch_mod, ctx, ops):
    torch = torch_mod
    g = Golden("fp16_v1")
    for case in TINY_CASES:
        for layer in range(2):
            p = f"cases.{case}.layers.{layer}"
            log(f"fp16 fixture {case} layer {layer}")
            q = g.arrays[f"{p}.q_rotary"].reshape(-1)
            tokens = q.size // 32
            ck, cv = g.arrays[f"{p}.cache_k"], g.arrays[f"{p}.cache_v"]
            out = _zeros(torch, tokens * 32)
            qd = torch.from_numpy(q.copy()).cuda()
            ops.attention_cached(ctx, qd, torch.from_numpy(ck.copy()).cuda(),
                                 torch.from_numpy(cv.copy()).cuda(), out, None, None,
                                 ops.CachedAttentionShape(tokens, 4, 2, 8, 32, 0))
            gate = g.meta["gates"][f"{p}.attention_context"]
            close(host(out), g.arrays[f"{p}.attention_context"].astype(np.float32),
                  atol=gate["atol"], rtol=gate["rtol"])


def test_gemma_kv_ring_owner_matches_fixture(torch_mod, ctx, ops):
    """Device WindowKvCache through every frozen step, including abort and retry."""
    torch = torch_mod
    from toklet_amd import kv as kvmod

    g = Golden("gemma_kv_v1")
    for case in g.meta["cases"]:
        hkv, hq, D, cap, W = case["kv_heads"], case["query_heads"], case["dims"], case["capacity"], case["window"]
        max_pos = max(sum(case["chunks"]), cap)
        cache = kvmod.WindowKvCache(ctx, hkv, D, cap, max_pos, W, torch.float32)
        for step in case["steps"]:
            log(f"gemma kv {case['name']} step {step['index']}")
            arr = {n: g[step["arrays"][n]] for n in step["arrays"]}
            tokens = step["count"]
            k_now, v_now = cache.committed()
            assert np.array_equal(host(k_now).reshape(-1), arr["ring_before_k"].reshape(-1))
            assert np.array_equal(host(v_now).reshape(-1), arr["ring_before_v"].reshape(-1))
            new_k = dev(arr["new_k"], "f32")
            new_v = dev(arr["new_v"], "f32")
            frame = cache.prepare(new_k, new_v, tokens)
            view = cache.view(frame)
            shape = view.attention_shape(hq, 1.0)
            assert shape.query_start == step["before"]
            assert shape.key_start == step["required_positions"][0]
            out = _zeros(torch, tokens * hq * D)
            ops.span_attention(ctx, dev(head_major_to_token_major(arr["q"], hq, tokens, D), "f32"),
                               view.segments(), out, None, None, shape)
            close(host(out), head_major_to_token_major(arr["context"], hq, tokens, D))
            if step["abort_expected"]:
                del frame  # discarded proposal: committed state unchanged
                k_now, _ = cache.committed()
                assert np.array_equal(host(k_now).reshape(-1), arr["ring_before_k"].reshape(-1))
                frame = cache.prepare(new_k, new_v, tokens)
            gen = cache.generation
            cache.commit(frame)
            assert cache.generation == gen + 1 and cache.offset == step["after"]
            k_now, v_now = cache.committed()
            assert np.array_equal(host(k_now).reshape(-1), arr["ring_after_k"].reshape(-1))
            assert np.array_equal(host(v_now).reshape(-1), arr["ring_after_v"].reshape(-1))
            with pytest.raises(ops.TkhError) as e:  # the committed frame is now stale
                cache.view(frame).attention_shape(hq, 1.0)
            assert e.value.name == "InvalidConfig"


def test_logit_softcap_fixture(torch_mod, ctx, ops, orc):
    torch = torch_mod
    g = Golden("gemma_softcap_v1")
    for case in g.meta["cases"]:
        if case["width"] == 0:
            continue
        log(f"softcap {case['name']}")
        x = dev(g[case["input"]], "f32")
        ops.logit_softcap(ctx, x, case["cap"])
        got = host(x)
        close(got, g[case["math"]])
        assert max_err(got, orc.logit_softcap(g[case["input"]], case["cap"])) <= 1e-6
    bad = dev(np.array([1.0, np.nan, 2.0]), "f32")
    with pytest.raises(ops.TkhError) as e:
        ops.logit_softcap(ctx, bad, 30.0)
    assert e.value.name == "NonFinite"
    assert np.isnan(host(bad)[1]) and host(bad)[0] == 1.0  # nothing written


# ---------------------------------------------------------------- MFMA path, seeded

def _chunked_session(torch, ctx, ops, orc, *, hq, hkv, D, dt, chunks, capacity, seed,
                     key_scale=None, qk_scale=1.0):
    """Prefill/decode through attention_cached chunk by chunk, checking each call."""
    rng = np.random.default_rng(seed)
    total = sum(chunks)
    k_rows = rng.standard_normal((total, hkv, D)).astype(np.float32) * qk_scale
    v_rows = rng.standard_normal((total, hkv, D)).astype(np.float32)
    if key_scale is not None:
        mask = rng.random((total, hkv)) < key_scale
        k_rows[mask] *= 8.0
    q_rows = rng.standard_normal((total, hq, D)).astype(np.float32) * qk_scale
    kc = head_major_cache(stored(k_rows, dt), hkv, capacity, D)
    vc = head_major_cache(stored(v_rows, dt), hkv, capacity, D)
    kd, vd = dev(kc, dt), dev(vc, dt)
    qs = stored(q_rows, dt)
    start = 0
    worst = 0.0
    contexts = []
    for n in chunks:
        q = qs[start:start + n].reshape(-1)
        out = _zeros(torch, n * hq * D)
        ops.attention_cached(ctx, dev(q, dt), kd, vd, out, None, None,
                             ops.CachedAttentionShape(n, hq, hkv, D, capacity, start))
        got = host(out)
        # the oracle reads the same stored values widened to FP32, with a clean tail
        kcl = np.nan_to_num(kc, nan=0.0)
        vcl = np.nan_to_num(vc, nan=0.0)
        ref, _, _ = orc.attention_cached(q, kcl, vcl, n, hq, hkv, D, capacity, start)
        err = max_err(got, ref)
        worst = max(worst, err)
        assert err <= TOL_HALF, f"chunk at {start}: max abs error {err}"
        contexts.append((got.reshape(n, hq * D), ref.reshape(n, hq * D)))
        start += n
    return worst, contexts


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_mfma_qwen3_chunked_prefill_then_decode(torch_mod, ctx, ops, orc, dt):
    torch = torch_mod
    log(f"qwen3 16/8/128 {dt} prefill 2x128 + 6 decode")
    worst, ctxs = _chunked_session(torch, ctx, ops, orc, hq=16, hkv=8, D=128, dt=dt,
                                   chunks=[128, 128, 1, 1, 1, 1, 1, 1], capacity=300, seed=1)
    rng = np.random.default_rng(99)
    w = rng.standard_normal((4096, 16 * 128)).astype(np.float32)
    for got, ref in ctxs:
        assert_tokens_agree(got, ref, w)
    log(f"  worst max abs error {worst:.3e}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_mfma_qwen25_shape_d64_gqa7(torch_mod, ctx, ops, orc, dt):
    torch = torch_mod
    log(f"qwen2.5 14/2/64 {dt} chunks 37+91+1")
    _chunked_session(torch, ctx, ops, orc, hq=14, hkv=2, D=64, dt=dt,
                     chunks=[37, 91, 1, 1], capacity=140, seed=2)


def test_mfma_peaky_keys_llama_shape(torch_mod, ctx, ops, orc):
    torch = torch_mod
    log("llama 32/8/128 bf16 with 5% of key rows x8")
    worst, _ = _chunked_session(torch, ctx, ops, orc, hq=32, hkv=8, D=128, dt="bf16",
                                chunks=[200, 128, 1], capacity=400, seed=3, key_scale=0.05)
    log(f"  worst max abs error {worst:.3e}")


def test_mfma_d256_window_softcap(torch_mod, ctx, ops, orc):
    """Gemma-style 8/4/256 sliding window with the tanh score softcap (cap 50)."""
    torch = torch_mod
    rng = np.random.default_rng(4)
    hq, hkv, D, W, cap = 8, 4, 256, 96, 50.0
    keys, queries = 300, 64
    for dt in ("bf16", "f16"):
        for softcap in (0.0, cap):
            log(f"gemma window {dt} softcap {softcap}")
            k = stored(rng.standard_normal((hkv, keys, D)) * 3, dt)
            v = stored(rng.standard_normal((hkv, keys, D)), dt)
            q = stored(rng.standard_normal((queries, hq, D)) * 3, dt).reshape(-1)
            out = _zeros(torch, queries * hq * D)
            shape = ops.WindowAttentionShape(queries, keys, keys, hq, hkv, D, keys - queries + 1000,
                                             1000, W, 1.0 / 16.0, softcap)
            ops.window_attention(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None, shape)
            ref, _, _ = orc.window_attention(q, k.reshape(-1), v.reshape(-1), queries, keys, keys, hq,
                                             hkv, D, keys - queries + 1000, 1000, W, 1.0 / 16.0,
                                             softcap=softcap)
            err = max_err(host(out), ref)
            log(f"  max abs error {err:.3e}")
            assert err <= TOL_HALF


def test_mfma_span_attention_over_ring(torch_mod, ctx, ops, orc):
    """A bf16 ring (W=64) fed in chunks through the device KV owner and span_attention."""
    torch = torch_mod
    from toklet_amd import kv as kvmod

    rng = np.random.default_rng(5)
    hq, hkv, D, W = 8, 4, 128, 64
    cache = kvmod.WindowKvCache(ctx, hkv, D, W, 4096, W, torch.bfloat16)
    ring_k = np.zeros((hkv, W, D), np.float32)
    ring_v = np.zeros((hkv, W, D), np.float32)
    offset = 0
    for n in (40, 50, 1, 1, 100, 3):
        log(f"ring chunk {n} at offset {offset}")
        nk = stored(rng.standard_normal((hkv, n, D)), "bf16")
        nv = stored(rng.standard_normal((hkv, n, D)), "bf16")
        q = stored(rng.standard_normal((n, hq, D)), "bf16").reshape(-1)
        frame = cache.prepare(dev(nk, "bf16"), dev(nv, "bf16"), n)
        view = cache.view(frame)
        shape = view.attention_shape(hq, 1.0 / np.sqrt(D))
        shape.softcap = 50.0
        out = _zeros(torch, n * hq * D)
        ops.span_attention(ctx, dev(q, "bf16"), view.segments(), out, None, None, shape)
        segs = []
        for position, slot, rows in orc.old_spans(W, offset, W):
            if rows == 0:
                segs.append(orc.Segment(np.zeros(0), np.zeros(0), 0, 0, offset))
                continue
            b = slot * D
            e = (hkv - 1) * W * D + b + rows * D
            segs.append(orc.Segment(ring_k.reshape(-1)[b:e], ring_v.reshape(-1)[b:e], rows, W * D,
                                    position))
        segs.append(orc.Segment(nk.reshape(-1), nv.reshape(-1), n, n * D, offset))
        ref, _, _ = orc.span_attention(q, segs, n, shape.keys, hq, hkv, D, offset, shape.key_start,
                                       W, np.float32(1.0 / np.sqrt(D)), softcap=50.0)
        err = max_err(host(out), ref)
        assert err <= TOL_HALF, err
        cache.commit(frame)
        for src, slot, rows in orc.copy_runs(W, offset, n, True):
            ring_k[:, slot:slot + rows] = nk[:, src:src + rows]
            ring_v[:, slot:slot + rows] = nv[:, src:src + rows]
        offset += n
        ck, cv = cache.committed()
        assert np.array_equal(host(ck), ring_k) and np.array_equal(host(cv), ring_v)


def test_decode_batch_varlen_f16(torch_mod, ctx, ops, orc):
    torch = torch_mod
    rng = np.random.default_rng(6)
    hq, hkv, D, B = 16, 8, 128, 6
    lengths = rng.integers(100, 1500, size=B)
    caps = lengths + rng.integers(0, 40, size=B)
    offsets = np.concatenate([[0], np.cumsum(hkv * caps * D)[:-1]])
    total = int((hkv * caps * D).sum())
    kpool = np.full(total, np.nan, np.float32)
    vpool = np.full(total, np.nan, np.float32)
    q = np.zeros((B, hq, D), np.float32)
    refs = []
    for b in range(B):
        s = rng.uniform(0.5, 2.0)
        k = head_major_cache(stored(rng.standard_normal((lengths[b], hkv, D)) * s, "f16"), hkv, caps[b], D)
        v = head_major_cache(stored(rng.standard_normal((lengths[b], hkv, D)) * s, "f16"), hkv, caps[b], D)
        kpool[offsets[b]:offsets[b] + k.size] = k.reshape(-1)
        vpool[offsets[b]:offsets[b] + v.size] = v.reshape(-1)
        q[b] = stored(rng.standard_normal((hq, D)) * s, "f16")
        ref, _, _ = orc.attention_cached(q[b].reshape(-1), np.nan_to_num(k), np.nan_to_num(v), 1, hq,
                                         hkv, D, int(caps[b]), int(lengths[b]) - 1)
        refs.append(ref)
    log(f"decode batch f16 lengths {lengths.tolist()}")
    out = _zeros(torch, B * hq * D)
    ops.decode_batch(ctx, dev(q, "f16"), dev(kpool, "f16"), dev(vpool, "f16"), offsets,
                     hkv * 0 + caps * D, lengths, out, query_heads=hq, kv_heads=hkv, head_dim=D,
                     scale=float(np.float32(1.0) / np.sqrt(np.float32(D))))
    got = host(out).reshape(B, -1)
    for b in range(B):
        assert max_err(got[b], refs[b]) <= TOL_HALF


def _context_with_env(ops, env):
    """A context created under extra TKH_* settings (read once at creation)."""
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return ops.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("waves", ["4", "8"])
def test_prefill_workgroup_widths_chunked(torch_mod, ops, orc, waves):
    """The prefill kernel with four- and eight-wave workgroups forced (the planner takes
    eight only for launches whose 256-row blocks fill the device), on chunked prefill
    with key splits and merges, then decode."""
    log(f"qwen3 16/8/128 bf16 chunked prefill, {waves}-wave prefill workgroups")
    c = _context_with_env(ops, {"TKH_PREFILL_WAVES": waves})
    try:
        worst, ctxs = _chunked_session(torch_mod, c, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                                       chunks=[256, 256, 128, 1, 1], capacity=700, seed=4)
        rng = np.random.default_rng(98)
        w = rng.standard_normal((4096, 16 * 128)).astype(np.float32)
        for got, ref in ctxs:
            assert_tokens_agree(got, ref, w)
        log(f"  worst max abs error {worst:.3e}")
    finally:
        c.close()


@pytest.mark.parametrize("waves", ["0", "4", "8"])
def test_prefill_batch_bf16(torch_mod, ops, orc, waves):
    """Batched prefill over three sessions, with the planner's workgroup width and with
    four and eight waves forced."""
    torch = torch_mod
    ctx = _context_with_env(ops, {"TKH_PREFILL_WAVES": waves})
    rng = np.random.default_rng(7)
    hq, hkv, D, B, T = 32, 8, 128, 3, 128
    pos = rng.integers(50, 400, size=B)
    caps = pos + T
    offsets = np.concatenate([[0], np.cumsum(hkv * caps * D)[:-1]])
    total = int((hkv * caps * D).sum())
    kpool = np.zeros(total, np.float32)
    vpool = np.zeros(total, np.float32)
    q = stored(rng.standard_normal((B, T, hq, D)), "bf16")
    refs = []
    for b in range(B):
        rows = rng.standard_normal((caps[b], hkv, D)).astype(np.float32)
        rows[rng.random((caps[b], hkv)) < 0.05] *= 8.0
        k = head_major_cache(stored(rows, "bf16"), hkv, caps[b], D)
        v = head_major_cache(stored(rng.standard_normal((caps[b], hkv, D)), "bf16"), hkv, caps[b], D)
        kpool[offsets[b]:offsets[b] + k.size] = k.reshape(-1)
        vpool[offsets[b]:offsets[b] + v.size] = v.reshape(-1)
        ref, _, _ = orc.attention_cached(q[b].reshape(-1), k, v, T, hq, hkv, D, int(caps[b]), int(pos[b]))
        refs.append(ref)
    log(f"prefill batch bf16 positions {pos.tolist()}")
    out = _zeros(torch, B * T * hq * D)
    ops.prefill_batch(ctx, dev(q, "bf16"), dev(kpool, "bf16"), dev(vpool, "bf16"), offsets,
                      caps * D, pos, out, tokens=T, query_heads=hq, kv_heads=hkv, head_dim=D,
                      scale=float(1.0 / np.sqrt(np.float32(D))))
    got = host(out).reshape(B, -1)
    ctx.close()
    for b in range(B):
        err = max_err(got[b], refs[b])
        assert err <= TOL_HALF, err


@pytest.mark.parametrize("D,hq,hkv", [(128, 32, 8), (64, 14, 2), (256, 8, 4)])
def test_prefill_batch_compact_arguments(torch_mod, ops, orc, D, hq, hkv):
    """Batched prefill whose chunks travel in the kernel's own arguments (one
    shape, no key splits: the split target is forced to one workgroup) against
    the same launch with its descriptors uploaded (bit for bit) and the oracle;
    ragged positions, a zero-length cached prefix, one-token chunks."""
    torch = torch_mod
    rng = np.random.default_rng(31 + D)
    for B, T in ((5, 128), (3, 1)):
        pos = rng.integers(0, 300, size=B)
        pos[0] = 0
        caps = pos + T + rng.integers(0, 9, size=B)  # spare cache rows past the chunk
        offsets = np.concatenate([[0], np.cumsum(hkv * caps * D)[:-1]])
        total = int((hkv * caps * D).sum())
        kpool = np.zeros(total, np.float32)
        vpool = np.zeros(total, np.float32)
        q = stored(rng.standard_normal((B, T, hq, D)), "bf16")
        refs = []
        for b in range(B):
            k = head_major_cache(stored(rng.standard_normal((caps[b], hkv, D)), "bf16"), hkv, caps[b], D)
            v = head_major_cache(stored(rng.standard_normal((caps[b], hkv, D)), "bf16"), hkv, caps[b], D)
            kpool[offsets[b]:offsets[b] + k.size] = k.reshape(-1)
            vpool[offsets[b]:offsets[b] + v.size] = v.reshape(-1)
            ref, _, _ = orc.attention_cached(q[b].reshape(-1), k, v, T, hq, hkv, D, int(caps[b]), int(pos[b]))
            refs.append(ref)
        log(f"compact prefill batch D={D} B={B} T={T} positions {pos.tolist()}")
        outs = {}
        for compact in ("1", "0"):
            ctx = _context_with_env(ops, {"TKH_PREFILL_COMPACT": compact, "TKH_PREFILL_GROUPS": "1",
                                          "TKH_PREFILL16_GROUPS": "1"})
            out = _zeros(torch, B * T * hq * D)
            ops.prefill_batch(ctx, dev(q, "bf16"), dev(kpool, "bf16"), dev(vpool, "bf16"), offsets,
                              caps * D, pos, out, tokens=T, query_heads=hq, kv_heads=hkv, head_dim=D,
                              scale=float(1.0 / np.sqrt(np.float32(D))))
            outs[compact] = host(out).reshape(B, -1)
            ctx.close()
        assert np.array_equal(outs["1"], outs["0"])
        for b in range(B):
            err = max_err(outs["1"][b], refs[b])
            assert err <= TOL_HALF, err


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_nonfinite_visible_input_reports_nonfinite(torch_mod, ctx, ops, dt):
    """A NaN in visible Q/K/V is NonFinite (src/cpu/attention.rs:247-251); the context
    contents are then unspecified and the caller discards them (src/cpu/mod.rs:5-7)."""
    torch = torch_mod
    rng = np.random.default_rng(8)
    hq, hkv, D, cap = 16, 8, 128, 64
    k = rng.standard_normal((hkv, cap, D)).astype(np.float32)
    v = rng.standard_normal((hkv, cap, D)).astype(np.float32)
    q = rng.standard_normal((4, hq, D)).astype(np.float32)
    for which in ("k", "v", "q"):
        log(f"non-finite {which} {dt}")
        kk, vv, qq = k.copy(), v.copy(), q.copy()
        {"k": kk, "v": vv, "q": qq}[which].reshape(-1)[37] = np.nan
        out = torch.full((4 * hq * D,), 123.0, device="cuda")
        with pytest.raises(ops.TkhError) as e:
            ops.attention_cached(ctx, dev(qq, dt), dev(kk, dt), dev(vv, dt), out, None, None,
                                 ops.CachedAttentionShape(4, hq, hkv, D, cap, 20))
        assert e.value.name == "NonFinite"
    # afterwards the context works again (status was cleared)
    out = _zeros(torch, 4 * hq * D)
    ops.attention_cached(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None,
                         ops.CachedAttentionShape(4, hq, hkv, D, cap, 20))
    assert np.all(np.isfinite(host(out)))


def test_kv_append_rounds_and_flags(torch_mod, ctx, ops):
    torch = torch_mod
    from toklet_amd import kv as kvmod

    layer = kvmod.LayerKv(ctx, 2, 128, 16, torch.bfloat16)
    rng = np.random.default_rng(9)
    rows = rng.standard_normal((5, 2, 128)).astype(np.float32)
    layer.append(dev(rows, "f32"), dev(rows * 2, "f32"), 3)
    k, v = layer.committed()
    kk, vv = host(k), host(v)
    assert np.array_equal(kk[:, 3:8], stored(rows, "bf16").transpose(1, 0, 2))
    assert np.array_equal(vv[:, 3:8], stored(rows * 2, "bf16").transpose(1, 0, 2))
    assert np.all(kk[:, :3] == 0) and np.all(kk[:, 8:] == 0)
    rows[1, 1, 5] = np.inf
    with pytest.raises(ops.TkhError) as e:
        layer.append(dev(rows, "f32"), dev(rows, "f32"), 0)
    assert e.value.name == "NonFinite"
    with pytest.raises(ops.TkhError) as e:
        layer.append(dev(rows, "f32"), dev(rows, "f32"), 12)
    assert e.value.name == "Capacity"


def test_fp32_qwen25_prefill_decode_argmax(torch_mod, ctx, ops, orc):
    """The FP32 configuration: 14/2/64, prefill 128 then 32 decode steps, 1e-5 and same tokens."""
    torch = torch_mod
    rng = np.random.default_rng(10)
    hq, hkv, D, cap = 14, 2, 64, 160
    total = 160
    q_rows = orc.rotary(rng.standard_normal((total, hq, D)), total, hq, D, 0, 1e6).reshape(total, hq, D)
    k_rows = orc.rotary(rng.standard_normal((total, hkv, D)), total, hkv, D, 0, 1e6)
    v_rows = rng.standard_normal((total, hkv, D)).astype(np.float32)
    kc = head_major_cache(k_rows.reshape(total, hkv, D), hkv, cap, D)
    vc = head_major_cache(v_rows, hkv, cap, D)
    kd, vd = dev(kc, "f32"), dev(vc, "f32")
    w = rng.standard_normal((8192, hq * D)).astype(np.float32)
    start = 0
    for n in [128] + [1] * 32:
        q = q_rows[start:start + n].reshape(-1)
        out = _zeros(torch, n * hq * D)
        ops.attention_cached(ctx, dev(q, "f32"), kd, vd, out, None, None,
                             ops.CachedAttentionShape(n, hq, hkv, D, cap, start))
        ref, _, _ = orc.attention_cached(q, np.nan_to_num(kc), np.nan_to_num(vc), n, hq, hkv, D, cap, start)
        got = host(out)
        assert max_err(got, ref) <= TOL_F32
        assert_tokens_agree(got.reshape(n, -1), ref.reshape(n, -1), w)
        start += n
