"""Every BASELINE configuration at its stated size through the HIP path, checked
against the CPU oracle on sampled rows (max abs error 2e-3 for bf16/f16 KV,
greedy tokens identical to the oracle's on every checked row, over a random
projection).

  configs[1]  Qwen3 16/8/128 bf16 session: RMSNorm (weights N(1, 0.02)) + rotary
              1e6, 2048 prompt tokens in 128-token chunks, then 256 single-token
              decode steps (the producer folded into the decode kernel).
  configs[2]  64 f16 sessions, L ~ U[512, 8192], one query token each, Q/K/V
              N(0, 1) times a scale U[0.5, 2] per (session, KV head).
  configs[3]  Gemma3-style 8/4/256 bf16 session: 5 sliding layers (W = 1024) and
              1 global, scale 1/16, score softcap 50, 4096 prompt tokens in
              128-token chunks then 128 decode steps.
  configs[4]  32 bf16 sessions x (4096 cached + 128 new) at 32/8/128, Q/K
              through the producer's rotary (theta 500000), 5% of key rows x8,
              through tkh_prefill_batch.
  tkh_attention (token-major K/V) at bf16 and f16.
"""

import math

import numpy as np
import pytest

from gpu_util import TOL_F32, TOL_HALF, assert_tokens_identical, dev, host, log, max_err, stored

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


@pytest.fixture(scope="module")
def sess_mod():
    from toklet_amd import session

    return session


def _t(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")


def _produce(orc, x, w, rows, heads, D, position, theta, dt):
    """Oracle producer (rmsnorm when w is given, split-half rotary), rounded to the cache dtype."""
    y = orc.rmsnorm(x.reshape(-1), w, rows * heads, D, 1e-6) if w is not None else x.reshape(-1)
    return stored(orc.rotary(y, rows, heads, D, position, theta), dt).reshape(rows, heads, D)


def _projection_weights(torch, vocab, hidden, seed):
    """A seeded N(0, 1) FP32 output projection [vocab, hidden], on the device and the host."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(vocab, hidden, generator=g, device="cuda")
    return w, w.cpu().numpy()


def _check_projection(torch, ops, orc, ctx, got_rows, ref_rows, w_dev, w_host, label):
    """Device o-projection + greedy of the device contexts: logits bit-exact with the
    oracle's FP32 matmul and tokens equal to its greedy pick, and to the tokens of
    the oracle's own contexts."""
    rows, hidden = got_rows.shape
    vocab = w_host.shape[0]
    c = torch.from_numpy(np.ascontiguousarray(got_rows)).cuda()
    tokens = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    logits = torch.full((rows, vocab), np.nan, dtype=torch.float32, device="cuda")
    ops.project_greedy(ctx, c, w_dev, tokens, logits)
    tok = tokens.cpu().numpy().view(np.uint32)
    lg = host(logits)
    for r in range(rows):
        ref = orc.matmul(got_rows[r], w_host, 1, hidden, vocab)
        assert np.array_equal(lg[r].view(np.uint32), ref.view(np.uint32)), f"{label} row {r} logits"
        assert tok[r] == orc.greedy(ref), f"{label} row {r} token"
    assert_tokens_identical(got_rows, ref_rows, w_host)
    log(f"{label}: {rows} rows projected onto {vocab} ids on the device, logits bit-exact, "
        f"tokens identical, also to the oracle's contexts' tokens")


def test_configs0_fp32_session_and_projection_full_size(torch_mod, ops, sess_mod, orc):
    """Qwen2.5-0.5B-shaped FP32 attention (14/2/64, rotary 1e6, scale 1/8),
    a 128-token prompt then 32 decode steps, and the greedy token of every row over a
    seeded 896 x 151936 projection on the device."""
    torch = torch_mod
    rng = np.random.default_rng(100)
    hq, hkv, D, prompt, steps = 14, 2, 64, 128, 32
    total = prompt + steps
    qp = rng.standard_normal((total, hq, D)).astype(np.float32)
    kp = rng.standard_normal((total, hkv, D)).astype(np.float32)
    vp = rng.standard_normal((total, hkv, D)).astype(np.float32)
    ctx = ops.Context(0)
    out = torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda")
    s = sess_mod.Session(ctx, sess_mod.Options(capacity=total, prefill_chunk_size=128,
                                               vocab_size=151936, layers=1, query_heads=hq,
                                               kv_heads=hkv, head_dim=D, storage="f32", theta=1e6))
    io = [sess_mod.LayerIo(_t(torch, qp), _t(torch, kp), _t(torch, vp), out)]
    s.set_tokens([5] * prompt)
    assert s.evaluate(io) == prompt
    s.append([6] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    got = host(out)
    q = _produce(orc, qp, None, total, hq, D, 0, 1e6, "f32")
    k = _produce(orc, kp, None, total, hkv, D, 0, 1e6, "f32")
    ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), vp.reshape(-1), total, hq, hkv, D)
    ref = ref.reshape(total, hq * D)
    err = max_err(got, ref)
    log(f"configs[0] FP32 session: {total} rows, max abs error {err:.3e}")
    assert err <= TOL_F32
    w_dev, w_host = _projection_weights(torch, 151936, hq * D, 100)
    sample = [0, 63, 127] + list(range(prompt, total))
    _check_projection(torch, ops, orc, ctx, got[sample], ref[sample], w_dev, w_host,
                      "configs[0] prompt rows 0/63/127 and all 32 decode steps")
    s.close()
    ctx.close()


def test_configs1_qwen3_session_full_size(torch_mod, ops, sess_mod, orc):
    torch = torch_mod
    rng = np.random.default_rng(101)
    hq, hkv, D, prompt, steps, chunk = 16, 8, 128, 2048, 256, 128
    total = prompt + steps
    qp = rng.standard_normal((total, hq, D)).astype(np.float32)
    kp = rng.standard_normal((total, hkv, D)).astype(np.float32)
    vp = rng.standard_normal((total, hkv, D)).astype(np.float32)
    wq = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    wk = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    ctx = ops.Context(0, synchronous=False)
    out = torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda")
    s = sess_mod.Session(ctx, sess_mod.Options(capacity=total, prefill_chunk_size=chunk,
                                               vocab_size=151936, layers=1, query_heads=hq,
                                               kv_heads=hkv, head_dim=D, storage="bf16", theta=1e6))
    io = [sess_mod.LayerIo(_t(torch, qp), _t(torch, kp), _t(torch, vp), out, _t(torch, wq),
                           _t(torch, wk))]
    s.set_tokens([7] * prompt)
    assert s.evaluate(io) == prompt
    s.append([9] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    s.synchronize()
    got = host(out)
    k = _produce(orc, kp, wk, total, hkv, D, 0, 1e6, "bf16").transpose(1, 0, 2).copy()
    v = stored(vp, "bf16").transpose(1, 0, 2).copy()
    rows = sorted({p for c in range(prompt // chunk) for p in (c * chunk, c * chunk + 63, c * chunk + 127)}
                  | {prompt, prompt + 1, prompt + 127, total - 1})
    refs, gots, worst = [], [], 0.0
    for p in rows:
        q = _produce(orc, qp[p:p + 1], wq, 1, hq, D, p, 1e6, "bf16").reshape(-1)
        ref, _, _ = orc.attention_cached(q, k.reshape(-1), v.reshape(-1), 1, hq, hkv, D, total, p)
        worst = max(worst, max_err(got[p], ref))
        refs.append(ref)
        gots.append(got[p])
    w = rng.standard_normal((4096, hq * D)).astype(np.float32)
    assert_tokens_identical(np.stack(gots), np.stack(refs), w)
    log(f"configs[1] session: {len(rows)} rows (every chunk's first, middle and last, decode "
        f"steps 1, 2, 128, 256), max abs error {worst:.3e}, greedy tokens identical")
    assert worst <= TOL_HALF
    del w
    w_dev, w_host = _projection_weights(torch, 151936, hq * D, 101)
    decode = [i for i, p in enumerate(rows) if p >= prompt]
    _check_projection(torch, ops, orc, ctx, np.stack(gots)[decode], np.stack(refs)[decode], w_dev,
                      w_host, "configs[1] decode steps 1, 2, 128, 256")
    s.close()
    ctx.close()


def test_configs2_batched_decode_full_size(torch_mod, ops, orc):
    torch = torch_mod
    rng = np.random.default_rng(102)
    hq, hkv, D, B = 16, 8, 128, 64
    G = hq // hkv
    lengths = rng.integers(512, 8193, B)
    scales = rng.uniform(0.5, 2.0, (B, hkv)).astype(np.float32)   # per (session, KV head)
    gd = torch.Generator(device="cuda").manual_seed(102)
    offsets, total = [], 0
    for L in lengths:
        offsets.append(total)
        total += hkv * int(L) * D
    kpool = torch.randn(total, generator=gd, device="cuda")
    vpool = torch.randn(total, generator=gd, device="cuda")
    sc = torch.from_numpy(scales).cuda()
    for b, L in enumerate(lengths):
        n = hkv * int(L) * D
        seg = (slice(offsets[b], offsets[b] + n))
        kpool[seg] = (kpool[seg].view(hkv, -1) * sc[b][:, None]).reshape(-1)
        vpool[seg] = (vpool[seg].view(hkv, -1) * sc[b][:, None]).reshape(-1)
    kpool, vpool = kpool.half(), vpool.half()
    q = (torch.randn(B, hq, D, generator=gd, device="cuda") *
         sc.repeat_interleave(G, dim=1)[:, :, None]).half()
    out = torch.full((B * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.decode_batch(ops.Context(0), q, kpool, vpool, offsets, [int(L) * D for L in lengths],
                     [int(L) for L in lengths], out, query_heads=hq, kv_heads=hkv, head_dim=D,
                     scale=1.0 / math.sqrt(D))
    got = host(out).reshape(B, -1)
    kh, vh, qh = host(kpool), host(vpool), host(q)
    worst, refs = 0.0, []
    for b, L in enumerate(lengths):
        n = hkv * int(L) * D
        ref, _, _ = orc.attention_cached(qh[b].reshape(-1), kh[offsets[b]:offsets[b] + n],
                                         vh[offsets[b]:offsets[b] + n], 1, hq, hkv, D, int(L),
                                         int(L) - 1)
        worst = max(worst, max_err(got[b], ref))
        refs.append(ref)
    w = rng.standard_normal((4096, hq * D)).astype(np.float32)
    assert_tokens_identical(got, np.stack(refs), w)
    log(f"configs[2] 64 sessions (sum of lengths {int(lengths.sum())}): max abs error {worst:.3e}, "
        f"greedy tokens identical")
    assert worst <= TOL_HALF


def test_configs3_gemma_local_global_session_full_size(torch_mod, ops, sess_mod, orc):
    torch = torch_mod
    rng = np.random.default_rng(103)
    hq, hkv, D, W, prompt, steps, layers = 8, 4, 256, 1024, 4096, 128, 6
    total = prompt + steps
    windows = [W] * 5 + [0]
    projs = [(rng.standard_normal((total, hq, D)).astype(np.float32),
              rng.standard_normal((total, hkv, D)).astype(np.float32),
              rng.standard_normal((total, hkv, D)).astype(np.float32)) for _ in range(layers)]
    outs = [torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda") for _ in range(layers)]
    io = [sess_mod.LayerIo(_t(torch, q), _t(torch, k), _t(torch, v), o) for (q, k, v), o in zip(projs, outs)]
    ctx = ops.Context(0, synchronous=False)
    s = sess_mod.Session(ctx, sess_mod.Options(
        capacity=total, prefill_chunk_size=128, vocab_size=262144, layers=layers, query_heads=hq,
        kv_heads=hkv, head_dim=D, storage="bf16", score_scale=1.0 / 16.0, softcap=50.0, theta=1e6,
        layer_windows=windows))
    s.set_tokens([3] * prompt)
    assert s.evaluate(io) == prompt
    s.append([4] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    s.synchronize()
    rows = sorted({p for c in (0, 7, 8, 9, 16, 31) for p in (c * 128, c * 128 + 127)}
                  | {prompt, prompt + 63, total - 1})
    w = rng.standard_normal((2048, hq * D)).astype(np.float32)
    for layer in range(layers):
        qp, kp, vp = projs[layer]
        k = _produce(orc, kp, None, total, hkv, D, 0, 1e6, "bf16").transpose(1, 0, 2).copy()
        v = stored(vp, "bf16").transpose(1, 0, 2).copy()
        got = host(outs[layer])
        worst, refs, gots = 0.0, [], []
        for p in rows:
            lo = max(0, p - W + 1) if windows[layer] else 0
            n = p + 1 - lo
            q = _produce(orc, qp[p:p + 1], None, 1, hq, D, p, 1e6, "bf16").reshape(-1)
            ref, _, _ = orc.window_attention(q, k[:, lo:p + 1].reshape(-1), v[:, lo:p + 1].reshape(-1),
                                             1, n, n, hq, hkv, D, p, lo,
                                             W if windows[layer] else None, 1.0 / 16.0, softcap=50.0)
            worst = max(worst, max_err(got[p], ref))
            refs.append(ref)
            gots.append(got[p])
        assert_tokens_identical(np.stack(gots), np.stack(refs), w)
        log(f"configs[3] layer {layer} ({'W=1024' if windows[layer] else 'global'}): {len(rows)} rows, "
            f"max abs error {worst:.3e}, greedy tokens identical")
        assert worst <= TOL_HALF
    s.close()
    ctx.close()


def test_configs4_batched_prefill_full_size(torch_mod, ops, orc):
    """per session, N(0, 1) FP32 Q/K/V projections (5% of K rows x8)
    through tkh_produce_qkv with split-half rotary theta 500000: the 4096 cached
    positions into the session's bf16 cache, then the 128 new ones (Q to the
    batch, K/V appended); then one tkh_prefill_batch.  Sessions 0 and 31 are
    checked against the oracle's rotary -> bf16 rounding -> attention_cached
    (src/cpu/attention.rs:10-64, :201-296), with identical greedy tokens."""
    torch = torch_mod
    hq, hkv, D, B, cached, tokens, theta = 32, 8, 128, 32, 4096, 128, 5e5
    cap = cached + tokens
    per = hkv * cap * D
    ctx = ops.Context(0)
    gd = torch.Generator(device="cuda").manual_seed(104)
    k = torch.empty(B * per, dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    q = torch.empty(B, tokens, hq, D, dtype=torch.bfloat16, device="cuda")
    q_prefix = torch.zeros(cached, hq, D, device="cuda")  # the cached positions' Q is not used
    q_scratch = torch.empty(cached, hq, D, dtype=torch.bfloat16, device="cuda")
    kept = {}
    for b in range(B):
        kp = torch.randn(cap, hkv, D, generator=gd, device="cuda")
        mask = torch.rand(cap, hkv, 1, generator=gd, device="cuda") < 0.05
        kp = torch.where(mask, kp * 8.0, kp)
        vp = torch.randn(cap, hkv, D, generator=gd, device="cuda")
        qp = torch.randn(tokens, hq, D, generator=gd, device="cuda")
        kb, vb = k[b * per:(b + 1) * per], v[b * per:(b + 1) * per]
        ops.produce_qkv(ctx, ops.ProducerShape(cached, hq, hkv, D, 0, theta=theta), q_prefix,
                        kp[:cached], vp[:cached], None, None, q_scratch, kb, vb, cap * D)
        ops.produce_qkv(ctx, ops.ProducerShape(tokens, hq, hkv, D, cached, theta=theta), qp,
                        kp[cached:], vp[cached:], None, None, q[b], kb[cached * D:],
                        vb[cached * D:], cap * D)
        if b in (0, B - 1):
            kept[b] = (host(qp), host(kp), host(vp))
    out = torch.full((B * tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.prefill_batch(ctx, q, k, v, [b * per for b in range(B)], [cap * D] * B,
                      [cached] * B, out, tokens=tokens, query_heads=hq, kv_heads=hkv, head_dim=D,
                      scale=1.0 / math.sqrt(D))
    got = host(out).reshape(B, tokens * hq * D)
    assert np.all(np.isfinite(got))
    rng = np.random.default_rng(104)
    w = rng.standard_normal((2048, hq * D)).astype(np.float32)
    for b, (qp, kp, vp) in kept.items():
        qr = _produce(orc, qp, None, tokens, hq, D, cached, theta, "bf16").reshape(-1)
        kr = _produce(orc, kp, None, cap, hkv, D, 0, theta, "bf16").transpose(1, 0, 2).reshape(-1)
        vr = stored(vp, "bf16").transpose(1, 0, 2).reshape(-1)
        ref, _, _ = orc.attention_cached(qr, kr, vr, tokens, hq, hkv, D, cap, cached)
        err = max_err(got[b], ref)
        assert_tokens_identical(got[b].reshape(tokens, -1), ref.reshape(tokens, -1), w)
        log(f"configs[4] session {b} (rotary theta 5e5; 128 rows x 32 heads over 4224 keys): "
            f"max abs error {err:.3e}, greedy tokens identical")
        assert err <= TOL_HALF
    ctx.close()


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_full_prefix_attention_token_major_half(torch_mod, ops, orc, dt):
    """tkh_attention (src/cpu/attention.rs:85): token-major K/V [T, Hkv, D] as a strided
    segment through the MFMA chunk kernel."""
    torch = torch_mod
    rng = np.random.default_rng(105)
    T, hq, hkv, D = 300, 16, 8, 128
    q = stored(rng.standard_normal((T, hq, D)), dt).reshape(-1)
    k = stored(rng.standard_normal((T, hkv, D)), dt).reshape(-1)
    v = stored(rng.standard_normal((T, hkv, D)), dt).reshape(-1)
    out = torch.full((T * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ctx = ops.Context(0)
    ops.attention(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None,
                  ops.AttentionShape(T, hq, hkv, D))
    ref, _, _ = orc.attention(q, k, v, T, hq, hkv, D)
    err = max_err(host(out), ref)
    log(f"full-prefix attention {dt} {T} tokens: max abs error {err:.3e}")
    assert err <= TOL_HALF
    ctx.close()
