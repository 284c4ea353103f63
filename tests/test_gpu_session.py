"""GPU parity of the producer (RMSNorm -> rotary -> cache rounding) and of the
session driver (tkh_session) against the CPU oracle.

The producer is compared with the oracle's rmsnorm and rotary on the same FP32
projections; the session's per-layer contexts with full-prefix attention over
the oracle-produced (and cache-rounded) Q/K/V, which is what the reference's
session equals (tests/session.rs:262-306, src/cpu/attention.rs:194-195).
"""

import numpy as np
import pytest

from gpu_util import TOL_HALF, host, log, max_err, stored

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


@pytest.fixture(scope="module")
def ctx(torch_mod, ops):
    return ops.Context(0)


def _t(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")
    return t if dtype is None else t.to(dtype)


def _oracle_produce(orc, x, w, tokens, heads, D, position, *, eps=1e-6, rotary="split",
                    theta=1e6, rotated=0, factor=1.0, low=1.0, high=4.0, original=8192):
    y = orc.rmsnorm(x.reshape(-1), w, tokens * heads, D, eps) if w is not None else x.reshape(-1)
    if rotary == "split":
        y = orc.rotary(y, tokens, heads, D, position, theta)
    elif rotary == "proportional":
        y = orc.proportional_rotary(y, tokens, heads, D, rotated, position, theta, factor)
    elif rotary == "llama3":
        y = orc.llama3_rotary(y, tokens, heads, D, position, theta, factor, low, high, original)
    return y.reshape(tokens, heads, D)


def _ulp_diff_f32(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


@pytest.mark.parametrize("norm", [True, False])
def test_producer_qwen3_norm_rotary_f32(torch_mod, ctx, ops, orc, norm):
    """FP32 outputs against the oracle within 1 ulp (FP64 sum order and device
    sin/cos/pow may move a rounding tie); V copied exactly; K/V head-major."""
    torch = torch_mod
    rng = np.random.default_rng(1)
    T, hq, hkv, D, pos, cap = 37, 16, 8, 128, 2000, 64
    q = rng.standard_normal((T, hq, D)).astype(np.float32) * 3
    k = rng.standard_normal((T, hkv, D)).astype(np.float32) * 3
    v = rng.standard_normal((T, hkv, D)).astype(np.float32)
    wq = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32) if norm else None
    wk = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32) if norm else None
    qo = torch.zeros(T * hq * D, dtype=torch.float32, device="cuda")
    kc = torch.full((hkv, cap, D), np.nan, dtype=torch.float32, device="cuda")
    vc = torch.full((hkv, cap, D), np.nan, dtype=torch.float32, device="cuda")
    off = 9
    ops.produce_qkv(ctx, ops.ProducerShape(T, hq, hkv, D, pos), _t(torch, q), _t(torch, k),
                    _t(torch, v), _t(torch, wq) if norm else None, _t(torch, wk) if norm else None,
                    qo, kc[:, off:], vc[:, off:], cap * D)
    rq = _oracle_produce(orc, q, wq, T, hq, D, pos)
    rk = _oracle_produce(orc, k, wk, T, hkv, D, pos)
    gq = host(qo).reshape(T, hq, D)
    gk = host(kc)[:, off:off + T].transpose(1, 0, 2)
    gv = host(vc)[:, off:off + T].transpose(1, 0, 2)
    for name, g, r in (("q", gq, rq), ("k", gk, rk)):
        u = _ulp_diff_f32(g, r)
        log(f"{name}: exact {np.mean(u == 0):.6f}, max ulp {u.max()}")
        assert u.max() <= 1 and np.mean(u == 0) > 0.999
    assert np.array_equal(gv, v)
    assert np.isnan(host(kc)[:, :off]).all() and np.isnan(host(kc)[:, off + T:]).all()


def test_producer_proportional_partial_bf16(torch_mod, ctx, ops, orc):
    """Gemma geometry (8/4/256), proportional rotary on 64 of 256 features, bf16 outputs:
    equal to the oracle's FP32 result rounded once, up to one bf16 ulp at ties."""
    torch = torch_mod
    rng = np.random.default_rng(2)
    T, hq, hkv, D, pos = 20, 8, 4, 256, 4000
    q = rng.standard_normal((T, hq, D)).astype(np.float32)
    k = rng.standard_normal((T, hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, hkv, D)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    qo = torch.zeros(T * hq * D, dtype=torch.bfloat16, device="cuda")
    ko = torch.zeros(hkv * T * D, dtype=torch.bfloat16, device="cuda")
    vo = torch.zeros(hkv * T * D, dtype=torch.bfloat16, device="cuda")
    shape = ops.ProducerShape(T, hq, hkv, D, pos, 1e-6, ops.ROTARY_PROPORTIONAL, 1e6, 64, 8.0)
    ops.produce_qkv(ctx, shape, _t(torch, q), _t(torch, k), _t(torch, v), _t(torch, w), _t(torch, w),
                    qo, ko, vo, T * D)
    rq = stored(_oracle_produce(orc, q, w, T, hq, D, pos, rotary="proportional", rotated=64, factor=8.0), "bf16")
    rk = stored(_oracle_produce(orc, k, w, T, hkv, D, pos, rotary="proportional", rotated=64, factor=8.0), "bf16")
    gq = host(qo).reshape(T, hq, D)
    gk = host(ko).reshape(hkv, T, D).transpose(1, 0, 2)
    for g, r in ((gq, rq), (gk, rk)):
        d = np.abs(g - r)
        assert np.mean(d == 0) > 0.999
        assert np.all(d <= np.abs(r) * 2.0 ** -7 + 1e-30)
    assert np.array_equal(host(vo).reshape(hkv, T, D).transpose(1, 0, 2), stored(v, "bf16"))


def _llama3_shape(ops, T, hq, hkv, D, pos, theta, factor, low, high, original):
    return ops.ProducerShape(T, hq, hkv, D, pos, 1e-6, ops.ROTARY_LLAMA3, theta, 0, factor, low,
                             high, original)


def test_producer_llama3_matches_llama3_rotary_fixture(torch_mod, ctx, ops, orc):
    """Every case of llama3-rotary-v1 through the producer (Q heads, no norm, FP32):
    within the reference's gate 1e-5 + 1e-4|e| of the frozen outputs
    (src/cpu/llama3_rotary/tests.rs:63-95), and within 1 ulp of the oracle."""
    from goldens import Golden, close

    torch = torch_mod
    g = Golden("llama3_rotary_v1")
    for case in g.meta["cases"]:
        name, T, H, D = case["name"], case["tokens"], case["heads"], case["head_dim"]
        x = g.arrays[f"{name}.input"].reshape(T, H, D)
        zeros = np.zeros((T, 1, D), np.float32)
        qo = torch.full((T * H * D,), np.nan, dtype=torch.float32, device="cuda")
        ko = torch.zeros(T * D, dtype=torch.float32, device="cuda")
        vo = torch.zeros(T * D, dtype=torch.float32, device="cuda")
        shape = _llama3_shape(ops, T, H, 1, D, case["offset"], case["theta"], case["factor"],
                              case["low"], case["high"], case["original"])
        ops.produce_qkv(ctx, shape, _t(torch, x), _t(torch, zeros), _t(torch, zeros), None, None,
                        qo, ko, vo, T * D)
        got = host(qo)
        close(got, g.arrays[f"{name}.output"])
        ref = orc.llama3_rotary(x.reshape(-1), T, H, D, case["offset"], case["theta"],
                                case["factor"], case["low"], case["high"], case["original"])
        u = _ulp_diff_f32(got, ref)
        log(f"{name}: max ulp {u.max()}")
        assert u.max() <= 1


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_producer_llama3_across_original_context_edge(torch_mod, ctx, ops, orc, dtype):
    """Llama 3.1 8B geometry (32/8/128, theta 500000, factor 8, bands 1/4 over 8192)
    at positions 8160..8223, across the original context length: FP32 within 1 ulp
    of the oracle (device pow/sin/cos may move a rounding tie), bf16 equal to the
    oracle rounded once up to a bf16 ulp at ties; V copied."""
    torch = torch_mod
    rng = np.random.default_rng(11)
    T, hq, hkv, D, pos = 64, 32, 8, 128, 8160
    q = rng.standard_normal((T, hq, D)).astype(np.float32) * 2
    k = rng.standard_normal((T, hkv, D)).astype(np.float32) * 2
    v = rng.standard_normal((T, hkv, D)).astype(np.float32)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    qo = torch.zeros(T * hq * D, dtype=tdt, device="cuda")
    ko = torch.zeros(hkv * T * D, dtype=tdt, device="cuda")
    vo = torch.zeros(hkv * T * D, dtype=tdt, device="cuda")
    shape = _llama3_shape(ops, T, hq, hkv, D, pos, 500000.0, 8.0, 1.0, 4.0, 8192)
    ops.produce_qkv(ctx, shape, _t(torch, q), _t(torch, k), _t(torch, v), None, None, qo, ko, vo,
                    T * D)
    kw = dict(rotary="llama3", theta=500000.0, factor=8.0, low=1.0, high=4.0, original=8192)
    rq = _oracle_produce(orc, q, None, T, hq, D, pos, **kw)
    rk = _oracle_produce(orc, k, None, T, hkv, D, pos, **kw)
    gq = host(qo).reshape(T, hq, D)
    gk = host(ko).reshape(hkv, T, D).transpose(1, 0, 2)
    gv = host(vo).reshape(hkv, T, D).transpose(1, 0, 2)
    for name, gg, r in (("q", gq, rq), ("k", gk, rk)):
        if dtype == "f32":
            u = _ulp_diff_f32(gg, r)
            log(f"{name}: exact {np.mean(u == 0):.6f}, max ulp {u.max()}")
            assert u.max() <= 1 and np.mean(u == 0) > 0.999
        else:
            r = stored(r, "bf16")
            d = np.abs(gg - r)
            assert np.mean(d == 0) > 0.999
            assert np.all(d <= np.abs(r) * 2.0 ** -7 + 1e-30)
    assert np.array_equal(gv, v if dtype == "f32" else stored(v, "bf16"))
    # The scaling matters here: the ordinary rotary differs from both.
    plain = _oracle_produce(orc, q, None, T, hq, D, pos, rotary="split", theta=500000.0)
    assert not np.allclose(plain, rq, atol=1e-3)


def test_producer_nonfinite_input_reports(torch_mod, ctx, ops):
    torch = torch_mod
    T, hq, hkv, D = 2, 2, 1, 64
    q = np.ones((T, hq, D), np.float32)
    q[1, 1, 5] = np.inf
    k = np.ones((T, hkv, D), np.float32)
    v = np.ones((T, hkv, D), np.float32)
    out = [torch.zeros(n, dtype=torch.float32, device="cuda") for n in (T * hq * D, T * hkv * D, T * hkv * D)]
    with pytest.raises(ops.TkhError) as e:
        ops.produce_qkv(ctx, ops.ProducerShape(T, hq, hkv, D, 0), _t(torch, q), _t(torch, k),
                        _t(torch, v), None, None, out[0], out[1], out[2], T * D)
    assert e.value.name == "NonFinite"


def _session_inputs(rng, layers, total, hq, hkv, D, scale=1.0):
    qs = [rng.standard_normal((total, hq, D)).astype(np.float32) * scale for _ in range(layers)]
    ks = [rng.standard_normal((total, hkv, D)).astype(np.float32) * scale for _ in range(layers)]
    vs = [rng.standard_normal((total, hkv, D)).astype(np.float32) for _ in range(layers)]
    wq = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float32) for _ in range(layers)]
    wk = [(1 + 0.02 * rng.standard_normal(D)).astype(np.float32) for _ in range(layers)]
    return qs, ks, vs, wq, wk


def test_session_qwen3_prefill_chunks_then_decode_steps(torch_mod, ctx, ops, sess_mod, orc):
    """Two Qwen3-shaped layers (16/8/128, bf16 KV, QK-norm, rotary 1e6, position offset 7):
    300 prompt tokens in 128-token chunks, then 6 single-token decode steps.  Each
    layer's contexts equal full-prefix attention over the oracle-produced Q/K/V."""
    torch = torch_mod
    rng = np.random.default_rng(3)
    L, hq, hkv, D, prompt, steps, off = 2, 16, 8, 128, 300, 6, 7
    total = prompt + steps
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
    opts = sess_mod.Options(capacity=total + 10, prefill_chunk_size=128, position_offset=off,
                            vocab_size=1000, layers=L, query_heads=hq, kv_heads=hkv, head_dim=D,
                            storage="bf16")
    s = sess_mod.Session(ctx, opts)
    ctxs = [torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda") for _ in range(L)]
    io = [sess_mod.LayerIo(_t(torch, qs[l]), _t(torch, ks[l]), _t(torch, vs[l]), ctxs[l],
                           _t(torch, wq[l]), _t(torch, wk[l])) for l in range(L)]
    tokens = list(rng.integers(0, 1000, total))
    s.set_tokens(tokens[:prompt])
    assert s.evaluate(io) == prompt
    s.append(tokens[prompt:])
    assert s.evaluate(io, chunk_limit=1) == steps
    assert (s.evaluated_len(), s.pending_len()) == (total, 0) and s.distribution_valid()
    for l in range(L):
        q = stored(_oracle_produce(orc, qs[l], wq[l], total, hq, D, off), "bf16")
        k = stored(_oracle_produce(orc, ks[l], wk[l], total, hkv, D, off), "bf16")
        v = stored(vs[l], "bf16")
        ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), v.reshape(-1), total, hq, hkv, D)
        err = max_err(host(ctxs[l]).reshape(-1), ref)
        log(f"layer {l}: max abs error {err:.3e}")
        assert err <= TOL_HALF


@pytest.mark.parametrize("fused", ["1", "0"])
def test_session_sliding_and_global_layers_gemma_shape(torch_mod, ctx, ops, sess_mod, orc, fused):
    """A sliding (W=64, ring cache) and a global layer at 8/4/256, scale 1/16, score
    softcap 50, proportional rotary: 200 prompt tokens in 64-token chunks, 5 decode steps.
    fused "1": the decode steps fold the producer into the decode launch (new K/V row
    to the ring's staging row, then the batched ring commit); "0": separate launches."""
    import os

    torch = torch_mod
    rng = np.random.default_rng(4)
    L, hq, hkv, D, prompt, steps, W = 2, 8, 4, 256, 200, 5, 64
    total = prompt + steps
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D, scale=2.0)
    opts = sess_mod.Options(capacity=total, prefill_chunk_size=64, vocab_size=100, layers=L,
                            query_heads=hq, kv_heads=hkv, head_dim=D, storage="bf16",
                            score_scale=1.0 / 16.0, softcap=50.0, rotary=2, theta=1e6,
                            rotated_dims=128, factor=8.0, layer_windows=[W, 0])
    saved = os.environ.get("TKH_FUSED_DECODE")
    os.environ["TKH_FUSED_DECODE"] = fused
    try:
        s = sess_mod.Session(ctx, opts)
    finally:
        if saved is None:
            os.environ.pop("TKH_FUSED_DECODE", None)
        else:
            os.environ["TKH_FUSED_DECODE"] = saved
    ctxs = [torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda") for _ in range(L)]
    io = [sess_mod.LayerIo(_t(torch, qs[l]), _t(torch, ks[l]), _t(torch, vs[l]), ctxs[l],
                           _t(torch, wq[l]), _t(torch, wk[l])) for l in range(L)]
    s.set_tokens([1] * prompt)
    assert s.evaluate(io) == prompt
    s.append([2] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    for l, window in enumerate([W, None]):
        kw = dict(rotary="proportional", theta=1e6, rotated=128, factor=8.0)
        q = stored(_oracle_produce(orc, qs[l], wq[l], total, hq, D, 0, **kw), "bf16")
        k = stored(_oracle_produce(orc, ks[l], wk[l], total, hkv, D, 0, **kw), "bf16")
        v = stored(vs[l], "bf16")
        kh = k.transpose(1, 0, 2).copy()
        vh = v.transpose(1, 0, 2).copy()
        ref, _, _ = orc.window_attention(q.reshape(-1), kh.reshape(-1), vh.reshape(-1), total, total,
                                         total, hq, hkv, D, 0, 0, window, 1.0 / 16.0, softcap=50.0)
        err = max_err(host(ctxs[l]).reshape(-1), ref)
        log(f"fused {fused} layer {l} window {window}: max abs error {err:.3e}")
        assert err <= TOL_HALF


@pytest.mark.parametrize("fused", ["1", "0"])
def test_session_llama3_rotary_prefill_then_decode(torch_mod, ctx, ops, sess_mod, orc, fused):
    """Llama 3.2 1B attention geometry (32/8/64, theta 500000, factor 32, bands 1/4
    over 8192), bf16 KV, no QK-norm, position offset 8100: 200 prompt tokens in
    64-token chunks, then 4 decode steps, crossing the original context length.
    Each context equals full-prefix attention over the oracle's Llama 3 rotary
    (PositionPlan::Llama3, src/model/position.rs:32-43)."""
    import os

    torch = torch_mod
    rng = np.random.default_rng(12)
    L, hq, hkv, D, prompt, steps, off = 1, 32, 8, 64, 200, 4, 8100
    total = prompt + steps
    qs, ks, vs, _, _ = _session_inputs(rng, L, total, hq, hkv, D)
    opts = sess_mod.Options(capacity=total, prefill_chunk_size=64, position_offset=off,
                            vocab_size=100, layers=L, query_heads=hq, kv_heads=hkv, head_dim=D,
                            storage="bf16", rotary=ops.ROTARY_LLAMA3, theta=500000.0, factor=32.0,
                            low_freq_factor=1.0, high_freq_factor=4.0, original_max_positions=8192)
    saved = os.environ.get("TKH_FUSED_DECODE")
    os.environ["TKH_FUSED_DECODE"] = fused
    try:
        s = sess_mod.Session(ctx, opts)
    finally:
        if saved is None:
            os.environ.pop("TKH_FUSED_DECODE", None)
        else:
            os.environ["TKH_FUSED_DECODE"] = saved
    out = torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda")
    io = [sess_mod.LayerIo(_t(torch, qs[0]), _t(torch, ks[0]), _t(torch, vs[0]), out, None, None)]
    s.set_tokens([3] * prompt)
    assert s.evaluate(io) == prompt
    s.append([4] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    kw = dict(rotary="llama3", theta=500000.0, factor=32.0, low=1.0, high=4.0, original=8192)
    q = stored(_oracle_produce(orc, qs[0], None, total, hq, D, off, **kw), "bf16")
    k = stored(_oracle_produce(orc, ks[0], None, total, hkv, D, off, **kw), "bf16")
    v = stored(vs[0], "bf16")
    ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), v.reshape(-1), total, hq, hkv, D)
    err = max_err(host(out).reshape(-1), ref)
    log(f"fused {fused}: max abs error {err:.3e}")
    assert err <= TOL_HALF
    s.close()


@pytest.mark.parametrize("fused", ["1", "0"])
def test_session_shared_kv_layers_attend_over_their_producers(torch_mod, ctx, ops, sess_mod, orc,
                                                               fused):
    """Six Gemma-shaped layers (8/4/256, bf16, scale 1/16, softcap 50, proportional
    rotary), kinds sliding/full alternating with window 64, the last three shared
    (gemma-shared-kv-v1's alternating6 routing: 3 -> 1, 4 -> 2, 5 -> 1): 150 prompt
    tokens in 64-token chunks, then 4 decode steps.  A shared layer's context is its
    own Q (own q_norm) over its producer's K/V (the producer's k_norm), with its own
    window; its K/V projections are passed as None and never read."""
    import os

    torch = torch_mod
    rng = np.random.default_rng(14)
    L, hq, hkv, D, prompt, steps, W, shared = 6, 8, 4, 256, 150, 4, 64, 3
    total = prompt + steps
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D, scale=2.0)
    windows = [W, 0, W, 0, W, 0]
    opts = sess_mod.Options(capacity=total, prefill_chunk_size=64, vocab_size=100, layers=L,
                            query_heads=hq, kv_heads=hkv, head_dim=D, storage="bf16",
                            score_scale=1.0 / 16.0, softcap=50.0, rotary=2, theta=1e6,
                            rotated_dims=128, factor=8.0, layer_windows=windows,
                            shared_layers=shared)
    saved = os.environ.get("TKH_FUSED_DECODE")
    os.environ["TKH_FUSED_DECODE"] = fused
    try:
        s = sess_mod.Session(ctx, opts)
    finally:
        if saved is None:
            os.environ.pop("TKH_FUSED_DECODE", None)
        else:
            os.environ["TKH_FUSED_DECODE"] = saved
    route = [s.kv_producer(l) for l in range(L)]
    assert route == [0, 1, 2, 1, 2, 1]
    ctxs = [torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda") for _ in range(L)]
    io = []
    for l in range(L):
        own = l < L - shared
        io.append(sess_mod.LayerIo(_t(torch, qs[l]), _t(torch, ks[l]) if own else None,
                                   _t(torch, vs[l]) if own else None, ctxs[l], _t(torch, wq[l]),
                                   _t(torch, wk[l]) if own else None))
    s.set_tokens([1] * prompt)
    assert s.evaluate(io) == prompt
    s.append([2] * steps)
    assert s.evaluate(io, chunk_limit=1) == steps
    kw = dict(rotary="proportional", theta=1e6, rotated=128, factor=8.0)
    for l in range(L):
        p = route[l]
        q = stored(_oracle_produce(orc, qs[l], wq[l], total, hq, D, 0, **kw), "bf16")
        k = stored(_oracle_produce(orc, ks[p], wk[p], total, hkv, D, 0, **kw), "bf16")
        v = stored(vs[p], "bf16")
        kh = k.transpose(1, 0, 2).copy()
        vh = v.transpose(1, 0, 2).copy()
        window = windows[l] or None
        ref, _, _ = orc.window_attention(q.reshape(-1), kh.reshape(-1), vh.reshape(-1), total, total,
                                         total, hq, hkv, D, 0, 0, window, 1.0 / 16.0, softcap=50.0)
        err = max_err(host(ctxs[l]).reshape(-1), ref)
        log(f"fused {fused} layer {l} (KV of layer {p}, window {window}): max abs error {err:.3e}")
        assert err <= TOL_HALF
    assert s.memory()["kv_bytes"] > 0
    s.close()


@pytest.mark.parametrize("shape", ["qwen3", "gemma"])
@pytest.mark.parametrize("queued", [False, True])
@pytest.mark.parametrize("fused", ["1", "0"])
def test_layer_by_layer_chunks_with_layer_dependent_inputs(torch_mod, ops, sess_mod, orc, shape,
                                                           queued, fused):
    """A host whose next layer depends on this one (Model::run, src/model/mod.rs:530-755):
    three layers through tkh_session_chunk_*, layer l + 1's Q/K/V made on the device
    from layer l's context of the same chunk.  qwen3: 16/8/128 linear caches, QK-norm,
    attention_cached semantics; gemma: 8/4/256 with a sliding (W = 64, ring) layer
    between two global ones, scale 1/16, softcap 50, proportional rotary.  150 prompt
    tokens in 64-token chunks, then 3 decode steps, with a synchronous or a queued
    context.  Every layer matches attention over the oracle-produced Q/K/V of the
    inputs it was given, and feeding those inputs to tkh_session_evaluate gives the
    same contexts bit for bit."""
    import os

    torch = torch_mod
    ctx = ops.Context(0, synchronous=not queued)
    rng = np.random.default_rng(15)
    if shape == "qwen3":
        L, hq, hkv, D = 3, 16, 8, 128
        windows, extra = None, {}
        kw = {}
    else:
        L, hq, hkv, D = 3, 8, 4, 256
        windows = [0, 64, 0]
        extra = dict(score_scale=1.0 / 16.0, softcap=50.0, rotary=2, theta=1e6, rotated_dims=128,
                     factor=8.0, layer_windows=windows)
        kw = dict(rotary="proportional", theta=1e6, rotated=128, factor=8.0)
    prompt, steps = 150, 3
    total = prompt + steps
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
    opts = sess_mod.Options(capacity=total, prefill_chunk_size=64, vocab_size=100, layers=L,
                            query_heads=hq, kv_heads=hkv, head_dim=D, storage="bf16", **extra)

    def session():
        saved = os.environ.get("TKH_FUSED_DECODE")
        os.environ["TKH_FUSED_DECODE"] = fused
        try:
            return sess_mod.Session(ctx, opts)
        finally:
            if saved is None:
                os.environ.pop("TKH_FUSED_DECODE", None)
            else:
                os.environ["TKH_FUSED_DECODE"] = saved

    s = session()
    q_all = [np.zeros((total, hq, D), np.float32) for _ in range(L)]
    k_all = [np.zeros((total, hkv, D), np.float32) for _ in range(L)]
    v_all = [np.zeros((total, hkv, D), np.float32) for _ in range(L)]
    ctx_all = [np.zeros((total, hq * D), np.float32) for _ in range(L)]
    wq_d = [_t(torch, w) for w in wq]
    wk_d = [_t(torch, w) for w in wk]
    s.set_tokens([5] * prompt)
    for limit, todo in ((64, prompt), (1, steps)):
        if limit == 1:
            s.append([6] * steps)
        done = 0
        while done < todo:
            start, n = s.chunk_begin(limit)
            assert n > 0
            prev = None
            for l in range(L):
                if l == 0:
                    q = _t(torch, qs[0][start:start + n])
                    k = _t(torch, ks[0][start:start + n])
                    v = _t(torch, vs[0][start:start + n])
                else:
                    c = prev.view(n, hq, D)
                    q = (0.5 * c + _t(torch, qs[l][start:start + n])).contiguous()
                    k = (0.5 * c[:, :hkv] + _t(torch, ks[l][start:start + n])).contiguous()
                    v = (c[:, hkv:2 * hkv] + _t(torch, vs[l][start:start + n])).contiguous()
                out = torch.full((n, hq * D), np.nan, dtype=torch.float32, device="cuda")
                s.chunk_layer(l, sess_mod.LayerIo(q, k, v, out, wq_d[l], wk_d[l]))
                q_all[l][start:start + n] = host(q).reshape(n, hq, D)
                k_all[l][start:start + n] = host(k).reshape(n, hkv, D)
                v_all[l][start:start + n] = host(v).reshape(n, hkv, D)
                ctx_all[l][start:start + n] = host(out).reshape(n, hq * D)
                prev = out
            assert s.chunk_commit() == n
            done += n
    s.synchronize()
    assert (s.evaluated_len(), s.pending_len()) == (total, 0) and s.distribution_valid()
    for l in range(L):
        q = stored(_oracle_produce(orc, q_all[l], wq[l], total, hq, D, 0, **kw), "bf16")
        k = stored(_oracle_produce(orc, k_all[l], wk[l], total, hkv, D, 0, **kw), "bf16")
        v = stored(v_all[l], "bf16")
        if shape == "qwen3":
            ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), v.reshape(-1), total, hq, hkv, D)
        else:
            kh = k.transpose(1, 0, 2).copy()
            vh = v.transpose(1, 0, 2).copy()
            ref, _, _ = orc.window_attention(q.reshape(-1), kh.reshape(-1), vh.reshape(-1), total,
                                             total, total, hq, hkv, D, 0, 0, windows[l] or None,
                                             1.0 / 16.0, softcap=50.0)
        err = max_err(ctx_all[l].reshape(-1), ref)
        log(f"{shape} queued {queued} fused {fused} layer {l}: max abs error {err:.3e}")
        assert err <= TOL_HALF
    # The whole-chunk calls on the same inputs: the same kernels, the same bits.
    s2 = session()
    outs = [torch.full((total, hq * D), np.nan, dtype=torch.float32, device="cuda") for _ in range(L)]
    io = [sess_mod.LayerIo(_t(torch, q_all[l]), _t(torch, k_all[l]), _t(torch, v_all[l]), outs[l],
                           wq_d[l], wk_d[l]) for l in range(L)]
    s2.set_tokens([5] * prompt)
    assert s2.evaluate(io, chunk_limit=64) == prompt
    s2.append([6] * steps)
    assert s2.evaluate(io, chunk_limit=1) == steps
    s2.synchronize()
    for l in range(L):
        assert np.array_equal(host(outs[l]).reshape(total, -1).view(np.uint32),
                              ctx_all[l].view(np.uint32)), l
    s.close()
    s2.close()


def test_session_failed_chunk_commits_nothing_and_retry_succeeds(torch_mod, ctx, ops, sess_mod, orc):
    """src/session.rs:357-363: a chunk whose layer fails leaves the committed prefix
    and the pending history; fixing the input and evaluating again succeeds."""
    torch = torch_mod
    rng = np.random.default_rng(5)
    L, hq, hkv, D, total = 1, 4, 2, 64, 40
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
    opts = sess_mod.Options(capacity=64, prefill_chunk_size=16, vocab_size=10, layers=L,
                            query_heads=hq, kv_heads=hkv, head_dim=D, storage="f32")
    s = sess_mod.Session(ctx, opts)
    out = torch.zeros((total, hq * D), dtype=torch.float32, device="cuda")
    kbad = ks[0].copy()
    kbad[20, 1, 3] = np.nan
    io = [sess_mod.LayerIo(_t(torch, qs[0]), _t(torch, kbad), _t(torch, vs[0]), out, None, None)]
    s.set_tokens([3] * total)
    assert s.evaluate_next_chunk(io) == 16   # rows 0..15 are clean
    with pytest.raises(ops.TkhError) as e:
        s.evaluate(io)
    assert e.value.name == "NonFinite"
    assert (s.evaluated_len(), s.pending_len()) == (16, 24)
    io[0].k_proj = _t(torch, ks[0])
    assert s.evaluate(io) == 24
    q = _oracle_produce(orc, qs[0], None, total, hq, D, 0)
    k = _oracle_produce(orc, ks[0], None, total, hkv, D, 0)
    ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), vs[0].reshape(-1), total, hq, hkv, D)
    err = max_err(host(out).reshape(-1), ref)
    log(f"fp32 session after retry: max abs error {err:.3e}")
    assert err <= 1e-5


def test_session_queued_context_matches_synchronous(torch_mod, ops, sess_mod):
    """A queued context evaluates without per-chunk host waits; after synchronize the
    contexts are bit-identical to a synchronous context's."""
    torch = torch_mod
    rng = np.random.default_rng(6)
    L, hq, hkv, D, total = 1, 16, 8, 128, 150
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
    outs = []
    for sync in (True, False):
        c = ops.Context(0, synchronous=sync)
        s = sess_mod.Session(c, sess_mod.Options(capacity=total, prefill_chunk_size=128, layers=1,
                                                 query_heads=hq, kv_heads=hkv, head_dim=D))
        out = torch.zeros((total, hq * D), dtype=torch.float32, device="cuda")
        io = [sess_mod.LayerIo(_t(torch, qs[0]), _t(torch, ks[0]), _t(torch, vs[0]), out,
                               _t(torch, wq[0]), _t(torch, wk[0]))]
        s.set_tokens([1] * 140)
        s.evaluate(io)
        s.append([1] * 10)
        s.evaluate(io, chunk_limit=1)
        s.synchronize()
        assert s.evaluated_len() == total
        outs.append(host(out))
        s.close()
        c.close()
    assert np.array_equal(outs[0], outs[1])


def test_queued_ring_session_failure_rolls_back_to_last_ring_commit(torch_mod, ops, sess_mod, orc):
    """Queued context, a sliding (W=32, ring) and a global layer, chunks of 16: a NaN in
    the fourth chunk's keys surfaces at synchronize; the session stands at the end of
    the third chunk (its last ring commit), and evaluating again from there with clean
    inputs matches the oracle, so the rings held exactly the committed chunks."""
    torch = torch_mod
    rng = np.random.default_rng(7)
    L, hq, hkv, D, total, W = 2, 4, 2, 64, 100, 32
    qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
    c = ops.Context(0, synchronous=False)
    s = sess_mod.Session(c, sess_mod.Options(capacity=total, prefill_chunk_size=16, vocab_size=10,
                                             layers=L, query_heads=hq, kv_heads=hkv, head_dim=D,
                                             storage="f16", score_scale=0.125,
                                             layer_windows=[W, 0]))
    ctxs = [torch.zeros((total, hq * D), dtype=torch.float32, device="cuda") for _ in range(L)]
    kbad = ks[0].copy()
    kbad[50, 0, 7] = np.nan   # chunk [48, 64)
    io = [sess_mod.LayerIo(_t(torch, qs[l]), _t(torch, kbad if l == 0 else ks[l]), _t(torch, vs[l]),
                           ctxs[l], _t(torch, wq[l]), _t(torch, wk[l])) for l in range(L)]
    s.set_tokens([1] * total)
    assert s.evaluate(io) == total          # queued: nothing checked yet
    with pytest.raises(ops.TkhError) as e:
        s.synchronize()
    assert e.value.name == "NonFinite"
    assert (s.evaluated_len(), s.pending_len()) == (48, total - 48)
    io[0].k_proj = _t(torch, ks[0])
    assert s.evaluate(io) == total - 48
    s.synchronize()
    for l, window in enumerate([W, None]):
        q = stored(_oracle_produce(orc, qs[l], wq[l], total, hq, D, 0), "f16")
        k = stored(_oracle_produce(orc, ks[l], wk[l], total, hkv, D, 0), "f16")
        v = stored(vs[l], "f16")
        ref, _, _ = orc.window_attention(q.reshape(-1), k.transpose(1, 0, 2).reshape(-1),
                                         v.transpose(1, 0, 2).reshape(-1), total, total, total, hq,
                                         hkv, D, 0, 0, window, 0.125)
        err = max_err(host(ctxs[l]).reshape(-1), ref)
        log(f"queued ring session layer {l}: max abs error {err:.3e}")
        assert err <= TOL_HALF
    s.close()
    c.close()


def test_queued_ring_sessions_sharing_a_context_see_commits_skipped_for_the_other(
        torch_mod, ops, sess_mod, orc):
    """Two queued ring sessions on one context.  B's fourth chunk holds a NaN, and A's
    chunks are queued after it, so A's gated ring commits are all skipped.  B's
    synchronize reports NonFinite and clears the context's status word; A's then
    finds its committed length short of its evaluated length, reports a device
    error and rolls back to position 0, and re-evaluating A matches the oracle."""
    torch = torch_mod
    rng = np.random.default_rng(17)
    L, hq, hkv, D, total, W = 2, 4, 2, 64, 80, 32
    c = ops.Context(0, synchronous=False)
    opts = sess_mod.Options(capacity=total, prefill_chunk_size=16, vocab_size=10, layers=L,
                            query_heads=hq, kv_heads=hkv, head_dim=D, storage="bf16",
                            score_scale=0.125, layer_windows=[W, 0])
    sess, ios, inputs, ctxs = [], [], [], []
    for name in "AB":
        qs, ks, vs, wq, wk = _session_inputs(rng, L, total, hq, hkv, D)
        out = [torch.zeros((total, hq * D), dtype=torch.float32, device="cuda") for _ in range(L)]
        kk = [k.copy() for k in ks]
        if name == "B":
            kk[0][55, 1, 3] = np.nan   # chunk [48, 64) of B
        ios.append([sess_mod.LayerIo(_t(torch, qs[l]), _t(torch, kk[l]), _t(torch, vs[l]), out[l],
                                     _t(torch, wq[l]), _t(torch, wk[l])) for l in range(L)])
        inputs.append((qs, ks, vs, wq, wk))
        ctxs.append(out)
        sess.append(sess_mod.Session(c, opts))
    a, b = sess
    b.set_tokens([1] * total)
    assert b.evaluate(ios[1]) == total
    a.set_tokens([2] * total)
    assert a.evaluate(ios[0]) == total
    with pytest.raises(ops.TkhError) as e:
        b.synchronize()
    assert e.value.name == "NonFinite"
    with pytest.raises(ops.TkhError) as e:
        a.synchronize()
    log(f"session A after B's failure: {e.value}")
    assert e.value.name == "Device"
    assert (a.evaluated_len(), a.pending_len()) == (0, total)
    assert a.evaluate(ios[0]) == total
    a.synchronize()
    qs, ks, vs, wq, wk = inputs[0]
    for l, window in enumerate([W, None]):
        q = stored(_oracle_produce(orc, qs[l], wq[l], total, hq, D, 0), "bf16")
        k = stored(_oracle_produce(orc, ks[l], wk[l], total, hkv, D, 0), "bf16")
        v = stored(vs[l], "bf16")
        ref, _, _ = orc.window_attention(q.reshape(-1), k.transpose(1, 0, 2).reshape(-1),
                                         v.transpose(1, 0, 2).reshape(-1), total, total, total, hq,
                                         hkv, D, 0, 0, window, 0.125)
        err = max_err(host(ctxs[0][l]).reshape(-1), ref)
        log(f"shared-context ring session A layer {l}: max abs error {err:.3e}")
        assert err <= TOL_HALF
    a.close()
    b.close()
    c.close()


def test_queued_linear_session_failure_returns_to_checked_prefix(torch_mod, ops, sess_mod):
    torch = torch_mod
    rng = np.random.default_rng(8)
    hq, hkv, D, total = 4, 2, 64, 64
    qs, ks, vs, wq, wk = _session_inputs(rng, 1, total, hq, hkv, D)
    c = ops.Context(0, synchronous=False)
    s = sess_mod.Session(c, sess_mod.Options(capacity=total, prefill_chunk_size=16, vocab_size=10,
                                             layers=1, query_heads=hq, kv_heads=hkv, head_dim=D,
                                             storage="bf16"))
    out = torch.zeros((total, hq * D), dtype=torch.float32, device="cuda")
    vbad = vs[0].copy()
    vbad[40, 1, 0] = np.inf
    io = [sess_mod.LayerIo(_t(torch, qs[0]), _t(torch, ks[0]), _t(torch, vbad), out, None, None)]
    s.set_tokens([1] * 32)
    s.evaluate(io)
    s.synchronize()                          # 32 tokens checked
    s.append([1] * 32)
    s.evaluate(io)
    with pytest.raises(ops.TkhError):
        s.synchronize()
    assert (s.evaluated_len(), s.pending_len()) == (32, 32)
    assert not s.distribution_valid()
    s.close()
    c.close()


def test_queued_abort_after_a_failing_layer_keeps_the_checked_chunks(torch_mod, ops, sess_mod):
    """A queued context, layer by layer: chunk A committed and synchronized, chunk
    B begun, a non-finite value in its layer 0, B aborted.  The next synchronize
    reports B's non-finite value and the session keeps A (its checked prefix),
    as tkh_session_chunk_abort documents; a retry of B with clean inputs then
    commits."""
    torch = torch_mod
    rng = np.random.default_rng(9)
    hq, hkv, D, total = 4, 2, 64, 64
    qs, ks, vs, wq, wk = _session_inputs(rng, 1, total, hq, hkv, D)
    c = ops.Context(0, synchronous=False)
    s = sess_mod.Session(c, sess_mod.Options(capacity=total, prefill_chunk_size=16, vocab_size=10,
                                             layers=2, query_heads=hq, kv_heads=hkv, head_dim=D,
                                             storage="bf16"))
    out = torch.zeros((16, hq * D), dtype=torch.float32, device="cuda")
    good = [sess_mod.LayerIo(_t(torch, qs[0][p:p + 16]), _t(torch, ks[0][p:p + 16]),
                             _t(torch, vs[0][p:p + 16]), out, None, None) for p in (0, 16)]
    vbad = vs[0][16:32].copy()
    vbad[3, 1, 0] = np.nan
    bad = sess_mod.LayerIo(_t(torch, qs[0][16:32]), _t(torch, ks[0][16:32]), _t(torch, vbad), out,
                           None, None)
    s.set_tokens([1] * 32)
    assert s.chunk_begin(16) == (0, 16)
    s.chunk_layer(0, good[0])
    s.chunk_layer(1, good[0])
    assert s.chunk_commit() == 16
    s.synchronize()                          # chunk A checked
    assert s.chunk_begin(16) == (16, 16)
    s.chunk_layer(0, bad)                    # queued: nothing is checked yet
    s.chunk_abort()
    with pytest.raises(ops.TkhError) as e:
        s.synchronize()
    assert e.value.name == "NonFinite"
    assert (s.evaluated_len(), s.pending_len()) == (16, 16)
    assert s.chunk_begin(16) == (16, 16)
    s.chunk_layer(0, good[1])
    s.chunk_layer(1, good[1])
    assert s.chunk_commit() == 16
    s.synchronize()
    assert (s.evaluated_len(), s.pending_len()) == (32, 0)
    s.close()
    c.close()


@pytest.mark.parametrize("storage,hq,hkv,D", [("bf16", 16, 8, 128), ("f32", 8, 2, 64), ("f16", 8, 1, 64),
                                              ("bf16", 32, 8, 128), ("f32", 14, 2, 64),
                                              ("f32", 16, 4, 128)])
def test_decode_steps_with_fused_producer_match_separate_producer(torch_mod, ops, sess_mod, orc,
                                                                  storage, hq, hkv, D):
    """Decode steps run the producer inside the decode kernel; the contexts match the
    separate producer launch to rounding and the oracle within tolerance (1e-5 for
    FP32 storage).  Later steps read the rows earlier steps appended, so a wrong
    append shows up as an oracle mismatch."""
    import os

    torch = torch_mod
    rng = np.random.default_rng(9)
    prompt, steps = 70, 5
    total = prompt + steps
    qs, ks, vs, wq, wk = _session_inputs(rng, 1, total, hq, hkv, D)
    outs = []
    for fused in ("1", "0"):
        saved = os.environ.get("TKH_FUSED_DECODE")
        os.environ["TKH_FUSED_DECODE"] = fused
        try:
            c = ops.Context(0)
            s = sess_mod.Session(c, sess_mod.Options(capacity=total, prefill_chunk_size=32,
                                                     position_offset=3, layers=1, query_heads=hq,
                                                     kv_heads=hkv, head_dim=D, storage=storage))
        finally:
            if saved is None:
                os.environ.pop("TKH_FUSED_DECODE", None)
            else:
                os.environ["TKH_FUSED_DECODE"] = saved
        out = torch.zeros((total, hq * D), dtype=torch.float32, device="cuda")
        io = [sess_mod.LayerIo(_t(torch, qs[0]), _t(torch, ks[0]), _t(torch, vs[0]), out,
                               _t(torch, wq[0]), _t(torch, wk[0]))]
        s.set_tokens([1] * prompt)
        s.evaluate(io)
        s.append([1] * steps)
        assert s.evaluate(io, chunk_limit=1) == steps
        outs.append(host(out))
        s.close()
        c.close()
    q = stored(_oracle_produce(orc, qs[0], wq[0], total, hq, D, 3), storage)
    k = stored(_oracle_produce(orc, ks[0], wk[0], total, hkv, D, 3), storage)
    v = stored(vs[0], storage)
    ref, _, _ = orc.attention(q.reshape(-1), k.reshape(-1), v.reshape(-1), total, hq, hkv, D)
    errs = [max_err(o.reshape(-1), ref) for o in outs]
    log(f"{storage} {hq}/{hkv}/{D} decode steps, fused / separate producer: max abs error "
        f"{errs[0]:.3e} / {errs[1]:.3e}")
    assert max(errs) <= (1e-5 if storage == "f32" else TOL_HALF)
    # The new key is summed in a different order (after the stream, in one wave),
    # so the two agree to rounding, not bitwise.
    assert max_err(outs[0], outs[1]) <= 1e-5
