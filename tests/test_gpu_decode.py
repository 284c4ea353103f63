"""GPU parity of the streaming decode kernel (few query rows per KV head).

Long contexts split the keys over many workgroups, so these cases exercise the
split-K merge done by the last split of each KV head (completion flags with a
new epoch per launch), per-row causal limits when a short chunk has several
tokens, windows and the score softcap at head_dim 256, ring spans, both
planner regimes for many sessions, and the merge's bounded wait (forced from
the host).  The checker is the CPU oracle on the same stored (rounded) values.
"""

import os

import numpy as np
import pytest

from gpu_util import TOL_F32, TOL_HALF, assert_tokens_agree, dev, host, log, max_err, stored

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
def ctx(torch_mod, ops):
    return ops.Context(0)


def _cached_case(torch, ctx, ops, orc, *, hq, hkv, D, dt, capacity, offset, tokens, seed,
                 key_scale=None, k_mult=1.0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((hkv, capacity, D)).astype(np.float32) * k_mult
    if key_scale is not None:
        mask = rng.random((hkv, capacity)) < key_scale
        k[mask] *= 8.0
    v = rng.standard_normal((hkv, capacity, D)).astype(np.float32)
    q = rng.standard_normal((tokens, hq, D)).astype(np.float32)
    ks, vs, qs = stored(k, dt), stored(v, dt), stored(q, dt).reshape(-1)
    out = torch.full((tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(qs, dt), dev(ks, dt), dev(vs, dt), out, None, None,
                         ops.CachedAttentionShape(tokens, hq, hkv, D, capacity, offset))
    ref, _, _ = orc.attention_cached(qs, ks, vs, tokens, hq, hkv, D, capacity, offset)
    return host(out), ref


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("context", [1, 17, 300, 2049, 8192])
def test_single_token_decode_qwen3(torch_mod, ctx, ops, orc, dt, context):
    log(f"decode 16/8/128 {dt} context {context}")
    got, ref = _cached_case(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt=dt,
                            capacity=context + 5, offset=context - 1, tokens=1, seed=context)
    err = max_err(got, ref)
    log(f"  max abs error {err:.3e}")
    assert err <= TOL_HALF


def test_decode_peaky_keys_and_tokens(torch_mod, ctx, ops, orc):
    """5% of key rows x8 (configs[4]'s stress) at 6000 keys; greedy tokens identical."""
    rng = np.random.default_rng(77)
    w = rng.standard_normal((2048, 32 * 128)).astype(np.float32)
    got, ref = _cached_case(torch_mod, ctx, ops, orc, hq=32, hkv=8, D=128, dt="bf16",
                            capacity=6000, offset=5999, tokens=1, seed=5, key_scale=0.05)
    err = max_err(got, ref)
    log(f"llama 32/8/128 peaky decode: max abs error {err:.3e}")
    assert err <= TOL_HALF
    assert_tokens_agree(got.reshape(1, -1), ref.reshape(1, -1), w)


@pytest.mark.parametrize("tokens", [2, 3, 4])
def test_short_chunk_rows_have_their_own_causal_limit(torch_mod, ctx, ops, orc, tokens):
    log(f"short chunk of {tokens} tokens at offset 3000")
    got, ref = _cached_case(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                            capacity=3100, offset=3000, tokens=tokens, seed=tokens)
    assert max_err(got, ref) <= TOL_HALF


def test_gqa7_d64_and_fp32(torch_mod, ctx, ops, orc):
    """Qwen2.5 geometry (14/2/64, 7 rows per KV head) in bf16, and the FP32 path at 1e-5."""
    got, ref = _cached_case(torch_mod, ctx, ops, orc, hq=14, hkv=2, D=64, dt="bf16",
                            capacity=4000, offset=3999, tokens=1, seed=11)
    assert max_err(got, ref) <= TOL_HALF
    got, ref = _cached_case(torch_mod, ctx, ops, orc, hq=14, hkv=2, D=64, dt="f32",
                            capacity=4000, offset=3999, tokens=1, seed=12)
    err = max_err(got, ref)
    log(f"fp32 14/2/64 decode at 4000: max abs error {err:.3e}")
    assert err <= TOL_F32


def test_repeated_calls_are_identical_across_epochs(torch_mod, ctx, ops, orc):
    """Each launch waits for its own epoch: the same call twice is bit-identical, and a
    different split layout in between (other flags, other slots) does not disturb it."""
    a1, ref = _cached_case(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                           capacity=8192, offset=8191, tokens=1, seed=21)
    _cached_case(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt="bf16", capacity=1000,
                 offset=999, tokens=1, seed=22)
    a2, _ = _cached_case(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                         capacity=8192, offset=8191, tokens=1, seed=21)
    assert np.array_equal(a1, a2)
    assert max_err(a1, ref) <= TOL_HALF


@pytest.mark.parametrize("softcap", [0.0, 50.0])
def test_gemma_window_decode_d256(torch_mod, ctx, ops, orc, softcap):
    """Gemma3 local layer decode: 8/4/256, W=1024, scale 1/16, at position 4100."""
    torch = torch_mod
    rng = np.random.default_rng(31)
    hq, hkv, D, W = 8, 4, 256, 1024
    keys = 4101
    for dt in ("bf16", "f16"):
        k = stored(rng.standard_normal((hkv, keys, D)) * 3, dt)
        v = stored(rng.standard_normal((hkv, keys, D)), dt)
        q = stored(rng.standard_normal((1, hq, D)) * 3, dt).reshape(-1)
        out = torch.zeros(hq * D, dtype=torch.float32, device="cuda")
        shape = ops.WindowAttentionShape(1, keys, keys, hq, hkv, D, keys - 1, 0, W, 1.0 / 16.0,
                                         softcap)
        ops.window_attention(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None, shape)
        ref, _, _ = orc.window_attention(q, k.reshape(-1), v.reshape(-1), 1, keys, keys, hq, hkv, D,
                                         keys - 1, 0, W, 1.0 / 16.0, softcap=softcap)
        err = max_err(host(out), ref)
        log(f"gemma window decode {dt} softcap {softcap}: max abs error {err:.3e}")
        assert err <= TOL_HALF


@pytest.mark.parametrize("hq,hkv,D,W,offset", [
    (8, 4, 128, 1024, 5000),   # slot 5000 % 1024 = 904: the old spans wrap around the ring
    # One KV head, D=64: old spans of 1000 and 1047 rows plus the new one.  Rounded
    # up per segment at 32 keys per split they would need 32 + 33 + 1 = 66 splits,
    # two more than the merge reads; the planner must widen the splits instead.
    (1, 1, 64, 2048, 3095),
])
def test_ring_span_decode_wraps(torch_mod, ctx, ops, orc, hq, hkv, D, W, offset):
    """Decode over a ring whose view is two old spans plus the new row."""
    torch = torch_mod
    rng = np.random.default_rng(41)
    ring_k = stored(rng.standard_normal((hkv, W, D)), "bf16")
    ring_v = stored(rng.standard_normal((hkv, W, D)), "bf16")
    nk = stored(rng.standard_normal((hkv, 1, D)), "bf16")
    nv = stored(rng.standard_normal((hkv, 1, D)), "bf16")
    q = stored(rng.standard_normal((1, hq, D)), "bf16").reshape(-1)
    kd, vd = dev(ring_k, "bf16").reshape(-1), dev(ring_v, "bf16").reshape(-1)
    segs_dev, segs_ref = [], []
    logical = 0
    for position, slot, rows in orc.old_spans(W, offset, W):
        if rows == 0:
            segs_dev.append(ops.AttentionKvSegment(None, None, 0, 0, offset))
            segs_ref.append(orc.Segment(np.zeros(0), np.zeros(0), 0, 0, offset))
            continue
        b = slot * D
        e = (hkv - 1) * W * D + b + rows * D
        segs_dev.append(ops.AttentionKvSegment(kd[b:e], vd[b:e], rows, W * D, position))
        segs_ref.append(orc.Segment(ring_k.reshape(-1)[b:e], ring_v.reshape(-1)[b:e], rows, W * D,
                                    position))
        logical += rows
    assert sum(1 for sg in segs_ref if sg.keys) == 2, "the view must wrap the ring"
    nkd, nvd = dev(nk, "bf16").reshape(-1), dev(nv, "bf16").reshape(-1)
    segs_dev.append(ops.AttentionKvSegment(nkd, nvd, 1, D, offset))
    segs_ref.append(orc.Segment(nk.reshape(-1), nv.reshape(-1), 1, D, offset))
    key_start = offset - logical
    keys = logical + 1
    shape = ops.SpanAttentionShape(1, keys, hq, hkv, D, offset, key_start, W, 1.0 / np.sqrt(D), 0.0)
    out = torch.zeros(hq * D, dtype=torch.float32, device="cuda")
    ops.span_attention(ctx, dev(q, "bf16"), segs_dev, out, None, None, shape)
    ref, _, _ = orc.span_attention(q, segs_ref, 1, keys, hq, hkv, D, offset, key_start, W,
                                   np.float32(1.0 / np.sqrt(D)))
    err = max_err(host(out), ref)
    log(f"ring decode {hq}/{hkv}/{D} W={W}: keys {keys}, max abs error {err:.3e}")
    assert err <= TOL_HALF


@pytest.mark.parametrize("B,merge_batch", [(24, 0), (80, 0), (24, 1), (64, 1)])
def test_decode_batch_many_sessions_lengths_to_8192(torch_mod, ctx, ops, orc, B, merge_batch):
    """configs[2] in miniature: f16 sessions, lengths 1..8192, one query token each.
    Up to 64 sessions travel in the decode kernel's arguments; 80 upload their
    descriptors.  merge_batch: the compact batch's splits combined by a second
    launch (TKH_DECODE_MERGE_BATCH)."""
    torch = torch_mod
    if merge_batch:
        ctx = _context_with_env(ops, {"TKH_DECODE_MERGE_BATCH": 1})
    rng = np.random.default_rng(51)
    hq, hkv, D = 16, 8, 128
    lengths = np.concatenate([[1, 2, 8192, 513], rng.integers(1, 8193, B - 4)])
    scales = rng.uniform(0.5, 2.0, B)
    offsets, pool_k, pool_v, total = [], [], [], 0
    for b in range(B):
        n = hkv * int(lengths[b]) * D
        offsets.append(total)
        pool_k.append(stored(rng.standard_normal(n) * scales[b], "f16"))
        pool_v.append(stored(rng.standard_normal(n) * scales[b], "f16"))
        total += n
    kpool, vpool = np.concatenate(pool_k), np.concatenate(pool_v)
    q = stored(rng.standard_normal((B, hq, D)) * scales[:, None, None], "f16")
    out = torch.zeros(B * hq * D, dtype=torch.float32, device="cuda")
    ops.decode_batch(ctx, dev(q, "f16"), dev(kpool, "f16"), dev(vpool, "f16"), offsets,
                     [int(l) * D for l in lengths], [int(l) for l in lengths], out,
                     query_heads=hq, kv_heads=hkv, head_dim=D, scale=1.0 / np.sqrt(D))
    got = host(out).reshape(B, -1)
    worst = 0.0
    for b in range(B):
        L = int(lengths[b])
        kb = kpool[offsets[b]:offsets[b] + hkv * L * D]
        vb = vpool[offsets[b]:offsets[b] + hkv * L * D]
        ref, _, _ = orc.attention_cached(q[b].reshape(-1), kb, vb, 1, hq, hkv, D, L, L - 1)
        worst = max(worst, max_err(got[b], ref))
    log(f"decode batch of {B} (merge launch {merge_batch}): worst max abs error {worst:.3e}")
    assert worst <= TOL_HALF


def test_decode_batch_even_lengths_one_round(torch_mod, ctx, ops, orc):
    """8 bf16 sessions of 8192 keys: much work of even length, the planner's one-round
    regime (four-wave workgroups, two per CU)."""
    torch = torch_mod
    rng = np.random.default_rng(53)
    hq, hkv, D, B, L = 16, 8, 128, 8, 8192
    n = hkv * L * D
    kpool = stored(rng.standard_normal(B * n), "bf16")
    vpool = stored(rng.standard_normal(B * n), "bf16")
    q = stored(rng.standard_normal((B, hq, D)), "bf16")
    out = torch.zeros(B * hq * D, dtype=torch.float32, device="cuda")
    offsets = [b * n for b in range(B)]
    ops.decode_batch(ctx, dev(q, "bf16"), dev(kpool, "bf16"), dev(vpool, "bf16"), offsets,
                     [L * D] * B, [L] * B, out, query_heads=hq, kv_heads=hkv, head_dim=D,
                     scale=1.0 / np.sqrt(D))
    got = host(out).reshape(B, -1)
    worst = 0.0
    for b in range(B):
        ref, _, _ = orc.attention_cached(q[b].reshape(-1), kpool[b * n:(b + 1) * n],
                                         vpool[b * n:(b + 1) * n], 1, hq, hkv, D, L, L - 1)
        worst = max(worst, max_err(got[b], ref))
    log(f"decode batch of {B} x {L}: worst max abs error {worst:.3e}")
    assert worst <= TOL_HALF


def test_split_wait_is_bounded_and_reported(torch_mod, ops, orc):
    """Forced from the host: a context whose decode merges wait for a flag value no split
    stores, with a 20 us bound.  Every workgroup exits, the launch reports a device error
    naming the splits, and a normal context afterwards computes correctly."""
    saved = {k: os.environ.get(k) for k in ("TKH_TEST_SPLIT_WAIT_TICKS", "TKH_TEST_SPLIT_FLAG_SKEW")}
    os.environ["TKH_TEST_SPLIT_WAIT_TICKS"] = "2000"
    os.environ["TKH_TEST_SPLIT_FLAG_SKEW"] = "1"
    try:
        forced = ops.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    with pytest.raises(ops.TkhError) as e:
        _cached_case(torch_mod, forced, ops, orc, hq=16, hkv=8, D=128, dt="bf16", capacity=4100,
                     offset=4095, tokens=1, seed=31)
    assert e.value.name == "Device" and e.value.tensor == "decode splits"
    assert "timed out" in e.value.message
    forced.close()
    clean = ops.Context(0)
    got, ref = _cached_case(torch_mod, clean, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                            capacity=4100, offset=4095, tokens=1, seed=31)
    assert max_err(got, ref) <= TOL_HALF


def _context_with_env(ops, env):
    """A context created under extra TKH_* settings (read once at creation)."""
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return ops.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("groups,keys_per_lane", [(256, 4), (512, 2), (512, 4)])
def test_in_kernel_merge_of_many_splits(torch_mod, ops, orc, groups, keys_per_lane):
    """The last split's own merge (the second launch switched off) at 32 and 64
    splits per KV head: its output loads run over four split groups at a time, so
    these take two and four runs; against the oracle and bit-equal to the merge
    launch's result (the same weights and sums in the same order)."""
    torch = torch_mod
    env = {"TKH_DECODE_GROUPS": groups, "TKH_DECODE_KEYS_PER_LANE": keys_per_lane}
    inkernel = _context_with_env(ops, dict(env, TKH_DECODE_MERGE_LAUNCH=0))
    launch = _context_with_env(ops, dict(env, TKH_DECODE_MERGE_LAUNCH=1))
    got, ref = _cached_case(torch, inkernel, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                            capacity=8200, offset=8191, tokens=1, seed=groups + keys_per_lane)
    err = max_err(got, ref)
    log(f"in-kernel merge, {groups} groups, {keys_per_lane} keys per lane: max abs error {err:.3e}")
    assert err <= TOL_HALF
    again, _ = _cached_case(torch, launch, ops, orc, hq=16, hkv=8, D=128, dt="bf16",
                            capacity=8200, offset=8191, tokens=1, seed=groups + keys_per_lane)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_stream_load_form_does_not_change_results(torch_mod, ops, orc):
    """The K/V stream's load form (nontemporal for much work, plain for latency-bound
    launches) is forced both ways in both regimes: the outputs are bit-identical and
    match the oracle."""
    torch = torch_mod
    rng = np.random.default_rng(57)
    hq, hkv, D, B, L = 16, 8, 128, 16, 4096
    n = hkv * L * D
    kpool = stored(rng.standard_normal(B * n), "bf16")
    vpool = stored(rng.standard_normal(B * n), "bf16")
    q = stored(rng.standard_normal((B, hq, D)), "bf16")
    offsets = [b * n for b in range(B)]
    results = {}
    for nt in (0, 1):
        c = _context_with_env(ops, {"TKH_DECODE_STREAM_NT": nt})
        for batch in (1, B):  # one session: latency regime; sixteen: much work
            log(f"stream loads nt={nt}, {batch} session(s) x {L} keys")
            out = torch.zeros(batch * hq * D, dtype=torch.float32, device="cuda")
            ops.decode_batch(c, dev(q[:batch], "bf16"), dev(kpool[:batch * n], "bf16"),
                             dev(vpool[:batch * n], "bf16"), offsets[:batch], [L * D] * batch,
                             [L] * batch, out, query_heads=hq, kv_heads=hkv, head_dim=D,
                             scale=1.0 / np.sqrt(D))
            results[(nt, batch)] = host(out).reshape(batch, -1)
        c.close()
    for batch in (1, B):
        assert np.array_equal(results[(0, batch)], results[(1, batch)])
    worst = 0.0
    for b in (0, B - 1):
        ref, _, _ = orc.attention_cached(q[b].reshape(-1), kpool[b * n:(b + 1) * n],
                                         vpool[b * n:(b + 1) * n], 1, hq, hkv, D, L, L - 1)
        worst = max(worst, max_err(results[(1, B)][b], ref))
    log(f"  worst max abs error {worst:.3e}")
    assert worst <= TOL_HALF


@pytest.mark.parametrize("context", [300, 2049, 8192])
def test_stream_tail_reads_only_visible_rows(torch_mod, ctx, ops, orc, context):
    """A wave block past a split's last key reads the split's last row again (its
    loads are unconditional) and masks it.  Infinities in the cache rows past the
    query position are never read, so the result still matches the oracle; an
    infinity in V of the last visible row is reported as a non-finite input, as the
    reference's visible-prefix check reports it (src/cpu/attention.rs:247-251)."""
    torch = torch_mod
    rng = np.random.default_rng(71 + context)
    hq, hkv, D, capacity = 16, 8, 128, context + 40
    k = stored(rng.standard_normal((hkv, capacity, D)), "bf16")
    v = stored(rng.standard_normal((hkv, capacity, D)), "bf16")
    q = stored(rng.standard_normal((1, hq, D)), "bf16").reshape(-1)
    k[:, context:, :] = np.inf  # rows past the query position: never visible
    v[:, context:, :] = -np.inf
    shape = ops.CachedAttentionShape(1, hq, hkv, D, capacity, context - 1)
    log(f"stream tail: context {context}, infinities past it")
    out = torch.full((hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, None, None, shape)
    ref, _, _ = orc.attention_cached(q, np.where(np.isfinite(k), k, 0), np.where(np.isfinite(v), v, 0),
                                     1, hq, hkv, D, capacity, context - 1)
    assert max_err(host(out), ref) <= TOL_HALF
    v2 = v.copy()
    v2[3, context - 1, 5] = np.inf  # the last visible key of KV head 3
    log(f"stream tail: context {context}, infinity in the last visible V row")
    with pytest.raises(ops.TkhError) as e:
        ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v2, "bf16"), out, None, None,
                             shape)
    assert e.value.name == "NonFinite"
