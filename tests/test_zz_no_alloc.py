"""The allocation-free entry point (tkh_attention_cached_static) against the
context entry point it varies (tkh_attention_cached) and the CPU oracle.

Two calls in a row per path, the second smaller, so the second runs on the
fixed scratch the first left behind: a decode step over 70,000 keys of eight
KV heads (enough work for the decode kernel's in-kernel merge, whose
completion flags live in the scratch) then one over 8192 keys (split
partials merged by a second launch), a decode step over 8192 keys then one
over 300, and a 128-token chunk over 2176 keys (split prefill partials) then
a 40-token one.  The decode steps' static and context outputs are the same
kernels' with the same splits and must be bit-equal; a chunk's static splits
may be fewer (its partials must fit the scratch), so chunks agree to 2e-3.
A graph captured around the in-kernel-merge call is replayed with new Q
between replays (eager static calls in between move the epoch on) and
checked against eager calls each time.  Also: the caller's status word
receives a non-finite input's bits, and a call whose partials cannot fit the
scratch is rejected.
"""

import numpy as np
import pytest

from gpu_util import TOL_HALF, dev, host, log, max_err, stored

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


def _inputs(rng, tokens, hq, hkv, D, capacity, dt):
    k = stored(rng.standard_normal((hkv, capacity, D)), dt)
    v = stored(rng.standard_normal((hkv, capacity, D)), dt)
    q = stored(rng.standard_normal((tokens, hq, D)), dt).reshape(-1)
    return q, k, v


@pytest.mark.parametrize("calls", [
    [(1, 69999, 70000), (1, 8191, 8192)],    # decode: in-kernel flag merge, then a merge launch
    [(1, 8191, 8192), (1, 299, 300)],        # decode: split-K merge launch, then a smaller step
    [(128, 2048, 2176), (40, 100, 140)],     # chunks: split prefill partials, then a smaller chunk
])
def test_static_entry_point_matches_context_entry_point(torch_mod, ops, orc, calls):
    torch = torch_mod
    rng = np.random.default_rng(71)
    hq, hkv, D, dt = 16, 8, 128, "bf16"
    ctx = ops.Context(0)
    for i, (tokens, offset, capacity) in enumerate(calls):
        q, k, v = _inputs(rng, tokens, hq, hkv, D, capacity, dt)
        shape = ops.CachedAttentionShape(tokens, hq, hkv, D, capacity, offset)
        qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
        out_ctx = torch.full((tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
        out_static = torch.full_like(out_ctx, np.nan)
        log(f"static entry point call {i}: {tokens} tokens at offset {offset}")
        ops.attention_cached(ctx, qd, kd, vd, out_ctx, None, None, shape)
        ops.attention_cached_static(0, qd, kd, vd, out_static, shape)
        torch.cuda.synchronize()
        ref, _, _ = orc.attention_cached(q, k, v, tokens, hq, hkv, D, capacity, offset)
        a, b = host(out_static), host(out_ctx)
        diff, err = max_err(a, b), max_err(a, ref)
        log(f"  static vs context {diff:.3e} (identical: {np.array_equal(a, b)}), "
            f"static vs oracle {err:.3e}")
        # A decode step runs the same kernels with the same splits on both paths:
        # bit-equal.  A chunk's split partials must fit the scratch, so the static
        # path may take fewer, longer splits (another summation order).
        assert (np.array_equal(a, b) if tokens == 1 else diff <= TOL_HALF) and err <= TOL_HALF
    ctx.close()


def test_static_entry_point_in_a_replayed_graph(torch_mod, ops, orc):
    """A captured static call on the in-kernel flag merge (one token, eight KV
    heads, 70,000 keys), replayed three times with new Q written between the
    replays and an eager static call (a later epoch) before each: every
    replay equals the eager call on the same Q bit for bit, and the oracle."""
    torch = torch_mod
    rng = np.random.default_rng(73)
    hq, hkv, D, dt, cap = 16, 8, 128, "bf16", 70000
    shape = ops.CachedAttentionShape(1, hq, hkv, D, cap, cap - 1)
    _, k, v = _inputs(rng, 1, hq, hkv, D, cap, dt)
    kd, vd = dev(k, dt), dev(v, dt)
    qs = [stored(rng.standard_normal((1, hq, D)), dt).reshape(-1) for _ in range(4)]
    qd = dev(qs[0], dt)
    stream = torch.cuda.Stream()
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out_g = torch.zeros(hq * D, dtype=torch.float32, device="cuda")
    out_e = torch.zeros_like(out_g)
    other = torch.zeros_like(out_g)
    with torch.cuda.stream(stream):
        ops.attention_cached_static(0, qd, kd, vd, out_e, shape, stream=stream, status=status)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ops.attention_cached_static(0, qd, kd, vd, out_g, shape, stream=stream, status=status)
    torch.cuda.synchronize()
    for rep in range(1, 4):
        # An eager call on other Q first: it stores a later epoch and clears its flags.
        qd.copy_(dev(qs[rep - 1], dt))
        with torch.cuda.stream(stream):
            ops.attention_cached_static(0, qd, kd, vd, other, shape, stream=stream, status=status)
        torch.cuda.synchronize()
        qd.copy_(dev(qs[rep], dt))
        out_g.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ops.attention_cached_static(0, qd, kd, vd, out_e, shape, stream=stream, status=status)
        torch.cuda.synchronize()
        ref, _, _ = orc.attention_cached(qs[rep], k, v, 1, hq, hkv, D, cap, cap - 1)
        a, b = host(out_g), host(out_e)
        err = max_err(a, ref)
        log(f"graph replay {rep}: identical to the eager call {np.array_equal(a, b)}, "
            f"vs oracle {err:.3e}, status {int(status.item()):#x}")
        assert np.array_equal(a, b) and err <= TOL_HALF
        assert int(status.item()) == 0


def test_static_entry_point_status_word_and_scratch_limit(torch_mod, ops):
    torch = torch_mod
    rng = np.random.default_rng(72)
    hq, hkv, D, cap = 8, 2, 128, 1024
    q, k, v = _inputs(rng, 1, hq, hkv, D, cap, "f16")
    k[1, 500, 3] = np.nan
    shape = ops.CachedAttentionShape(1, hq, hkv, D, cap, cap - 1)
    out = torch.zeros(hq * D, dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.attention_cached_static(0, dev(q, "f16"), dev(k, "f16"), dev(v, "f16"), out, shape,
                                status=status)
    torch.cuda.synchronize()
    word = int(status.item())
    log(f"status word after a NaN key: {word:#x}")
    assert word != 0 and word & 8 == 0
    # Without a status word the same call waits and reports like a synchronous context.
    with pytest.raises(ops.TkhError) as e:
        ops.attention_cached_static(0, dev(q, "f16"), dev(k, "f16"), dev(v, "f16"), out, shape)
    assert e.value.name == "NonFinite"
    # A clean call after the failure: the caller cleared its word, it stays clear.
    k[1, 500, 3] = 0.0
    status.zero_()
    ops.attention_cached_static(0, dev(q, "f16"), dev(k, "f16"), dev(v, "f16"), out, shape,
                                status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    # FP32 chunks run one partial row per (token, head): 1024 x 16 x 130 x 4 bytes
    # exceed the scratch's half for them, so the call is refused.
    tokens, hq, hkv, D = 1024, 16, 8, 128
    shape = ops.CachedAttentionShape(tokens, hq, hkv, D, tokens, 0)
    qd = torch.zeros(tokens * hq * D, dtype=torch.float32, device="cuda")
    kd = torch.zeros(hkv * tokens * D, dtype=torch.float32, device="cuda")
    outd = torch.zeros_like(qd)
    with pytest.raises(ops.TkhError) as e:
        ops.attention_cached_static(0, qd, kd, kd, outd, shape)
    log(f"oversized call: {e.value}")
    assert e.value.name == "Unsupported" and e.value.tensor == "scratch"
