"""The reference's Half staged-attention fixtures replayed on the device:
staged-gqa-half-v1 (11 cases of GQA 4/2 and 16/8 at D64, src/metal/
staged_gqa_fixture.rs:6-40) and gemma3-staged-attention-v1 (8 local/full cases
at D32 and D256, src/metal/staged_attention/tests.rs:9-60).

Per case, through this build's KV owner at f16 storage
(src/model/window_cache.rs:193-337):
  * the owner is brought to the case's committed length and its storage set to
    the fixture's physical old rows (unwritten slots hold the fixture's NaN pad
    word, which no kernel may read);
  * tkh_kv_prepare stages the chunk, tkh_kv_view gives the segments and span
    shape (the case's view start and query origin), and tkh_span_attention
    computes scores, probabilities and context (the diagnostic FP32 kernel)
    and, separately, the context alone (the decode or MFMA chunk kernel);
  * scores, probabilities and the context rounded to Half meet each array's
    gate |got - main| <= atol + rtol |main| (atol max(2 x envelope, 1e-4),
    rtol 1e-3: the fixture's policy), and masked probabilities are +0;
  * the same attention over the fixture's physical staged buffer, whose head
    stride is 32 rows whatever the chunk (as the Metal kernels address it),
    gives the same context;
  * tkh_kv_commit_batch leaves the ring (or linear buffer) equal, word for
    word, to the fixture's after-commit state (its copy runs).
The physical arrays are rebuilt from the fixtures' recipe and checked against
the manifests' SHA-256 (tests/goldens.py: staged_physical).
"""

import numpy as np
import pytest

from goldens import Golden, staged_physical
from gpu_util import log

pytestmark = pytest.mark.gpu

FIXTURES = ("staged_gqa_half_v1", "gemma3_staged_attention_v1")
CHUNK = 32


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch


@pytest.fixture(scope="module")
def ops():
    from toklet_amd import ops

    return ops


def _gate(got, want, gate, label):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert got.shape == want.shape, (label, got.shape, want.shape)
    assert np.isfinite(got).all(), f"{label}: non-finite values"
    excess = np.abs(got - want) - (gate["atol"] + gate["rtol"] * np.abs(want))
    worst = float(np.abs(got - want).max())
    assert (excess <= 0).all(), (f"{label}: {int((excess > 0).sum())} values outside the gate, "
                                 f"worst abs difference {worst:.3e}")
    return worst


@pytest.mark.parametrize("fixture", FIXTURES)
def test_staged_fixture_cases_on_the_device(torch_mod, ops, fixture):
    torch = torch_mod
    from toklet_amd import kv as kvmod

    g = Golden(fixture)
    ctx = ops.Context(0)
    f16 = lambda words: torch.from_numpy(np.ascontiguousarray(words).view(np.float16).copy()).cuda()
    for case in g.meta["cases"]:
        name, d, n = case["name"], case["dim"], case["tokens"]
        qh, kv, committed = case["query_heads"], case["kv_heads"], case["committed"]
        window, cap = case["window"], case["capacity"]
        retention = window or cap
        phys = staged_physical(g, fixture, case)
        cache = kvmod.WindowKvCache(ctx, kv, d, retention, cap, window, torch.float16)
        if committed:
            zeros = torch.zeros(kv * committed * d, dtype=torch.float16, device="cuda")
            cache.commit(cache.prepare(zeros, zeros, committed))
        assert cache.offset == committed
        k_now, v_now = cache.committed()
        k_now.copy_(f16(phys["old_k"][:kv * retention * d]).view(kv, retention, d))
        v_now.copy_(f16(phys["old_v"][:kv * retention * d]).view(kv, retention, d))
        staged = {kind: phys["new_" + kind][:kv * CHUNK * d].reshape(kv, CHUNK, d)[:, :n]
                  for kind in ("k", "v")}
        frame = cache.prepare(f16(staged["k"]), f16(staged["v"]), n)
        view = cache.view(frame)
        scale = float(np.float32(1.0) / np.float32(np.sqrt(d)))
        shape = view.attention_shape(qh, scale)
        assert shape.query_start == committed and shape.key_start == case["view"]["start"]
        keys = shape.keys
        assert keys == case["view"]["end"] - case["view"]["start"]
        q = f16(phys["q"][:n * qh * d])
        context = torch.full((n * qh * d,), float("nan"), dtype=torch.float32, device="cuda")
        scores = torch.full((qh * n * keys,), float("nan"), dtype=torch.float32, device="cuda")
        probs = torch.full_like(scores, float("nan"))
        ops.span_attention(ctx, q, view.segments(), context, scores, probs, shape)
        want = {stage: g[f"{name}.{stage}"] for stage in ("scores", "probabilities", "context")}
        gates = case["gates"]
        got_p = probs.cpu().numpy()
        e_s = _gate(scores.cpu().numpy(), want["scores"], gates["scores"], f"{name} scores")
        e_p = _gate(got_p, want["probabilities"], gates["probabilities"], f"{name} probabilities")
        masked = want["probabilities"].ravel().view(np.uint32) == 0
        assert (got_p.ravel().view(np.uint32)[masked] == 0).all(), f"{name}: masked probability not +0"
        want_ctx = want["context"].ravel().view(np.float16).astype(np.float64)
        half = lambda t: t.cpu().numpy().astype(np.float16).astype(np.float64)
        e_c = _gate(half(context), want_ctx, gates["context"], f"{name} context (diagnostic kernel)")
        # The context alone takes the decode or MFMA chunk kernel.
        fast = torch.full_like(context, float("nan"))
        ops.span_attention(ctx, q, view.segments(), fast, None, None, shape)
        e_f = _gate(half(fast), want_ctx, gates["context"], f"{name} context (fast kernel)")
        # The same staged rows at the fixture's physical head stride (32 rows).
        segs = view.segments()
        span = (kv - 1) * CHUNK * d + n * d
        segs[2] = ops.AttentionKvSegment(f16(phys["new_k"][:span]), f16(phys["new_v"][:span]), n,
                                         CHUNK * d, committed)
        strided = torch.full_like(context, float("nan"))
        ops.span_attention(ctx, q, segs, strided, None, None, shape)
        assert torch.equal(strided, fast), f"{name}: physical staged stride changed the context"
        kvmod.commit_batch([cache], [frame])
        k_now, v_now = cache.committed()
        for kind, now in (("k", k_now), ("v", v_now)):
            after = now.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).ravel()
            assert np.array_equal(after, phys["expected_after_" + kind][:kv * retention * d]), \
                f"{name}: {kind} after commit differs"
        log(f"{fixture} {name} ({qh}/{kv}/D{d}, committed {committed}, {n} tokens, "
            f"{'window ' + str(window) if window else 'full'}): scores {e_s:.2e}, probabilities "
            f"{e_p:.2e}, context {e_c:.2e} / fast {e_f:.2e}, after-commit state equal")
        cache.close()
    ctx.close()
