"""Pin the CPU oracle against the reference's frozen vectors and closed forms.

Each oracle function is checked by at least one of: a reference fixture, a
known-answer case from the reference's tests, a closed form, or brute force.
"""

import math

import numpy as np
import pytest

from goldens import (TINY_CASES, Golden, close, head_major_to_token_major,
                     reference_attention_inputs)


@pytest.fixture(scope="module")
def tiny():
    return Golden("tiny_v1")


def _tiny_layer(tiny, case, layer):
    p = f"cases.{case}.layers.{layer}"
    return {k: tiny.arrays[f"{p}.{k}"] for k in (
        "q_projection", "k_projection", "q_rotary", "k_rotary", "v_projection",
        "attention_scores", "attention_probabilities", "attention_context")}


# ---- tiny-v1: rotary + full-prefix attention (tests/cpu_attention.rs:16-79) ----

def test_rotary_and_attention_match_tiny_fixture(orc, tiny):
    for case in TINY_CASES:
        tokens = len(tiny.arrays[f"cases.{case}.tokens"])
        offset = tiny.meta["cases"][case]["position_offset"]
        for layer in range(2):
            a = _tiny_layer(tiny, case, layer)
            q = orc.rotary(a["q_projection"], tokens, 4, 8, offset, 1e6)
            k = orc.rotary(a["k_projection"], tokens, 2, 8, offset, 1e6)
            close(q, a["q_rotary"])
            close(k, a["k_rotary"])
            ctx, sc, pr = orc.attention(q, k, a["v_projection"], tokens, 4, 2, 8)
            close(sc, a["attention_scores"])
            close(pr, a["attention_probabilities"])
            close(ctx, a["attention_context"])


def test_rotary_known_answer_and_chunk_offsets(orc, tiny):
    """src: tests/cpu_attention.rs:81-128."""
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    assert np.array_equal(orc.rotary(x, 1, 1, 4, 0, 1.0), x)
    out = orc.rotary(x, 1, 1, 4, 1, 1.0)
    s, c = np.float32(math.sin(1.0)), np.float32(math.cos(1.0))
    close(out, [c - 3 * s, 2 * c - 4 * s, s + 3 * c, 2 * s + 4 * c])
    inp = tiny.arrays["cases.capacity.layers.0.q_projection"].reshape(-1)
    whole = orc.rotary(inp, 32, 4, 8, 5, 1e6)
    for t in range(32):
        one = orc.rotary(inp[t * 32:(t + 1) * 32], 1, 4, 8, 5 + t, 1e6)
        assert np.array_equal(one, whole[t * 32:(t + 1) * 32])
        for h in range(4):
            a = inp[t * 32 + h * 8:t * 32 + h * 8 + 8].astype(np.float64)
            b = whole[t * 32 + h * 8:t * 32 + h * 8 + 8].astype(np.float64)
            assert abs((a ** 2).sum() - (b ** 2).sum()) <= 1e-6 * max((a ** 2).sum(), 1.0)


# ---- tiny-v1 over a head-major cache with NaN stale tails (tests/cached_attention.rs:5-56) ----

def test_cached_attention_with_stale_tails_at_all_offsets(orc, tiny):
    for case in TINY_CASES:
        for layer in range(2):
            a = _tiny_layer(tiny, case, layer)
            q = a["q_rotary"].reshape(-1)
            tokens = q.size // 32
            cap = tokens + 3
            kc = np.full(2 * cap * 8, np.nan, np.float32)
            vc = kc.copy()
            k = a["k_rotary"].reshape(tokens, 2, 8)
            v = a["v_projection"].reshape(tokens, 2, 8)
            for h in range(2):
                kc[h * cap * 8:(h * cap + tokens) * 8] = k[:, h].reshape(-1)
                vc[h * cap * 8:(h * cap + tokens) * 8] = v[:, h].reshape(-1)
            expected = a["attention_context"].reshape(-1)
            for offset in range(tokens):
                n = tokens - offset
                ctx, _, _ = orc.attention_cached(q[offset * 32:], kc, vc, n, 4, 2, 8, cap, offset)
                close(ctx, expected[offset * 32:])


def test_cached_equals_full_prefix_bitwise(orc, tiny):
    """The cached path keeps the full-prefix FP32 dot/context order (src/cpu/attention.rs:194-195)."""
    a = _tiny_layer(tiny, "capacity", 1)
    tokens = 32
    full, _, _ = orc.attention(a["q_rotary"], a["k_rotary"], a["v_projection"], tokens, 4, 2, 8)
    cap = 40
    kc = np.zeros(2 * cap * 8, np.float32)
    vc = kc.copy()
    k = a["k_rotary"].reshape(tokens, 2, 8)
    v = a["v_projection"].reshape(tokens, 2, 8)
    for h in range(2):
        kc[h * cap * 8:(h * cap + tokens) * 8] = k[:, h].reshape(-1)
        vc[h * cap * 8:(h * cap + tokens) * 8] = v[:, h].reshape(-1)
    q = a["q_rotary"].reshape(-1)
    out = np.zeros_like(full)
    start = 0
    for chunk in (7, 1, 13, 11):
        ctx, _, _ = orc.attention_cached(q[start * 32:(start + chunk) * 32], kc, vc, chunk, 4, 2, 8,
                                         cap, start)
        out[start * 32:(start + chunk) * 32] = ctx
        start += chunk
    assert np.array_equal(out.view(np.uint32), full.view(np.uint32))


# ---- known answers from tests/cpu_attention.rs:130-313 ----

def test_grouped_heads_read_shared_value_head(orc):
    ctx, sc, pr = orc.attention(np.zeros(8), np.zeros(4), [1.0, 2.0, 3.0, 4.0], 1, 4, 2, 2)
    assert ctx.tolist() == [1, 2, 1, 2, 3, 4, 3, 4]
    assert sc.tolist() == [0.0] * 4 and pr.tolist() == [1.0] * 4


def test_future_changes_preserve_earlier_context_and_zero_masked(orc, tiny):
    q = tiny.arrays["cases.prompt.layers.0.q_rotary"].reshape(-1).copy()
    k = tiny.arrays["cases.prompt.layers.0.k_rotary"].reshape(-1).copy()
    v = tiny.arrays["cases.prompt.layers.0.v_projection"].reshape(-1).copy()
    before, _, _ = orc.attention(q, k, v, 4, 4, 2, 8)
    q[96:] = 7.0
    k[48:] = -5.0
    v[48:] = 100.0
    after, _, pr = orc.attention(q, k, v, 4, 4, 2, 8)
    assert np.array_equal(before[:96], after[:96])
    assert not np.array_equal(before[96:], after[96:])
    pr = pr.reshape(4, 4, 4)
    for h in range(4):
        for t in range(4):
            assert np.all(pr[h, t, t + 1:].view(np.uint32) == 0)


def test_invalid_inputs_fail_before_mutation(orc):
    out = np.full(4, 123.0, np.float32)
    for theta in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(orc.OracleError) as e:
            orc.rotary(np.ones(4), 1, 1, 4, 0, theta)
        assert e.value.code == orc.INVALID_PARAMETER
    with pytest.raises(orc.OracleError) as e:
        orc.rotary(np.ones(3), 1, 1, 3, 0, 1e6)
    assert e.value.code == orc.INVALID_PARAMETER
    with pytest.raises(orc.OracleError) as e:
        orc.rotary(np.ones(4), 2, 1, 2, 2 ** 64 - 1, 1e6)
    assert e.value.code == orc.SIZE_OVERFLOW
    with pytest.raises(orc.OracleError) as e:
        orc.rotary(np.ones(4) * np.nan, 1, 1, 4, 0, 1e6)
    assert e.value.code == orc.NON_FINITE
    sc, pr = np.full(2, 456.0, np.float32), np.full(2, 789.0, np.float32)
    with pytest.raises(orc.OracleError) as e:
        orc.attention(np.ones(4), np.ones(6), np.ones(6), 1, 2, 3, 2, out=(out, sc, pr))
    assert e.value.code == orc.INVALID_PARAMETER
    with pytest.raises(orc.OracleError) as e:
        orc.attention(np.ones(4), np.ones(2), np.full(2, np.nan), 1, 2, 1, 2, out=(out, sc, pr))
    assert (e.value.code, e.value.tensor) == (orc.NON_FINITE, "v")
    with pytest.raises(orc.OracleError) as e:
        orc.attention(np.ones(4), np.ones(1), np.ones(2), 1, 2, 1, 2, out=(out, sc, pr))
    assert (e.value.code, e.value.tensor) == (orc.LENGTH, "k")
    assert out.tolist() == [123.0] * 4 and sc.tolist() == [456.0] * 2 and pr.tolist() == [789.0] * 2


def test_cached_rejects_invalid_shapes_before_writes(orc):
    """tests/cached_attention.rs:58-99."""
    for variant in range(7):
        shape = dict(tokens=1, query_heads=2, kv_heads=1, head_dim=2, capacity=3, offset=1)
        k, v, q = np.zeros(6, np.float32), np.zeros(6, np.float32), np.zeros(4, np.float32)
        if variant == 0:
            shape["offset"] = 2 ** 64 - 1
        elif variant == 1:
            shape["offset"] = 3
        elif variant == 2:
            shape["kv_heads"] = 3
        elif variant == 3:
            shape["tokens"] = 0
        elif variant == 4:
            shape["head_dim"] = 2 ** 64 - 1
        elif variant == 5:
            k[0] = np.nan
        else:
            v[2] = np.inf
        ctx = np.full(4, 123.0, np.float32)
        sc, pr = np.full(3, 456.0, np.float32), np.full(3, 789.0, np.float32)
        with pytest.raises(orc.OracleError):
            orc.attention_cached(q, k, v, shape["tokens"], shape["query_heads"], shape["kv_heads"],
                                 shape["head_dim"], shape["capacity"], shape["offset"],
                                 out=(ctx, sc, pr))
        assert ctx.tolist() == [123.0] * 4 and sc.tolist() == [456.0] * 3
        assert pr.tolist() == [789.0] * 3


def test_arithmetic_overflow_is_non_finite(orc):
    with pytest.raises(orc.OracleError) as e:
        orc.rotary(np.full(2, np.finfo(np.float32).max), 1, 1, 2, 1, 1.0)
    assert (e.value.code, e.value.tensor) == (orc.NON_FINITE, "rotary output")
    with pytest.raises(orc.OracleError) as e:
        orc.attention([np.finfo(np.float32).max], [2.0], [0.0], 1, 1, 1, 1)
    assert (e.value.code, e.value.tensor) == (orc.NON_FINITE, "attention scores")


# ---- closed forms that a dropped term / wrong index would break ----

def test_zero_query_gives_uniform_probabilities_and_mean_of_values(orc):
    """Zero Q -> probabilities 1/L; dyadic V -> exact mean (src/metal/native_profile.rs:96-197)."""
    rng = np.random.default_rng(3)
    L, D, hq, hkv = 16, 8, 4, 2
    cap = 20
    k = rng.standard_normal(hkv * cap * D).astype(np.float32)
    v = np.zeros((hkv, cap, D), np.float32)
    v[:, :L] = rng.integers(-8, 8, size=(hkv, L, D)) / 4.0
    q = np.zeros(hq * D, np.float32)
    ctx, sc, pr = orc.attention_cached(q, k, v.reshape(-1), 1, hq, hkv, D, cap, L - 1)
    assert np.all(pr[:L] == np.float32(1.0 / L))
    expected = v[:, :L].mean(axis=1)
    for h in range(hq):
        assert np.array_equal(ctx[h * D:(h + 1) * D], expected[h // 2])


def test_softmax_known_values_and_mask(orc):
    out = orc.softmax([0.0, math.log(3.0)], 1, 2)
    close(out, [0.25, 0.75], atol=1e-7, rtol=0)
    out = orc.softmax([1.0, 2.0, 3.0, 4.0], 2, 2, mask=[1, 0, 0, 1])
    assert out.tolist() == [1.0, 0.0, 0.0, 1.0]
    with pytest.raises(orc.OracleError) as e:
        orc.softmax([1.0, 2.0], 1, 2, mask=[0, 0])
    assert e.value.code == orc.FULLY_MASKED


def test_window_one_attends_to_self_only(orc):
    rng = np.random.default_rng(5)
    q = rng.standard_normal(3 * 2 * 4).astype(np.float32)
    k = rng.standard_normal(1 * 6 * 4).astype(np.float32)
    v = rng.standard_normal(1 * 6 * 4).astype(np.float32)
    ctx, _, pr = orc.window_attention(q, k, v, 3, 6, 6, 2, 1, 4, 3, 0, 1, 1.0)
    for t in range(3):
        for h in range(2):
            row = pr.reshape(2, 3, 6)[h, t]
            assert row[3 + t] == 1.0 and row.sum() == 1.0
            assert np.array_equal(ctx.reshape(3, 2, 4)[t, h], v.reshape(6, 4)[3 + t])


def test_window_equals_cached_composition_in_fp64(orc):
    """Independent FP64 brute force for a wide-window GQA case with absolute origins."""
    rng = np.random.default_rng(11)
    Q, K, hq, hkv, D, W, cap = 5, 12, 6, 3, 7, 4, 15
    q = rng.standard_normal(Q * hq * D).astype(np.float32)
    k = rng.standard_normal(hkv * cap * D).astype(np.float32)
    v = rng.standard_normal(hkv * cap * D).astype(np.float32)
    scale = 0.37
    ctx, sc, pr = orc.window_attention(q, k, v, Q, K, cap, hq, hkv, D, 107, 100, W, scale)
    qq = q.reshape(Q, hq, D).astype(np.float64)
    kk = k.reshape(hkv, cap, D).astype(np.float64)
    vv = v.reshape(hkv, cap, D).astype(np.float64)
    for h in range(hq):
        g = h // (hq // hkv)
        for t in range(Q):
            pos = 107 + t
            s = (kk[g, :K] @ qq[t, h]) * scale
            vis = [j for j in range(K) if 100 + j <= pos and pos - (100 + j) < W]
            p = np.exp(s[vis] - s[vis].max())
            p /= p.sum()
            close(pr.reshape(hq, Q, K)[h, t, vis], p, atol=1e-7, rtol=1e-6)
            close(ctx.reshape(Q, hq, D)[t, h], p @ vv[g, vis], atol=1e-6, rtol=1e-5)


# ---- gemma-local-attention-v1 (src/cpu/window_attention/tests.rs:31-131) ----

def test_window_attention_matches_gemma_local_fixture(orc):
    g = Golden("gemma_local_attention_v1")
    for case in g.meta["cases"]:
        if case["queries"] == 0:
            continue
        Q, K, hq, hkv, D = case["queries"], case["keys"], case["q_heads"], case["kv_heads"], case["dims"]
        cap = K + 2
        arr = {n: g[case["arrays"][n]] for n in case["arrays"]}
        q = head_major_to_token_major(arr["q"], hq, Q, D)
        k = np.full((hkv, cap, D), np.nan, np.float32)
        v = k.copy()
        k[:, :K] = arr["k"]
        v[:, :K] = arr["v"]
        ctx, sc, pr = orc.window_attention(
            q, k.reshape(-1), v.reshape(-1), Q, K, cap, hq, hkv, D,
            case["origin"] + K - Q, case["origin"], case["window"], case["scale"])
        close(ctx, head_major_to_token_major(arr["output"], hq, Q, D))
        close(sc, arr["scores"])
        close(pr, arr["probabilities"])
        mask = arr["mask"].reshape(-1)
        for h in range(hq):
            row = pr.reshape(hq, Q * K)[h]
            assert np.all(row[~mask].view(np.uint32) == 0)


# ---- gemma-kv-v1 ring views (src/cpu/span_attention/tests.rs:212) ----

def test_span_attention_over_ring_matches_gemma_kv_fixture(orc):
    g = Golden("gemma_kv_v1")
    checked = 0
    for case in g.meta["cases"]:
        hkv, hq, D, cap, W = case["kv_heads"], case["query_heads"], case["dims"], case["capacity"], case["window"]
        for step in case["steps"]:
            arr = {n: g[step["arrays"][n]] for n in step["arrays"]}
            tokens, offset = step["count"], step["before"]
            ring_k = arr["ring_before_k"].reshape(hkv, cap, D)
            ring_v = arr["ring_before_v"].reshape(hkv, cap, D)
            spans = orc.old_spans(cap, offset, W)
            frozen = step["old_spans"]
            live = [s for s in spans if s[2] > 0]
            assert [[s[1], s[2]] for s in live] == frozen
            segments = []
            for position, slot, rows in spans:
                if rows == 0:
                    segments.append(orc.Segment(np.zeros(0), np.zeros(0), 0, 0, offset))
                    continue
                stride = cap * D
                begin = slot * D
                end = (hkv - 1) * stride + begin + rows * D
                segments.append(orc.Segment(ring_k.reshape(-1)[begin:end], ring_v.reshape(-1)[begin:end],
                                            rows, stride, position))
            segments.append(orc.Segment(arr["new_k"].reshape(-1), arr["new_v"].reshape(-1), tokens,
                                        tokens * D, offset))
            start = orc.view_start(offset, W)
            keys = offset + tokens - start
            q = head_major_to_token_major(arr["q"], hq, tokens, D)
            ctx, _, _ = orc.span_attention(q, segments, tokens, keys, hq, hkv, D, offset, start, W, 1.0)
            close(ctx, head_major_to_token_major(arr["context"], hq, tokens, D))
            # committed ring after copy_runs equals the frozen state
            after_k, after_v = ring_k.copy(), ring_v.copy()
            new_k = arr["new_k"].reshape(hkv, tokens, D)
            new_v = arr["new_v"].reshape(hkv, tokens, D)
            for src, slot, rows in orc.copy_runs(cap, offset, tokens, W is not None):
                after_k[:, slot:slot + rows] = new_k[:, src:src + rows]
                after_v[:, slot:slot + rows] = new_v[:, src:src + rows]
            assert np.array_equal(after_k.reshape(-1), arr["ring_after_k"].reshape(-1))
            assert np.array_equal(after_v.reshape(-1), arr["ring_after_v"].reshape(-1))
            checked += 1
    assert checked >= 20


# ---- ring geometry brute force (src/model/window_rows.rs:95-190) ----

def test_old_spans_match_absolute_rows(orc):
    for cap in range(1, 13):
        for sliding in (False, True):
            window = cap if sliding else None
            for offset in range(49):
                if not sliding and offset > cap:
                    continue
                spans = orc.old_spans(cap, offset, window)
                actual = [(p + i, s + i) for p, s, r in spans for i in range(r)]
                expected = [(p, p % cap if sliding else p) for p in range(offset)
                            if not sliding or offset - p < cap]
                assert actual == expected
                assert orc.view_start(offset, window) == (expected[0][0] if expected else offset)


def test_copy_runs_match_tokenwise_oracle(orc):
    for cap in range(1, 13):
        for sliding in (False, True):
            for offset in range(49):
                for tokens in range(1, 17):
                    if offset + tokens > 64 or (not sliding and offset + tokens > cap):
                        continue
                    slot_of = (lambda p: p % cap) if sliding else (lambda p: p)
                    actual = [None] * cap
                    for p in range(offset):
                        actual[slot_of(p)] = p
                    expected = list(actual)
                    before = list(actual)
                    for p in range(offset, offset + tokens):
                        expected[slot_of(p)] = p
                    copied = [False] * cap
                    for src, slot, rows in orc.copy_runs(cap, offset, tokens, sliding):
                        for i in range(rows):
                            assert not copied[slot + i]
                            copied[slot + i] = True
                            actual[slot + i] = offset + src + i
                    assert actual == expected
                    assert sum(copied) == min(tokens, cap)
                    assert all(actual[s] == before[s] for s in range(cap) if not copied[s])


def test_ring_geometry_near_size_boundary(orc):
    offset = 2 ** 64 - 2
    spans = orc.old_spans(512, offset, 512)
    assert spans[0][2] + spans[1][2] == 511
    assert spans[0][0] == offset - 511
    assert spans[1][0] + spans[1][2] == offset
    runs = orc.copy_runs(512, offset, 1, True)
    assert runs[0] == (0, offset % 512, 1) and runs[1][2] == 0
    single = orc.old_spans(1, offset, 1)
    assert single[0][2] + single[1][2] == 0
    assert orc.view_start(offset, 1) == offset


# ---- gemma-softcap-v1 (src/cpu/softcap/tests.rs:19) + score-softcap extension ----

def test_logit_softcap_matches_fixture(orc):
    g = Golden("gemma_softcap_v1")
    checked = 0
    for case in g.meta["cases"]:
        if case["width"] == 0:
            with pytest.raises(orc.OracleError):
                orc.logit_softcap(np.zeros(0), case["cap"])
            continue
        out = orc.logit_softcap(g[case["input"]], case["cap"])
        close(out, g[case["math"]])
        close(out, g[case["staged_fp32"]])
        checked += 1
    assert checked == 5
    for cap in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(orc.OracleError):
            orc.logit_softcap(np.ones(3), cap)


def test_score_softcap_equals_softcapped_scores_then_softmax(orc):
    """The score-softcap extension composes logit_softcap with the window softmax."""
    rng = np.random.default_rng(9)
    Q, K, hq, D, cap = 3, 9, 2, 16, 50.0
    q = (rng.standard_normal(Q * hq * D) * 8).astype(np.float32)
    k = (rng.standard_normal(K * D) * 8).astype(np.float32)
    v = rng.standard_normal(K * D).astype(np.float32)
    _, raw, _ = orc.window_attention(q, k, v, Q, K, K, hq, 1, D, K - Q, 0, None, 0.25)
    ctx, sc, pr = orc.window_attention(q, k, v, Q, K, K, hq, 1, D, K - Q, 0, None, 0.25, softcap=cap)
    assert np.array_equal(sc, orc.logit_softcap(raw, cap))
    assert np.abs(sc).max() <= cap and np.abs(raw).max() > cap
    s = sc.reshape(hq, Q, K).astype(np.float64)
    for h in range(hq):
        for t in range(Q):
            vis = K - Q + t + 1
            p = np.exp(s[h, t, :vis] - s[h, t, :vis].max())
            p /= p.sum()
            close(pr.reshape(hq, Q, K)[h, t, :vis], p, atol=1e-7, rtol=1e-6)


# ---- fp16-v1: half-storage values widened to FP32 (manifest gate_policy) ----

def test_attention_on_half_storage_matches_fp16_fixture(orc):
    g = Golden("fp16_v1")
    for case in TINY_CASES:
        for layer in range(2):
            p = f"cases.{case}.layers.{layer}"
            q = g.arrays[f"{p}.q_rotary"].astype(np.float32).reshape(-1)
            tokens = q.size // 32
            ck = g.arrays[f"{p}.cache_k"].astype(np.float32)
            cv = g.arrays[f"{p}.cache_v"].astype(np.float32)
            assert np.all(ck[:, tokens:] == 0) and np.all(cv[:, tokens:] == 0)
            k = ck[:, :tokens].transpose(1, 0, 2).reshape(-1)
            v = cv[:, :tokens].transpose(1, 0, 2).reshape(-1)
            ctx, sc, pr = orc.attention(q, k, v, tokens, 4, 2, 8)
            for name, got in (("attention_scores", sc), ("attention_probabilities", pr),
                              ("attention_context", ctx)):
                gate = g.meta["gates"][f"{p}.{name}"]
                close(got, g.arrays[f"{p}.{name}"].astype(np.float32), atol=gate["atol"], rtol=gate["rtol"])
            # the cached operator over the frozen half cache gives the same context
            cctx, _, _ = orc.attention_cached(q, ck.reshape(-1), cv.reshape(-1), tokens, 4, 2, 8, 32, 0)
            assert np.array_equal(cctx, ctx)


def test_greedy_lowest_index_on_ties(orc):
    assert orc.greedy([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.greedy([-1.0]) == 0
    assert orc.greedy([-0.0, 0.0]) == 0 and orc.greedy([-1.0, 0.0, -0.0]) == 1  # zeros tie
    with pytest.raises(orc.OracleError):
        orc.greedy([1.0, float("nan")])
    with pytest.raises(orc.OracleError):
        orc.greedy([])


# ---- tiny-v1 linear projections and greedy trace (tests/cpu_linear.rs, tests/cpu_decoder.rs) ----

def test_matmul_manual_known_answers(orc):
    """tests/cpu_linear.rs:59-72: the 2x3 manual projection with and without bias."""
    g = Golden("tiny_v1_linear")
    x, w, b = g.arrays["manual.inputs"], g.arrays["manual.weight"], g.arrays["manual.bias"]
    assert orc.matmul(x, w, 2, 3, 2, bias=b).tolist() == [-3.75, 14.5, -2.75, 5.0]
    assert g.arrays["manual.output"].reshape(-1).tolist() == [-3.75, 14.5, -2.75, 5.0]
    assert orc.matmul(x[:1], w, 1, 3, 2).tolist() == [-4.0, 15.0]
    with pytest.raises(orc.OracleError) as e:
        orc.matmul([1.0, 1.0, 1.0], [1.0, np.nan, 1.0], 1, 3, 1)
    assert e.value.code == orc.NON_FINITE
    with pytest.raises(orc.OracleError) as e:
        orc.matmul([np.finfo(np.float32).max], [2.0], 1, 1, 1)
    assert (e.value.code, e.value.tensor) == (orc.NON_FINITE, "output")


def test_matmul_matches_every_tiny_projection(orc):
    """tests/cpu_linear.rs:75-165: q/k/v (with bias), o (the attention context's
    projection), gate, up and down of every case and layer."""
    g = Golden("tiny_v1_linear")
    checked = 0
    for case in TINY_CASES:
        tokens = len(g.arrays[f"cases.{case}.tokens"])
        for layer in range(2):
            pre, wp = f"cases.{case}.layers.{layer}", f"weights.layers.{layer}"
            for name, src, dst, bias in (("q", "input_norm", "q_projection", True),
                                         ("k", "input_norm", "k_projection", True),
                                         ("v", "input_norm", "v_projection", True),
                                         ("o", "attention_context", "attention_projection", False),
                                         ("gate", "post_attention_norm", "gate_projection", False),
                                         ("up", "post_attention_norm", "up_projection", False),
                                         ("down", "gated", "down_projection", False)):
                w = g.arrays[f"{wp}.{name}_proj.weight"]
                b = g.arrays[f"{wp}.{name}_proj.bias"] if bias else None
                out = orc.matmul(g.arrays[f"{pre}.{src}"].reshape(-1), w, tokens, w.shape[1],
                                 w.shape[0], bias=b)
                close(out, g.arrays[f"{pre}.{dst}"])
                checked += 1
    assert checked == 70


def test_greedy_matches_tiny_trace(orc):
    """tests/cpu_decoder.rs:170-192: each step's frozen logits choose the frozen token."""
    g = Golden("tiny_v1_linear")
    expected = g.meta["greedy"]["generated_tokens"]
    assert g.arrays["greedy.tokens"].tolist() == expected
    for step, token in enumerate(expected):
        assert orc.greedy(g.arrays[f"greedy.step_{step}.logits"]) == token


def test_rmsnorm_closed_form(orc):
    x = np.array([3.0, 4.0], np.float32)
    out = orc.rmsnorm(x, [1.0, 2.0], 1, 2, 1e-6)
    rms = math.sqrt((9 + 16) / 2 + 1e-6)
    close(out, [3 / rms, 8 / rms], atol=1e-7, rtol=1e-7)


# ---- tiny-v1 normalisations (tests/cpu_reductions.rs:16-62, 140-175) ----

def test_rmsnorm_matches_every_tiny_normalization(orc):
    """Every normalisation tiny-v1 freezes: per layer the input norm (of the
    embedding or the previous layer's output) and the post-attention norm (of the
    attention residual), then the final norm, hidden 32, epsilon 1e-6."""
    g = Golden("tiny_v1_norms")
    checked = 0
    for case in TINY_CASES:
        tokens = len(g.arrays[f"cases.{case}.tokens"])
        for layer in range(2):
            prefix = f"cases.{case}.layers.{layer}"
            first = f"cases.{case}.embedding" if layer == 0 else f"cases.{case}.layers.0.output"
            for src, weight, expected in (
                    (first, f"weights.layers.{layer}.input_layernorm", f"{prefix}.input_norm"),
                    (f"{prefix}.attention_residual", f"weights.layers.{layer}.post_attention_layernorm",
                     f"{prefix}.post_attention_norm")):
                out = orc.rmsnorm(g.arrays[src].reshape(-1), g.arrays[weight], tokens, 32, 1e-6)
                close(out, g.arrays[expected])
                checked += 1
        out = orc.rmsnorm(g.arrays[f"cases.{case}.layers.1.output"].reshape(-1), g.arrays["weights.norm"],
                          tokens, 32, 1e-6)
        close(out, g.arrays[f"cases.{case}.final_norm"])
        checked += 1
    assert checked == 25


def test_rmsnorm_edge_cases_and_epsilon(orc):
    """Zero rows, FP32 overflow of the squares, and an epsilon that decides the
    result (tests/cpu_reductions.rs:140-175)."""
    g = Golden("tiny_v1_norms")
    close(orc.rmsnorm(np.zeros(32), np.ones(32), 1, 32, 1e-6), g.arrays["edge.rmsnorm.zero_output"])
    close(orc.rmsnorm(g.arrays["edge.rmsnorm.large_input"].reshape(-1), np.ones(4), 1, 4, 1e-6),
          g.arrays["edge.rmsnorm.large_output"])
    fmax = float(np.finfo(np.float32).max)
    tiny = float(np.array([1], np.uint32).view(np.float32)[0])
    r = 2.0 / math.sqrt(3.0)
    close(orc.rmsnorm([fmax, -fmax, 0.0, fmax], np.ones(4), 1, 4, tiny), [r, -r, 0.0, r])
    # Epsilon is added to the mean square: x = 1e-3 over a row of 4 with epsilon 3e-6 gives
    # 1e-3 / sqrt(1e-6 + 3e-6) = 0.5, where an epsilon added to the root (or dropped) would not.
    close(orc.rmsnorm(np.full(4, 1e-3), np.ones(4), 1, 4, 3e-6), np.full(4, 0.5), atol=1e-7, rtol=1e-6)


# ---- gemma-rotary-v1 (src/cpu/proportional_rotary/tests.rs:34-71) ----

def test_proportional_rotary_matches_gemma_rotary_fixture(orc):
    """Every case of gemma-rotary-v1: factors 1, 2 and 2.5, rotated dims 0..128 of
    8..512, positions up to 131071.  Outputs within 1e-5 + 1e-4|e|, and the pairs
    past rotated_dims are copied bit for bit."""
    g = Golden("gemma_rotary_v1")
    checked = 0
    for case in g.meta["cases"]:
        if case["tokens"] == 0:
            continue  # empty sequences make no operator calls
        x = g[case["arrays"]["input"]].astype(np.float32).reshape(-1)
        out = orc.proportional_rotary(x, case["tokens"], case["heads"], case["dims"],
                                      case["rotated_dims"], case["offset"], case["base"], case["factor"])
        close(out, g[case["arrays"]["output"]])
        D, half = case["dims"], case["dims"] // 2
        for first in range(0, x.size, D):
            for pair in range(case["rotated_dims"] // 2, half):
                for i in (first + pair, first + pair + half):
                    assert out.view(np.uint32)[i] == x.view(np.uint32)[i]
        checked += 1
    assert checked == 7


# ---- llama3-rotary-v1 (src/cpu/llama3_rotary/tests.rs:63-302) ----

def _llama3_ordinary(theta, pair, head_dim):
    return float(np.float32(theta)) ** (-(2.0 * pair) / head_dim)


def test_llama3_rotary_matches_llama3_rotary_fixture(orc):
    """Every case of llama3-rotary-v1 (position 0, short inputs, the original
    context edge, the declared 131072 end, position 2^20, factor 1, other band
    parameters): FP64 inverse frequencies within 1e-15 + 1e-13|e| and outputs
    within 1e-5 + 1e-4|e|, the reference's own gates."""
    g = Golden("llama3_rotary_v1")
    for case in g.meta["cases"]:
        name, D = case["name"], case["head_dim"]
        s = orc.llama3_scaling(case["factor"], case["low"], case["high"], case["original"])
        want = g.arrays[f"{name}.inverse_frequencies"]
        assert want.size == D // 2
        for pair, e in enumerate(want):
            a = orc.llama3_inverse_frequency(s, _llama3_ordinary(case["theta"], pair, D))
            assert abs(a - e) <= 1e-15 + 1e-13 * abs(e), (name, pair, a, e)
        out = orc.llama3_rotary(g.arrays[f"{name}.input"], case["tokens"], case["heads"], D,
                                case["offset"], case["theta"], case["factor"], case["low"],
                                case["high"], case["original"])
        close(out, g.arrays[f"{name}.output"])
    assert len(g.meta["cases"]) == 7


def test_llama3_scaling_bands_and_edges(orc):
    """The fixture's controls, the band edges (wavelength original/high keeps the
    ordinary frequency, original/low divides it by factor exactly), continuity one
    ulp either side of each edge, and the 15/3/14 split of theta 500000, D 64 over
    the three bands (src/cpu/llama3_rotary/tests.rs:97-127)."""
    g = Golden("llama3_rotary_v1")
    s = orc.llama3_scaling(32.0, 1.0, 4.0, 8192)
    assert len(g.meta["controls"]) == 5
    for c in g.meta["controls"]:
        a = orc.llama3_inverse_frequency(s, c["ordinary"])
        assert abs(a - c["scaled"]) <= 1e-17 + 1e-13 * abs(c["scaled"])
    high = 2.0 * math.pi * 4.0 / 8192.0
    low = 2.0 * math.pi / 8192.0
    assert orc.llama3_inverse_frequency(s, high) == high
    assert orc.llama3_inverse_frequency(s, low) == low / 32.0
    for edge in (low, high):
        at = orc.llama3_inverse_frequency(s, edge)
        for x in (np.nextafter(edge, 0.0), np.nextafter(edge, 1.0)):
            assert abs(orc.llama3_inverse_frequency(s, float(x)) - at) < 1e-17
    # Inside the band the result is the linear blend of ordinary/factor and
    # ordinary in original/wavelength: at the band's middle (wavelength 4096,
    # original/wavelength 2 = low + (high - low) / 3) one third of the ordinary
    # frequency is kept.
    mid = 2.0 * math.pi / 4096.0
    want = (2.0 / 3.0) * mid / 32.0 + (1.0 / 3.0) * mid
    assert abs(orc.llama3_inverse_frequency(s, mid) - want) <= 1e-15 * want
    bands = [0, 0, 0]
    for pair in range(32):
        wavelength = 2.0 * math.pi / _llama3_ordinary(500000.0, pair, 64)
        assert wavelength not in (2048.0, 8192.0)
        bands[0 if wavelength < 2048.0 else (2 if wavelength > 8192.0 else 1)] += 1
    assert bands == [15, 3, 14]


def test_llama3_rotary_reduces_to_ordinary_rotary(orc):
    """Factor 1, and a theta whose every wavelength sits below original/high, give
    the split-half rotary bit for bit; at short positions the scaled pairs differ
    (scaling applies before the position, even for short inputs); chunks at
    absolute offsets join to the whole (src/cpu/llama3_rotary/tests.rs:130-204)."""
    x = np.array([((i * 7 % 31) - 15) * 0.125 for i in range(96)], np.float32)
    for theta, factor in ((500000.0, 1.0), (2.0, 32.0)):
        a = orc.llama3_rotary(x, 3, 2, 16, 131069, theta, factor, 1.0, 4.0, 8192)
        b = orc.rotary(x, 3, 2, 16, 131069, theta)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    x = np.array([((i * 7 % 31) - 15) * 0.125 for i in range(384)], np.float32)
    whole = orc.llama3_rotary(x, 3, 2, 64, 131069, 500000.0, 32.0, 1.0, 4.0, 8192)
    for chunk in (1, 2):
        parts = []
        for first in range(0, 3, chunk):
            n = min(chunk, 3 - first)
            parts.append(orc.llama3_rotary(x[first * 128:(first + n) * 128], n, 2, 64,
                                           131069 + first, 500000.0, 32.0, 1.0, 4.0, 8192))
        assert np.array_equal(np.concatenate(parts), whole)
    short = orc.llama3_rotary(x, 3, 2, 64, 1, 500000.0, 32.0, 1.0, 4.0, 8192)
    ordinary = orc.rotary(x, 3, 2, 64, 1, 500000.0)
    assert not np.array_equal(short.view(np.uint32), ordinary.view(np.uint32))
    # The pairs below original/high (the first 15 of 32) keep the ordinary rotation.
    sr, orr = short.reshape(3, 2, 64), ordinary.reshape(3, 2, 64)
    assert np.array_equal(sr[..., :15], orr[..., :15]) and np.array_equal(sr[..., 32:47], orr[..., 32:47])


def test_llama3_rotary_rejects_invalid_parameters(orc):
    """Llama3Scaling::new and llama3_rotary refuse what the reference refuses
    (src/cpu/llama3_rotary/tests.rs:207-302); position 2^53 is accepted."""
    bad = [(v, 1.0, 4.0, 8192) for v in (0.0, -1.0, 0.5, math.nan, math.inf)]
    bad += [(32.0, v, 4.0, 8192) for v in (0.0, -1.0, math.nan, math.inf)]
    bad += [(32.0, 1.0, v, 8192) for v in (0.0, -1.0, math.nan, math.inf)]
    bad += [(32.0, 4.0, 4.0, 8192), (32.0, 5.0, 4.0, 8192), (32.0, 1.0, 4.0, 0),
            (32.0, 1.0, 4.0, (1 << 53) + 1)]
    for args in bad:
        with pytest.raises(orc.OracleError) as e:
            orc.llama3_scaling(*args)
        assert e.value.name == "InvalidParameter"
    s = orc.llama3_scaling(32.0, 1.0, 4.0, 8192)
    for v in (0.0, -1.0, math.nan, math.inf, 5e-324):
        with pytest.raises(orc.OracleError):
            orc.llama3_inverse_frequency(s, v)
    ones = np.ones(16, np.float32)
    geometry = [(0, 1, 16, 1, 500000.0), (1, 0, 16, 1, 500000.0), (1, 1, 3, 1, 500000.0),
                (1, 1, 16, (1 << 53) + 1, 500000.0), (1, 1, 16, 1, 0.0), (1, 1, 16, 1, math.nan)]
    for tokens, heads, d, offset, theta in geometry:
        with pytest.raises(orc.OracleError):
            orc.llama3_rotary(ones, tokens, heads, d, offset, theta, 32.0, 1.0, 4.0, 8192)
    for value in (math.nan, math.inf, -math.inf):
        x = ones.copy()
        x[15] = value
        with pytest.raises(orc.OracleError) as e:
            orc.llama3_rotary(x, 1, 1, 16, 1, 500000.0, 32.0, 1.0, 4.0, 8192)
        assert e.value.name == "NonFinite"
    fmax = float(np.finfo(np.float32).max)
    with pytest.raises(orc.OracleError) as e:
        orc.llama3_rotary(np.array([fmax, -fmax], np.float32), 1, 1, 2, 1, 500000.0, 32.0, 1.0,
                          4.0, 8192)
    assert e.value.name == "NonFinite"
    orc.llama3_rotary(ones, 1, 1, 16, 1 << 53, 500000.0, 32.0, 1.0, 4.0, 8192)


# ---- gemma-reference-attention-v1 (tools/reference/test_gemma_reference_attention.py:46-58) ----

def _reference_attention_oracle(orc, case, q, k, v):
    """window_attention over one case: q [1, H, Q, D] head-major, k/v [1, 1, K, D], scale 1."""
    H, Q, K, D = case["heads"], case["queries"], case["keys"], case["head_dim"]
    qt = head_major_to_token_major(q.astype(np.float32), H, Q, D)
    return orc.window_attention(qt, k.astype(np.float32).reshape(-1), v.astype(np.float32).reshape(-1),
                                Q, K, K, H, 1, D, case["query_start"], case["key_start"],
                                case["window"], 1.0)


def test_window_attention_matches_reference_attention_contracts(orc):
    """The eight frozen cases (D up to 512, 1025 keys, windows 4 and 512, translated
    origins, mixed-sign cancellation, near ties): the oracle's window_attention on
    the staged FP32 inputs meets the staged contract's scores, probabilities and
    contexts at the reference's gate, and the FP64 contract's contexts too."""
    g = Golden("gemma_reference_attention_v1")
    for case in g.meta["cases"]:
        q, k, v = reference_attention_inputs(g, case, "staged_fp32")
        ctx, sc, pr = _reference_attention_oracle(orc, case, q, k, v)
        H, Q, D = case["heads"], case["queries"], case["head_dim"]
        name = case["name"]
        close(ctx, head_major_to_token_major(g.arrays[f"{name}.staged_fp32.context"], H, Q, D))
        close(sc, g.arrays[f"{name}.staged_fp32.scores"])
        close(pr, g.arrays[f"{name}.staged_fp32.probabilities"])
        close(ctx, head_major_to_token_major(g.arrays[f"{name}.math.context"], H, Q, D))
        mask = g.arrays[f"{name}.staged_fp32.probabilities"].reshape(-1) == 0
        assert np.all(pr.reshape(-1)[mask].view(np.uint32) == 0)


def test_proportional_rotary_reduces_to_rotary(orc):
    """Full rotated dims and factor 1 make proportional rotary the split-half rotary."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(3 * 2 * 8).astype(np.float32)
    a = orc.rotary(x, 3, 2, 8, 4, 10000.0)
    b = orc.proportional_rotary(x, 3, 2, 8, 8, 4, 10000.0, 1.0)
    assert np.array_equal(a, b)
    c = orc.proportional_rotary(x, 3, 2, 8, 4, 4, 10000.0, 1.0)
    xr = x.reshape(3, 2, 8)
    cr = c.reshape(3, 2, 8)
    assert np.array_equal(cr[:, :, 2:4], xr[:, :, 2:4]) and np.array_equal(cr[:, :, 6:], xr[:, :, 6:])


def test_token_agreement_gate_admits_rare_ties_only():
    """The GPU tests' greedy-token gate: one tie within the context error passes,
    a flip on many rows fails."""
    from gpu_util import assert_tokens_agree

    w = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    tied = np.array([[1.0, 0.999]], np.float32)
    assert assert_tokens_agree(np.array([[0.9995, 1.0]], np.float32), tied, w) == 1
    ref = np.tile(np.array([[1.0, 0.5]], np.float32), (10, 1))
    assert assert_tokens_agree(ref, ref, w) == 0
    with pytest.raises(AssertionError):
        assert_tokens_agree(ref[:, ::-1].copy(), ref, w)  # every row flips
