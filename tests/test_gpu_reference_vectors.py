"""The reference's own attention vectors and adversarial witnesses, run through
the HIP kernels.

  * gemma-reference-attention-v1: eight cases of the FP32 window path (D up to
    512, 1025 keys, windows 4 and 512, translated origins, mixed-sign
    cancellation, near ties), context and the score/probability diagnostics,
    against the fixture's staged-FP32 contract at the reference's gate and the
    oracle at 1e-5 (tools/reference/test_gemma_reference_attention.py:46-58).
  * The Metal kernels' adversarial witnesses (src/metal/online_attention.rs:
    140-280): key counts at and around the 16/32-key tile edges, 1-3 query
    rows, uniform scores, late maxima, one dominant key, and +-65504 extremes,
    at this build's head sizes and through every kernel a chunk can take (the
    streaming decode kernel, the MFMA chunk kernel, and both with 32-key
    splits so every split boundary is crossed).
  * qwen3-attention-inputs-v1: real Qwen3 layer-0 rows (16/8/128) at positions
    0, 41 and 65 (src/metal/compensated_attention.rs:465-561), f16 and bf16,
    through the decode and the chunk kernel.
  * bf16 V values beyond f16's range (the chunk kernel's FP32 recompute) and of
    small magnitude.
"""

import contextlib
import math
import os

import numpy as np
import pytest

from gpu_util import TOL_F32, TOL_HALF, dev, host, log, max_err, stored
from goldens import Golden, close, head_major_to_token_major, reference_attention_inputs

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


@contextlib.contextmanager
def _env(**values):
    """Planner settings are read when a context is created."""
    old = {k: os.environ.get(k) for k in values}
    os.environ.update({k: str(v) for k, v in values.items()})
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _contexts(ops):
    """name -> context: the default planner (decode kernel for few rows), the
    MFMA chunk kernel for every bf16/f16 call in its 32-row and 16-row forms
    (TKH_PREFILL16; the 16-row one in its default 64-row workgroups), and each
    with 32-key splits."""
    out = {"decode": ops.Context(0)}
    with _env(TKH_DECODE_DISABLE=1, TKH_PREFILL16=0):
        out["chunk32"] = ops.Context(0)
    with _env(TKH_DECODE_DISABLE=1, TKH_PREFILL16=1):
        out["chunk16"] = ops.Context(0)
    with _env(TKH_SPLIT_KEYS=32):
        out["decode/split32"] = ops.Context(0)
    with _env(TKH_DECODE_DISABLE=1, TKH_SPLIT_KEYS=32, TKH_PREFILL16=0):
        out["chunk32/split32"] = ops.Context(0)
    with _env(TKH_DECODE_DISABLE=1, TKH_SPLIT_KEYS=32, TKH_PREFILL16=1):
        out["chunk16/split32"] = ops.Context(0)
    return out


# ---- gemma-reference-attention-v1 ----

def test_reference_attention_cases_fp32(torch_mod, ops, orc):
    torch = torch_mod
    g = Golden("gemma_reference_attention_v1")
    ctx = ops.Context(0)
    for case in g.meta["cases"]:
        H, Q, K, D = case["heads"], case["queries"], case["keys"], case["head_dim"]
        q, k, v = reference_attention_inputs(g, case, "staged_fp32")
        qt = head_major_to_token_major(q, H, Q, D).astype(np.float32)
        kk, vv = k.reshape(-1).astype(np.float32), v.reshape(-1).astype(np.float32)
        shape = ops.WindowAttentionShape(Q, K, K, H, 1, D, case["query_start"], case["key_start"],
                                         case["window"], 1.0)
        out = torch.full((Q * H * D,), np.nan, dtype=torch.float32, device="cuda")
        sc = torch.full((H * Q * K,), np.nan, dtype=torch.float32, device="cuda")
        pr = torch.full_like(sc, np.nan)
        qd, kd, vd = (torch.from_numpy(a).cuda() for a in (qt, kk, vv))
        ops.window_attention(ctx, qd, kd, vd, out, sc, pr, shape)
        ref, ref_sc, ref_pr = orc.window_attention(qt, kk, vv, Q, K, K, H, 1, D, case["query_start"],
                                                   case["key_start"], case["window"], 1.0)
        name = case["name"]
        got = host(out)
        close(got, head_major_to_token_major(g.arrays[f"{name}.staged_fp32.context"], H, Q, D))
        close(host(sc), g.arrays[f"{name}.staged_fp32.scores"])
        close(host(pr), g.arrays[f"{name}.staged_fp32.probabilities"])
        masked = g.arrays[f"{name}.staged_fp32.probabilities"].reshape(-1) == 0
        assert np.all(host(pr)[masked].view(np.uint32) == 0)
        # The context-only launch (no diagnostics) takes the attention kernels.
        out2 = torch.full_like(out, np.nan)
        ops.window_attention(ctx, qd, kd, vd, out2, None, None, shape)
        err = max(max_err(got, ref), max_err(host(out2), ref))
        log(f"reference attention {name} (D={D}, keys {K}, window {case['window']}): "
            f"max abs error vs oracle {err:.3e}")
        assert err <= TOL_F32
    ctx.close()


# ---- adversarial witnesses ----

def _witness_keys(pattern, depth, hkv, cap, D):
    k = np.zeros((hkv, cap, D), np.float32)
    for p in range(depth):
        if pattern == 0:
            key = 0.0                                   # uniform distribution
        elif pattern == 1:
            key = (p // 16) * 8.0 - 8.0                 # later maxima, one per 16-key tile
        elif pattern == 2:
            key = 64.0 if p == depth - 1 else -64.0     # one dominant key
        else:
            key = 65504.0 if p == depth - 1 else -65504.0
        k[:, p] = key
    return k


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_adversarial_witnesses_every_kernel(torch_mod, ops, orc, dt, D):
    torch = torch_mod
    hq, hkv, cap = 4, 2, 96
    ctxs = _contexts(ops)
    worst, cases = 0.0, 0
    for depth in (15, 16, 17, 31, 32, 33, 63, 64, 65):
        for rows in (1, 2, 3):
            offset = depth - rows
            for pattern in range(4):
                query = 65504.0 if pattern == 3 else 1.0
                q = np.full((rows, hq, D), query, np.float32)
                k = _witness_keys(pattern, depth, hkv, cap, D)
                v = np.zeros((hkv, cap, D), np.float32)
                for h in range(hkv):
                    for p in range(depth):
                        v[h, p] = (p - 16.0) * 0.125 + h + np.arange(D) * 0.0625 / (D / 8)
                qs, ks, vs = stored(q, dt).reshape(-1), stored(k, dt), stored(v, dt)
                ref, _, _ = orc.attention_cached(qs, ks, vs, rows, hq, hkv, D, cap, offset)
                outs = []
                for name, c in ctxs.items():
                    out = torch.full((rows * hq * D,), np.nan, dtype=torch.float32, device="cuda")
                    ops.attention_cached(c, dev(qs, dt), dev(ks, dt), dev(vs, dt), out, None, None,
                                         ops.CachedAttentionShape(rows, hq, hkv, D, cap, offset))
                    got = host(out)
                    err = max_err(got, ref)
                    worst = max(worst, err)
                    assert err <= TOL_HALF, f"{name} depth {depth} rows {rows} pattern {pattern}: {err}"
                    outs.append(got)
                cases += 1
    log(f"witnesses {dt} D={D}: {cases} cases x {len(ctxs)} kernels, max abs error {worst:.3e}")
    for c in ctxs.values():
        c.close()


# ---- qwen3-attention-inputs-v1 ----

@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_qwen3_layer0_rows_decode_and_chunk_kernels(torch_mod, ops, orc, dt):
    torch = torch_mod
    g = Golden("qwen3_attention_inputs_v1")
    hq, hkv, D = g.meta["query_heads"], g.meta["kv_heads"], g.meta["head_dim"]
    qrows = g.arrays["q_rotary"].astype(np.float32)
    k_tok = g.arrays["k_rotary"].astype(np.float32).reshape(-1, hkv, D)
    v_tok = g.arrays["v_projection"].astype(np.float32).reshape(-1, hkv, D)
    cap = 69
    k = np.full((hkv, cap, D), np.nan, np.float32)
    v = np.full((hkv, cap, D), np.nan, np.float32)
    n = k_tok.shape[0]
    k[:, :n] = k_tok.transpose(1, 0, 2)
    v[:, :n] = v_tok.transpose(1, 0, 2)
    ks, vs = stored(k, dt), stored(v, dt)
    ctxs = _contexts(ops)
    for row, position in enumerate(g.meta["positions"]):
        qs = stored(qrows[row], dt)
        ref, _, _ = orc.attention_cached(qs, ks, vs, 1, hq, hkv, D, cap, position)
        for name, c in ctxs.items():
            out = torch.full((hq * D,), np.nan, dtype=torch.float32, device="cuda")
            ops.attention_cached(c, dev(qs, dt), dev(ks, dt), dev(vs, dt), out, None, None,
                                 ops.CachedAttentionShape(1, hq, hkv, D, cap, position))
            err = max_err(host(out), ref)
            log(f"qwen3 layer-0 {dt} position {position} {name}: max abs error {err:.3e}")
            assert err <= TOL_HALF
    for c in ctxs.values():
        c.close()


# ---- bf16 V values beyond f16's range and of small magnitude ----

def _chunk_case(rng, tokens, hq, hkv, D, cap, offset, v_value, where):
    q = stored(rng.standard_normal((tokens, hq, D)), "bf16").reshape(-1)
    k = stored(rng.standard_normal((hkv, cap, D)), "bf16")
    v = stored(rng.standard_normal((hkv, cap, D)), "bf16")
    v[where] = v_value
    return q, k, v


# The chunk kernel's forms: 32 rows per wave, and 16 rows per wave in four-wave
# (64-row, the default) and eight-wave (128-row) workgroups.
FORMS = {"32": {"TKH_PREFILL16": 0}, "16x4": {"TKH_PREFILL16_WAVES": 4}, "16x8": {"TKH_PREFILL16_WAVES": 8}}


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("offset", [0, 2000])  # 2000: the chunk's keys are split
def test_bf16_value_range_of_the_chunk_kernel(torch_mod, ops, orc, offset, D, form):
    """Every finite bf16 V is computed, as the reference computes it
    (src/cpu/attention.rs:247-251 rejects only non-finite values): 65280, the
    largest value f16 holds, on the MFMA path; 65536, 2^24 - 2^16, 2^24,
    -2^25 and 2^100 by the kernel's FP32 recompute of the rows it overflowed;
    inf is a non-finite input.  The decode kernel computes 2^24 in FP32."""
    torch = torch_mod
    rng = np.random.default_rng(81)
    hq, hkv, tokens = 8, 4, 64
    cap = offset + tokens
    with _env(**FORMS[form]):
        ctx = ops.Context(0)
    shape = ops.CachedAttentionShape(tokens, hq, hkv, D, cap, offset)
    where = (2, offset + 5, 17)
    for v_value, expect in ((65280.0, None), (65536.0, None), (16711680.0, None), (2.0 ** 24, None),
                            (-(2.0 ** 25), None), (2.0 ** 100, None), (np.inf, "NonFinite")):
        q, k, v = _chunk_case(rng, tokens, hq, hkv, D, cap, offset, v_value, where)
        out = torch.zeros(tokens * hq * D, dtype=torch.float32, device="cuda")
        if expect is None:
            ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, None, None,
                                 shape)
            ref, _, _ = orc.attention_cached(q, k, v, tokens, hq, hkv, D, cap, offset)
            got = host(out)
            assert np.isfinite(got).all()
            rel = max_err(got, ref) / float(np.abs(ref).max())
            log(f"bf16 V {v_value:g} at offset {offset}, D={D}, form {form}: relative error {rel:.3e}")
            assert rel <= 2e-3
            continue
        with pytest.raises(ops.TkhError) as e:
            ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, None, None,
                                 shape)
        log(f"bf16 V {v_value:g} at offset {offset}: {e.value}")
        assert e.value.name == expect
    # The decode kernel widens bf16 V to FP32: 2^24 is an ordinary value there.
    q, k, v = _chunk_case(rng, 1, hq, hkv, D, cap, cap - 1, 2.0 ** 24, (1, cap - 3, 9))
    out = torch.zeros(hq * D, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, None, None,
                         ops.CachedAttentionShape(1, hq, hkv, D, cap, cap - 1))
    ref, _, _ = orc.attention_cached(q, k, v, 1, hq, hkv, D, cap, cap - 1)
    assert max_err(host(out), ref) / float(np.abs(ref).max()) <= 1e-5
    ctx.close()


@pytest.mark.parametrize("offset", [0, 2000])
def test_small_bf16_values_in_the_chunk_kernel(torch_mod, ops, orc, offset):
    """V of magnitude about 1e-4 (bf16 values above f16's smallest normal are
    carried exactly): the context's error relative to its own magnitude stays
    at the bar of ordinary values."""
    torch = torch_mod
    rng = np.random.default_rng(82)
    hq, hkv, D, tokens = 8, 4, 128, 64
    cap = offset + tokens
    ctx = ops.Context(0)
    q = stored(rng.standard_normal((tokens, hq, D)), "bf16").reshape(-1)
    k = stored(rng.standard_normal((hkv, cap, D)), "bf16")
    v = stored(1e-4 * rng.standard_normal((hkv, cap, D)), "bf16")
    out = torch.zeros(tokens * hq * D, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, None, None,
                         ops.CachedAttentionShape(tokens, hq, hkv, D, cap, offset))
    ref, _, _ = orc.attention_cached(q, k, v, tokens, hq, hkv, D, cap, offset)
    rel = max_err(host(out), ref) / float(np.abs(ref).max())
    log(f"bf16 V of scale 1e-4 at offset {offset}: relative error {rel:.3e}")
    assert rel <= 2e-3
    ctx.close()
