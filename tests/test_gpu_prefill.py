"""GPU parity of the MFMA prefill kernel on long contexts.

A chunk whose (KV head, row block) workgroups are too few to fill the device
has its visible keys split over several workgroups; the split partials
(running max, mass, unnormalised context) are combined by a second kernel.
These cases make that happen at every supported head size, with GQA groups
that do not divide the 128-row block (7 query heads per KV head), windows
whose splits leave some rows without visible keys, and the score softcap.
The checker is the CPU oracle on the same stored (rounded) values.
"""

import os

import numpy as np
import pytest

from gpu_util import TOL_HALF, assert_tokens_agree, dev, host, log, max_err, stored

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


def _tuned_context(ops, **env):
    """A context created under TKH_* tuning variables (read once, at creation)."""
    saved = {k: os.environ.get(k) for k in env}
    try:
        os.environ.update({k: str(v) for k, v in env.items()})
        return ops.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _cached_chunk(torch, ctx, ops, orc, *, hq, hkv, D, dt, offset, tokens, seed, key_scale=None):
    rng = np.random.default_rng(seed)
    capacity = offset + tokens
    k = rng.standard_normal((hkv, capacity, D)).astype(np.float32)
    if key_scale is not None:
        k[rng.random((hkv, capacity)) < key_scale] *= 8.0
    v = rng.standard_normal((hkv, capacity, D)).astype(np.float32)
    q = rng.standard_normal((tokens, hq, D)).astype(np.float32)
    ks, vs, qs = stored(k, dt), stored(v, dt), stored(q, dt).reshape(-1)
    out = torch.full((tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(qs, dt), dev(ks, dt), dev(vs, dt), out, None, None,
                         ops.CachedAttentionShape(tokens, hq, hkv, D, capacity, offset))
    ref, _, _ = orc.attention_cached(qs, ks, vs, tokens, hq, hkv, D, capacity, offset)
    return host(out), ref


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("offset", [384, 1000, 2048])
def test_qwen3_chunk_over_long_prefix(torch_mod, ctx, ops, orc, dt, offset):
    """configs[1] chunk geometry: 128 tokens of 16/8/128 after `offset` cached keys."""
    log(f"qwen3 chunk of 128 at offset {offset} {dt}")
    got, ref = _cached_chunk(torch_mod, ctx, ops, orc, hq=16, hkv=8, D=128, dt=dt, offset=offset,
                             tokens=128, seed=offset)
    err = max_err(got, ref)
    log(f"  max abs error {err:.3e}")
    assert err <= TOL_HALF
    w = np.random.default_rng(5).standard_normal((2048, 16 * 128)).astype(np.float32)
    ties = assert_tokens_agree(got.reshape(128, -1), ref.reshape(128, -1), w)
    log(f"  tokens identical except {ties} tie(s) within the error bound")


def test_peaky_keys_chunk_llama_shape(torch_mod, ctx, ops, orc):
    """configs[4] stress in one session: 5% of key rows x8, 4096 cached + 128 new."""
    got, ref = _cached_chunk(torch_mod, ctx, ops, orc, hq=32, hkv=8, D=128, dt="bf16", offset=4096,
                             tokens=128, seed=9, key_scale=0.05)
    err = max_err(got, ref)
    log(f"llama 32/8/128 peaky chunk at 4096: max abs error {err:.3e}")
    assert err <= TOL_HALF


def test_gqa7_d64_chunk_rows_straddle_blocks(torch_mod, ctx, ops, orc):
    """14/2/64: 7 query heads per KV head, so a token's rows straddle 128-row blocks."""
    got, ref = _cached_chunk(torch_mod, ctx, ops, orc, hq=14, hkv=2, D=64, dt="bf16", offset=1500,
                             tokens=100, seed=13)
    err = max_err(got, ref)
    log(f"14/2/64 chunk of 100 at 1500: max abs error {err:.3e}")
    assert err <= TOL_HALF


# The chunk kernel's forms: 32 rows per wave, and 16 rows per wave in four-wave
# (64-row, the default) and eight-wave (128-row) workgroups.
FORMS = {"32": {"TKH_PREFILL16": 0}, "16x4": {"TKH_PREFILL16_WAVES": 4}, "16x8": {"TKH_PREFILL16_WAVES": 8}}


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("softcap", [0.0, 50.0])
def test_window_d256_chunk_with_split_keys(torch_mod, ops, orc, softcap, form):
    """configs[3] sliding layer: 8/4/256, W=1024, chunk of 128 at position 3000.  The
    visible range spans 1151 keys, so splits at its ends hold keys only some rows see."""
    torch = torch_mod
    ctx = _tuned_context(ops, **FORMS[form])
    rng = np.random.default_rng(17)
    hq, hkv, D, W = 8, 4, 256, 1024
    queries, keys = 128, 3128
    for dt in ("bf16", "f16"):
        k = stored(rng.standard_normal((hkv, keys, D)) * 3, dt)
        v = stored(rng.standard_normal((hkv, keys, D)), dt)
        q = stored(rng.standard_normal((queries, hq, D)) * 3, dt).reshape(-1)
        out = torch.full((queries * hq * D,), np.nan, dtype=torch.float32, device="cuda")
        shape = ops.WindowAttentionShape(queries, keys, keys, hq, hkv, D, keys - queries, 0, W,
                                         1.0 / 16.0, softcap)
        ops.window_attention(ctx, dev(q, dt), dev(k, dt), dev(v, dt), out, None, None, shape)
        ref, _, _ = orc.window_attention(q, k.reshape(-1), v.reshape(-1), queries, keys, keys, hq, hkv,
                                         D, keys - queries, 0, W, 1.0 / 16.0, softcap=softcap)
        err = max_err(host(out), ref)
        log(f"gemma window chunk {dt} softcap {softcap} form {form}: max abs error {err:.3e}")
        assert err <= TOL_HALF
    ctx.close()


def test_split_results_do_not_depend_on_split_count(torch_mod, ctx, ops, orc):
    """The same chunk through contexts that split its keys 1, 4 and 16 ways agrees with
    the oracle each time (the merge weights are in the kernel's log2 units)."""
    torch = torch_mod
    rng = np.random.default_rng(23)
    hq, hkv, D, T, off = 16, 8, 128, 128, 2000
    cap = off + T
    k = stored(rng.standard_normal((hkv, cap, D)) * 2, "bf16")
    v = stored(rng.standard_normal((hkv, cap, D)), "bf16")
    q = stored(rng.standard_normal((T, hq, D)) * 2, "bf16").reshape(-1)
    ref, _, _ = orc.attention_cached(q, k, v, T, hq, hkv, D, cap, off)
    qd, kd, vd = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16")
    for max_splits in (1, 4, 16):
        c = _tuned_context(ops, TKH_PREFILL_MAX_SPLITS=max_splits, TKH_PREFILL_MIN_KEYS=32)
        out = torch.full((T * hq * D,), np.nan, dtype=torch.float32, device="cuda")
        ops.attention_cached(c, qd, kd, vd, out, None, None,
                             ops.CachedAttentionShape(T, hq, hkv, D, cap, off))
        err = max_err(host(out), ref)
        log(f"max splits {max_splits}: max abs error {err:.3e}")
        assert err <= TOL_HALF


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("key", [40, 256 + 5])
def test_minus_infinity_score_is_nonfinite(torch_mod, ctx, ops, orc, dt, key):
    """A key with -inf in a feature where every query of its group is positive gives
    exactly -inf scores (p = 0, nothing else non-finite): the prefill kernel still
    reports NonFinite, as the reference rejects non-finite K (src/cpu/attention.rs:247-251).
    Key 40 lies in a full tile of the cached prefix, key 261 in the causal diagonal
    tile (visible to the chunk's tokens 5 and later)."""
    torch = torch_mod
    rng = np.random.default_rng(61)
    hq, hkv, D, tokens, offset = 16, 8, 128, 128, 256
    capacity = offset + tokens
    k = rng.standard_normal((hkv, capacity, D)).astype(np.float32)
    v = rng.standard_normal((hkv, capacity, D)).astype(np.float32)
    q = rng.standard_normal((tokens, hq, D)).astype(np.float32)
    g = hq // hkv
    q[:, 3 * g:4 * g, 7] = np.abs(q[:, 3 * g:4 * g, 7]) + 0.25
    bad_k = k.copy()
    bad_k[3, key, 7] = -np.inf
    log(f"prefill -inf score {dt} at key {key}")
    out = torch.full((tokens * hq * D,), 123.0, dtype=torch.float32, device="cuda")
    with pytest.raises(ops.TkhError) as e:
        ops.attention_cached(ctx, dev(stored(q, dt), dt), dev(stored(bad_k, dt), dt),
                             dev(stored(v, dt), dt), out, None, None,
                             ops.CachedAttentionShape(tokens, hq, hkv, D, capacity, offset))
    assert e.value.name == "NonFinite"
    # The same call with the finite key computes correctly afterwards.
    qs, ks, vs = stored(q, dt).reshape(-1), stored(k, dt), stored(v, dt)
    out = torch.full((tokens * hq * D,), np.nan, dtype=torch.float32, device="cuda")
    ops.attention_cached(ctx, dev(qs, dt), dev(ks, dt), dev(vs, dt), out, None, None,
                         ops.CachedAttentionShape(tokens, hq, hkv, D, capacity, offset))
    ref, _, _ = orc.attention_cached(qs, ks, vs, tokens, hq, hkv, D, capacity, offset)
    assert max_err(host(out), ref) <= TOL_HALF
