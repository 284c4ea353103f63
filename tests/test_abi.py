"""The C-ABI library loads, exports every declared symbol, and validates on the host.

These tests run without a GPU: every call below fails host-side validation (or
has a NULL context) before anything touches the device.
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tokhip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tkh_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from toklet_amd import _lib

    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name


def test_bindings_cover_the_header():
    from toklet_amd import _lib

    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_abi_version(lib):
    from toklet_amd import _lib

    text = open(HEADER).read()
    assert lib.tkh_abi_version() == _lib.ABI_VERSION == 2
    assert re.search(r"#define TKH_ABI_VERSION 2u", text)


def test_struct_layouts_match_header():
    """The ctypes mirrors' sizes equal the C structures' (gcc on the header)."""
    import subprocess
    import tempfile

    from toklet_amd import _lib

    names = {"tkh_producer_shape": _lib.ProducerShape, "tkh_session_options": _lib.SessionOptions}
    src = '#include <stdio.h>\n#include "tokhip.h"\nint main(void){' + "".join(
        f'printf("%zu\\n", sizeof({n}));' for n in names) + "return 0;}"
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "s.c"), os.path.join(d, "s")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        sizes = [int(x) for x in subprocess.run([exe], check=True, capture_output=True,
                                                text=True).stdout.split()]
    for (n, cls), size in zip(names.items(), sizes):
        assert ctypes.sizeof(cls) == size, n


def _cached(lib, shape, q_len, kv_len, ctx_len, scores_len=0):
    from toklet_amd import _lib

    err = _lib.Error()
    s = _lib.CachedShape(*shape)
    rc = lib.tkh_attention_cached(None, ctypes.byref(s), _lib.BF16, None, q_len, None, kv_len,
                                  None, kv_len, None, ctx_len, None, scores_len, None, 0,
                                  ctypes.byref(err))
    return rc, err


def test_cached_validation_order_mirrors_reference(lib):
    """Codes follow src/cpu/attention.rs:218-245 (tests/cached_attention.rs:58-99)."""
    from toklet_amd import _lib

    base = (1, 2, 1, 2, 3, 1)  # tokens, Hq, Hkv, D, capacity, offset
    rc, _ = _cached(lib, base, 4, 6, 4)
    assert rc == _lib.INVALID_PARAMETER  # valid shape: only the NULL context remains
    rc, err = _cached(lib, (1, 2, 1, 2, 3, 2 ** 64 - 1), 4, 6, 4)
    assert rc == _lib.SIZE_OVERFLOW
    rc, err = _cached(lib, (1, 2, 1, 2, 3, 3), 4, 6, 4)
    assert rc == _lib.INVALID_PARAMETER and b"capacity" in err.tensor
    rc, err = _cached(lib, (1, 2, 3, 2, 3, 1), 4, 6, 4)
    assert rc == _lib.INVALID_PARAMETER and b"divisible" in err.tensor
    rc, err = _cached(lib, (0, 2, 1, 2, 3, 1), 4, 6, 4)
    assert rc == _lib.ZERO_DIMENSION and err.tensor == b"tokens"
    rc, err = _cached(lib, (1, 2, 1, 2 ** 64 - 1, 3, 1), 4, 6, 4)
    assert rc == _lib.SIZE_OVERFLOW
    rc, err = _cached(lib, base, 4, 5, 4)
    assert rc == _lib.LENGTH and err.tensor == b"k cache" and err.expected == 6 and err.actual == 5
    rc, err = _cached(lib, base, 3, 6, 4)
    assert rc == _lib.LENGTH and err.tensor == b"q"


def test_window_validation_and_fully_masked(lib):
    from toklet_amd import _lib

    def call(**kw):
        d = dict(queries=2, keys=4, capacity=4, query_heads=2, kv_heads=1, head_dim=2,
                 query_start=2, key_start=0, has_window=1, window=2, scale=1.0, softcap=0.0)
        d.update(kw)
        s = _lib.WindowShape(**d)
        err = _lib.Error()
        q = d["queries"] * d["query_heads"] * d["head_dim"]
        kv = d["kv_heads"] * d["capacity"] * d["head_dim"]
        rc = lib.tkh_window_attention(None, ctypes.byref(s), _lib.F32, None, q, None, kv, None,
                                      kv, None, q, None, 0, None, 0, ctypes.byref(err))
        return rc, err

    assert call()[0] == _lib.INVALID_PARAMETER  # NULL context after a valid shape
    assert call(window=0)[0] == _lib.INVALID_PARAMETER
    assert call(scale=0.0)[0] == _lib.INVALID_PARAMETER
    assert call(keys=5)[0] == _lib.INVALID_PARAMETER
    assert call(softcap=-1.0)[0] == _lib.INVALID_PARAMETER
    assert call(queries=0)[0] == _lib.ZERO_DIMENSION
    # queries at positions 7, 8 with keys at [0, 4) and window 2: nothing visible
    rc, err = call(query_start=7)
    assert rc == _lib.FULLY_MASKED and err.index == 0


def test_span_segment_validation(lib):
    from toklet_amd import _lib

    s = _lib.SpanShape(1, 3, 2, 1, 2, 2, 0, 0, 0, 1.0, 0.0)
    segs = (_lib.Segment * 3)()
    segs[0] = _lib.Segment(None, 4, None, 4, 2, 4, 0)
    segs[1] = _lib.Segment(None, 0, None, 0, 0, 0, 2)
    segs[2] = _lib.Segment(None, 2, None, 2, 1, 2, 2)
    err = _lib.Error()
    rc = lib.tkh_span_attention(None, ctypes.byref(s), _lib.F32, None, 4, segs, None, 4, None, 0,
                                None, 0, ctypes.byref(err))
    assert rc == _lib.INVALID_PARAMETER and err.tensor == b"context"
    segs[2] = _lib.Segment(None, 2, None, 2, 1, 2, 3)  # wrong logical origin
    rc = lib.tkh_span_attention(None, ctypes.byref(s), _lib.F32, None, 4, segs, None, 4, None, 0,
                                None, 0, ctypes.byref(err))
    assert rc == _lib.INVALID_PARAMETER and b"origin" in err.tensor
    segs[2] = _lib.Segment(None, 2, None, 2, 1, 2, 2)
    segs[0] = _lib.Segment(None, 4, None, 4, 2, 3, 0)  # heads overlap
    rc = lib.tkh_span_attention(None, ctypes.byref(s), _lib.F32, None, 4, segs, None, 4, None, 0,
                                None, 0, ctypes.byref(err))
    assert rc == _lib.INVALID_PARAMETER and b"overlap" in err.tensor


def test_softcap_validation(lib):
    from toklet_amd import _lib

    err = _lib.Error()
    assert lib.tkh_logit_softcap(None, None, 0, 30.0, ctypes.byref(err)) == _lib.ZERO_DIMENSION
    for cap in (0.0, -1.0, float("nan"), float("inf")):
        assert lib.tkh_logit_softcap(None, None, 4, cap, ctypes.byref(err)) == _lib.INVALID_PARAMETER


def test_project_greedy_validation_order(lib):
    """matmul's checks in order (src/cpu/mod.rs:192-201), then greedy's vocabulary
    bound (src/sampling.rs:7-9), all before any launch."""
    from toklet_amd import _lib

    err = _lib.Error()

    def call(rows, hidden, vocab, ctx_len, w_len, logits_len, tok_len, logits=False):
        lg = ctypes.cast(1, _lib.fptr) if logits else None
        return lib.tkh_project_greedy(None, rows, hidden, vocab, None, ctx_len, None, w_len, lg,
                                      logits_len, None, tok_len, ctypes.byref(err))

    assert call(0, 4, 8, 0, 32, 0, 0) == _lib.ZERO_DIMENSION and err.tensor == b"tokens"
    assert call(2, 0, 8, 0, 0, 0, 2) == _lib.ZERO_DIMENSION and err.tensor == b"in_features"
    assert call(2, 4, 0, 8, 0, 0, 2) == _lib.ZERO_DIMENSION and err.tensor == b"out_features"
    assert call(2, 4, 8, 7, 32, 0, 2) == _lib.LENGTH and err.tensor == b"input"
    assert call(2, 4, 8, 8, 31, 0, 2) == _lib.LENGTH and err.tensor == b"weights"
    assert call(2, 4, 8, 8, 32, 15, 2, logits=True) == _lib.LENGTH and err.tensor == b"output"
    assert call(2, 4, 8, 8, 32, 0, 3) == _lib.LENGTH and err.tensor == b"tokens"
    assert call(1, 1, 2 ** 33, 1, 2 ** 33, 0, 1) == _lib.INVALID_PARAMETER
    assert call(2 ** 40, 2 ** 30, 8, 0, 0, 0, 0) == _lib.SIZE_OVERFLOW
    assert call(2, 4, 8, 8, 32, 16, 2, logits=True) == _lib.INVALID_PARAMETER  # no context


def test_kv_planned_bytes_mirror_kv_owner(lib):
    """capacity::KvOwner::at_capacity (src/capacity.rs:49-80) with a bf16 storage kind."""
    from toklet_amd import _lib

    out = ctypes.c_uint64()
    err = _lib.Error()
    assert lib.tkh_kv_planned_bytes(8, 128, 2048, 0, 0, _lib.BF16, 36, ctypes.byref(out),
                                    ctypes.byref(err)) == 0
    assert out.value == 2 * 36 * 8 * 2048 * 128 * 2
    assert lib.tkh_kv_planned_bytes(4, 256, 4096, 1, 1024, _lib.F32, 1, ctypes.byref(out),
                                    ctypes.byref(err)) == 0
    assert out.value == 2 * 4 * 1024 * 256 * 4
    assert lib.tkh_kv_planned_bytes(0, 1, 1, 0, 0, _lib.F32, 1, ctypes.byref(out),
                                    ctypes.byref(err)) == _lib.ZERO_DIMENSION
    assert lib.tkh_kv_planned_bytes(1, 1, 1, 1, 0, _lib.F32, 1, ctypes.byref(out),
                                    ctypes.byref(err)) == _lib.ZERO_DIMENSION
    assert lib.tkh_kv_planned_bytes(2 ** 40, 2 ** 20, 2 ** 10, 0, 0, _lib.F32, 1,
                                    ctypes.byref(out), ctypes.byref(err)) == _lib.SIZE_OVERFLOW
