"""Loaders for the frozen reference vectors under tests/golden/ (data only)."""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class Golden:
    def __init__(self, name: str):
        self.meta = json.load(open(os.path.join(GOLDEN, name + ".json")))
        self.arrays = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)

    def __getitem__(self, key):
        if isinstance(key, dict):
            key = key["array"]
        return self.arrays[key]


def close(actual, expected, atol=1e-5, rtol=1e-4):
    """The reference's per-operation gate |a-e| <= atol + rtol*|e| (tests/cpu_attention.rs:6-14)."""
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.all(np.isfinite(a)), "non-finite output"
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    assert not bad.any(), f"{bad.sum()} mismatches, first at {np.argmax(bad)}: {a[bad][:4]} vs {e[bad][:4]}"


def head_major_to_token_major(x, heads, tokens, dims):
    """[heads, tokens, D] -> [tokens, heads, D] (the fixtures' q/output layout)."""
    return np.asarray(x).reshape(heads, tokens, dims).transpose(1, 0, 2).reshape(-1)


TINY_CASES = ["prompt", "future_changed", "offset", "single", "capacity"]


# ---- gemma-reference-attention-v1 inputs ----

# The fixture's published input recipe ("rational13-and-cancellation-near-ties-v1",
# tools/reference/gemma_reference_attention_oracle.py:29-35): rationals n/13 from a
# modular walk over (head, position, feature), and for `cancellation` mixed-sign
# dyadic rows with near-tied keys.

def _cancellation_value(kind: str, position: int, feature: int) -> float:
    if kind == "q":
        return (1024.0, 1.0, -1024.0, -1.0)[feature % 4]
    if kind == "k":
        return 1.0 + (position % 2) * 2.0 ** -20 + ((position % 7) * 2.0 ** -24 if feature % 4 == 1 else 0.0)
    return (0.0 if position == 512 else (1024.0, 1.0, -1024.0, -1.0)[position % 4]) + (feature % 7) * 2.0 ** -8


def reference_attention_inputs(golden: "Golden", case: dict, contract: str):
    """q [1, heads, queries, D], k/v [1, 1, keys, D] of one case and contract
    ("math": FP64, "staged_fp32": FP32), rebuilt from the recipe and checked
    byte for byte against the SHA-256 the fixture's manifest records."""
    out = []
    for name in ("q", "k", "v"):
        item = next(i for i in golden.meta["inputs"]
                    if (i["case"], i["contract"], i["name"]) == (case["name"], contract, name))
        origin = case["query_start"] if name == "q" else case["key_start"]
        heads = case["heads"] if name == "q" else 1
        n = case["queries"] if name == "q" else case["keys"]
        d = case["head_dim"]
        h, p, f = np.meshgrid(np.arange(heads), np.arange(n), np.arange(d), indexing="ij")
        if case["name"] == "cancellation":
            values = np.array([_cancellation_value(name, origin + pp, ff)
                               for pp, ff in zip(p.ravel(), f.ravel())])
        else:
            shift = {"q": 3, "k": 11, "v": 23}[name]
            values = (((h * 31 + (origin + p) * 17 + f * 7 + shift) % 53) - 26) / 13.0
        values = np.asarray(values, dtype=item["dtype"]).reshape(item["shape"])
        digest = hashlib.sha256(np.ascontiguousarray(values).tobytes()).hexdigest()
        assert digest == item["sha256"], f"rebuilt {case['name']}/{contract}/{name} differs"
        out.append(values)
    return out


# ---- staged-gqa-half-v1 and gemma3-staged-attention-v1 physical inputs ----

# The fixtures' published seeded recipe (tools/reference/staged_gqa_half.py:75-110 and
# tools/reference/gemma3_staged_attention.py:93-133): Half rows of small dyadic
# rationals from modular walks over (position, head, feature), laid out as the
# staged kernels' physical buffers -- old rows [kv, retention, D] at their ring or
# linear slots, staged rows [kv, 32, D] (head stride 32 whatever the chunk), Q
# [32, Hq, D] -- with every unwritten word, and a 7-word guard, holding the pad
# word.  Rebuilt here and checked word for word against the SHA-256 each
# manifest records for the arrays.

STAGED_CHUNK = 32


def _half_words(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float64).astype(np.float16).view(np.uint16)


def _staged_row(fixture: str, case: dict, position: int, head: int, kind: str) -> np.ndarray:
    d = case["dim"]
    f = np.arange(d)
    if fixture == "staged_gqa_half_v1":
        if kind == "k":
            values = ((position * 5 + head * 7 + f * 3 + 1) % 17 - 8) / 32
        else:
            values = ((position * 11 + head * 13 + f * 5 + 7) % 31 - 15) / 16
        words = _half_words(values)
        if case["name"] == "tiny_single" and kind == "v" and position == 0:
            words[0] = 0x0001 if head == 0 else 0x8001
        return words
    if kind == "v" and case["pattern"] == "uniform":
        values = np.zeros(d)
        for feature, key in enumerate((0, 1, 512, 513)):
            if position == key:
                values[feature] = 512.0
        return _half_words(values)
    modulus, divisor, shift = (17, 32, 1) if kind == "k" else (19, 16, 7)
    return _half_words(((position * 5 + f * 3 + shift) % modulus - modulus // 2) / divisor)


def staged_physical(golden: "Golden", fixture: str, case: dict) -> dict:
    """The physical u16 arrays of one case: q, old_k/old_v, new_k/new_v and the
    expected after-commit expected_after_k/_v, each with its guard, each checked
    against the manifest's SHA-256."""
    guard, pad = golden.meta["guard"], golden.meta["pad"]
    d, n, committed = case["dim"], case["tokens"], case["committed"]
    window = case["window"]
    retention = window or case["capacity"]
    qh, kv = case["query_heads"], case["kv_heads"]
    out = {}
    old = {}
    for kind in ("k", "v"):
        words = np.full(kv * retention * d + guard, pad, np.uint16)
        first = max(0, committed - retention) if window else 0
        for head in range(kv):
            for position in range(first, committed):
                slot = position % retention if window else position
                words[(head * retention + slot) * d:(head * retention + slot + 1) * d] = \
                    _staged_row(fixture, case, position, head, kind)
        old[kind] = words
        staged = np.full(kv * STAGED_CHUNK * d + guard, pad, np.uint16)
        for head in range(kv):
            for token in range(n):
                off = (head * STAGED_CHUNK + token) * d
                staged[off:off + d] = _staged_row(fixture, case, committed + token, head, kind)
        out["old_" + kind] = words
        out["new_" + kind] = staged
        after = words.copy()
        for head in range(kv):
            for run in case["copy_runs"]:
                src = (head * STAGED_CHUNK + run["source_row"]) * d
                dst = (head * retention + run["destination_row"]) * d
                after[dst:dst + run["rows"] * d] = staged[src:src + run["rows"] * d]
        out["expected_after_" + kind] = after
    q = np.full(STAGED_CHUNK * qh * d + guard, pad, np.uint16)
    f = np.arange(d)
    for token in range(n):
        for head in range(qh):
            if case.get("pattern") == "uniform":
                values = np.zeros(d)
            else:
                values = ((7 * (committed + token) + 5 * head + 3 * f) % 13 - 6) / 32
            q[(token * qh + head) * d:(token * qh + head + 1) * d] = _half_words(values)
    out["q"] = q
    for name, words in out.items():
        want = case["input_sha256"][name]
        assert words.size == want["words"], (case["name"], name)
        digest = hashlib.sha256(words.astype("<u2").tobytes()).hexdigest()
        assert digest == want["sha256"], f"rebuilt {case['name']}/{name} differs"
    return out
