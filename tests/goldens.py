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
