"""Loaders for the frozen reference vectors under tests/golden/ (data only)."""

from __future__ import annotations

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
