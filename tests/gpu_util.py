"""Helpers shared by the GPU parity tests (seeded inputs, dtype rounding, oracle calls)."""

from __future__ import annotations

import sys

import numpy as np

TOL_HALF = 2e-3   # max abs error for bf16/f16 K/V (and Q stored in the same dtype)
TOL_F32 = 1e-5    # max abs error for the FP32 path


def log(msg: str):
    print(msg, flush=True)
    sys.stdout.flush()


def torch_dtype(name: str):
    import torch

    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[name]


def stored(a: np.ndarray, name: str) -> np.ndarray:
    """The FP32 widening of `a` after rounding to the storage dtype (what the kernels read)."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(torch_dtype(name)).to(torch.float32).numpy()


def dev(a: np.ndarray, name: str):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(torch_dtype(name))


def host(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def max_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    assert np.all(np.isfinite(a)), "non-finite device output"
    return float(np.abs(a - b).max()) if a.size else 0.0


def head_major_cache(rows_tok_major: np.ndarray, kv_heads: int, capacity: int, dims: int,
                     fill=np.nan) -> np.ndarray:
    """[tokens, Hkv, D] -> [Hkv, capacity, D] with `fill` in the unused tail."""
    tokens = rows_tok_major.shape[0]
    out = np.full((kv_heads, capacity, dims), fill, np.float32)
    out[:, :tokens] = rows_tok_major.reshape(tokens, kv_heads, dims).transpose(1, 0, 2)
    return out


def greedy_tokens(context: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """Lowest-index argmax of context @ weight.T per row (src/sampling.rs:5-18)."""
    logits = context.astype(np.float32) @ weight.T.astype(np.float32)
    return np.argmax(logits, axis=1)


def assert_tokens_agree(got: np.ndarray, ref: np.ndarray, weight: np.ndarray, max_ties: float = 0.01):
    """Greedy tokens of the GPU context against the oracle's.  A row may differ only
    where the oracle's two candidates are tied at the precision the contexts agree
    to: for tokens a (oracle) and b (GPU), |logit_a - logit_b| <= sum_d |W_a - W_b| * err,
    err the row's max abs context difference.  Such ties must stay rare: at most one
    row or `max_ties` of the rows, whichever is larger.  Returns the number of ties."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    w = weight.astype(np.float64)
    ta, tb = greedy_tokens(ref, weight), greedy_tokens(got, weight)
    ties = 0
    for r in np.nonzero(ta != tb)[0]:
        a, b = ta[r], tb[r]
        err = np.abs(got[r] - ref[r]).max()
        gap = abs(ref[r] @ w[a] - ref[r] @ w[b])
        bound = np.abs(w[a] - w[b]).sum() * err
        assert gap <= bound, f"row {r}: token {b} instead of {a}, logit gap {gap:.3e} > {bound:.3e}"
        ties += 1
    assert ties <= max(1, int(max_ties * len(ta))), f"{ties} of {len(ta)} rows changed token"
    return ties


def assert_tokens_identical(got: np.ndarray, ref: np.ndarray, weight: np.ndarray):
    """Greedy tokens of the GPU context equal the oracle's on every row (the
    north star's "argmax-identical next tokens"), with no allowance for ties."""
    ta, tb = greedy_tokens(ref, weight), greedy_tokens(got, weight)
    rows = np.nonzero(ta != tb)[0]
    assert rows.size == 0, (f"{rows.size} of {len(ta)} rows changed token "
                            f"(first rows {rows[:8].tolist()})")
