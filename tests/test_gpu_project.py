"""GPU parity of the o-projection + greedy pick (tkh_project_greedy) against the
oracle's FP32 matmul (src/cpu/mod.rs:183-247) and greedy (src/sampling.rs:5-18).

The device forms each logit in the reference's own FP32 order, so logits are
compared bit for bit and tokens must be identical.
"""

import numpy as np
import pytest

from gpu_util import host, log

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


def _run(torch, ops, ctx, context, weights, want_logits=True):
    c = torch.from_numpy(np.ascontiguousarray(context, np.float32)).cuda()
    w = torch.from_numpy(np.ascontiguousarray(weights, np.float32)).cuda()
    rows, vocab = context.shape[0], weights.shape[0]
    tokens = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    logits = torch.full((rows, vocab), np.nan, dtype=torch.float32, device="cuda") if want_logits else None
    ops.project_greedy(ctx, c, w, tokens, logits)
    return tokens.cpu().numpy().view(np.uint32), \
        (host(logits) if want_logits else None)


def test_manual_projection_and_ties(torch_mod, ops, ctx, orc):
    from goldens import Golden

    torch = torch_mod
    g = Golden("tiny_v1_linear")
    x, w = g.arrays["manual.inputs"], g.arrays["manual.weight"]
    tokens, logits = _run(torch, ops, ctx, x, w)
    assert logits[0].tolist() == [-4.0, 15.0] and tokens.tolist() == [1, 1]
    # equal rows tie to the lowest id; +0 and -0 tie
    w = np.array([[1.0, 0.0], [2.0, 0.0], [2.0, 0.0], [0.5, 0.0]], np.float32)
    tokens, _ = _run(torch, ops, ctx, np.array([[3.0, 1.0], [-1.0, 0.0]], np.float32), w)
    assert tokens.tolist() == [1, 3]
    w = np.array([[-1.0], [1.0], [0.0]], np.float32)
    tokens, logits = _run(torch, ops, ctx, np.array([[0.0], [-0.0]], np.float32), w)
    assert tokens.tolist() == [0, 0]


def test_non_finite_inputs_are_reported(torch_mod, ops, ctx):
    torch = torch_mod
    rng = np.random.default_rng(7)
    for where in ("weight_nan", "weight_inf", "context_nan", "overflow"):
        c = rng.standard_normal((3, 70)).astype(np.float32)
        w = rng.standard_normal((300, 70)).astype(np.float32)
        if where == "weight_nan":
            w[123, 5] = np.nan
        elif where == "weight_inf":
            w[299, 69] = np.inf
        elif where == "context_nan":
            c[2, 0] = np.nan
        else:
            c[:] = 1e20
            w[:] = 1e20
        with pytest.raises(ops.TkhError) as e:
            _run(torch, ops, ctx, c, w)
        assert e.value.name == "NonFinite", where


@pytest.mark.parametrize("rows,hidden,vocab", [(1, 896, 3000), (1, 80, 1500), (1, 20, 257),
                                               (3, 70, 1025), (17, 257, 600), (40, 128, 513)])
def test_logits_bit_exact_and_tokens_identical(torch_mod, ops, ctx, orc, rows, hidden, vocab):
    """Every build of the kernel (1, 4 and 16 rows per workgroup; 16-byte and
    scalar weight loads; vocabularies that end inside a workgroup; several row
    blocks) against the oracle's matmul and greedy."""
    torch = torch_mod
    rng = np.random.default_rng(rows * 1000 + hidden)
    c = rng.standard_normal((rows, hidden)).astype(np.float32)
    w = rng.standard_normal((vocab, hidden)).astype(np.float32)
    tokens, logits = _run(torch, ops, ctx, c, w)
    ref = orc.matmul(c.reshape(-1), w, rows, hidden, vocab).reshape(rows, vocab)
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
    assert tokens.tolist() == [orc.greedy(ref[r]) for r in range(rows)]
    tokens2, _ = _run(torch, ops, ctx, c, w, want_logits=False)
    assert np.array_equal(tokens, tokens2)
    log(f"projection {rows}x{hidden} -> {vocab}: logits bit-exact, tokens {tokens[:4].tolist()}...")
