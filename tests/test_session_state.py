"""Session state machine (tkh_session) against the reference's transition tests.

A host-only session (no device context) runs the token state machine alone:
evaluation commits state and computes nothing.  The expected values are the
ones src/session.rs's tests assert (tests/session.rs:343-502), with
`logits().is_some()` read as `distribution_valid()`.
"""

import pytest

from toklet_amd import _lib
from toklet_amd.ops import TkhError
from toklet_amd.session import Options, Session

BASE = [1, 7, 13, 3, 47, 11]


def host_session(capacity, chunk, offset=0, vocab=64):
    return Session(None, Options(capacity=capacity, prefill_chunk_size=chunk,
                                 position_offset=offset, vocab_size=vocab, layers=1,
                                 query_heads=4, kv_heads=2, head_dim=8))


def test_reusable_prefix_edits_and_shortening_match_reference_table():
    """tests/session.rs:343-380: (tokens, kept prefix) after a fully evaluated BASE."""
    for offset in (0, 5):
        s = host_session(27, 3, offset)
        for tokens, keep in [(BASE, 6), ([1, 7, 13, 3, 47, 12], 5), ([1, 8, 13, 3], 1),
                             ([2, 7, 13], 0), (BASE[:4], 3), (BASE[:1], 0), ([], 0)]:
            s.reset()
            s.set_tokens(BASE)
            s.evaluate(None)
            s.set_tokens(tokens)
            assert s.evaluated_len() == keep, (tokens, keep)
            assert s.history() == tokens
            if keep < len(tokens):
                assert not s.distribution_valid()
            s.evaluate(None)
            assert s.evaluated_len() == len(tokens)
            assert s.distribution_valid() == (len(tokens) > 0)


def test_pending_sampled_token_is_not_committed_kv():
    """tests/session.rs:381-408."""
    s = host_session(27, 3)
    for pending in (47, 48):
        s.reset()
        s.set_tokens(BASE)
        s.evaluate(None)
        s.append([47])
        s.set_tokens(BASE + [pending])
        assert (s.evaluated_len(), s.pending_len()) == (6, 1)
        s.evaluate(None)
        assert s.distribution_valid()
    s.reset()
    s.set_tokens(BASE)
    s.evaluate(None)
    s.append([47])
    s.set_tokens(BASE)
    assert (s.evaluated_len(), s.pending_len()) == (6, 0)
    assert s.distribution_valid()


def test_cancelled_edit_discard_stages_one_replay_token():
    """tests/session.rs:405-450: discard after an edited request replays one token."""
    s = host_session(27, 3)
    s.set_tokens(BASE)
    s.evaluate(None)
    s.set_tokens([1, 7, 13, 3, 47, 12])
    assert s.evaluated_len() == 5
    assert not s.distribution_valid()
    s.discard_pending()
    assert s.history() == BASE[:5]
    assert (s.evaluated_len(), s.pending_len()) == (4, 1)
    assert not s.distribution_valid()
    s.discard_pending()
    assert s.history() == BASE[:5]
    assert (s.evaluated_len(), s.pending_len()) == (4, 1)
    s.append([12, 13])
    s.discard_pending()
    s.discard_pending()
    assert s.history() == BASE[:5]
    assert (s.evaluated_len(), s.pending_len()) == (4, 1)
    s.set_tokens(s.history())
    s.discard_pending()
    assert s.history() == BASE[:5]
    assert (s.evaluated_len(), s.pending_len()) == (4, 1)
    s.evaluate(None)
    assert s.distribution_valid() and s.evaluated_len() == 5
    # A fully cached request at the truncated boundary still needs its replay.
    s.set_tokens([1, 7, 13, 3, 48])
    assert s.evaluated_len() == 4
    s.set_tokens(BASE[:4])
    assert (s.evaluated_len(), s.pending_len()) == (3, 1)
    s.discard_pending()
    s.discard_pending()
    assert s.history() == BASE[:4]
    assert (s.evaluated_len(), s.pending_len()) == (3, 1)
    s.evaluate(None)
    assert s.distribution_valid()


def test_chunk_boundaries_cached_prompt_and_reset():
    """tests/session.rs:455-502 (options(32, 2, 0))."""
    s = host_session(32, 2)
    s.set_tokens([1, 7, 13, 3])
    assert s.next_chunk() == (0, 2)
    assert s.evaluate_next_chunk(None) == 2
    assert (s.evaluated_len(), s.pending_len()) == (2, 2)
    s.evaluate(None)
    assert s.distribution_valid()
    s.set_tokens([1, 7, 13, 3])
    assert s.evaluated_len() == 4
    assert s.evaluate_next_chunk(None) == 0
    assert s.distribution_valid()
    s.set_tokens([1, 7, 13, 3, 47, 11])
    assert s.evaluated_len() == 4
    s.discard_pending()
    assert s.distribution_valid() and s.history() == [1, 7, 13, 3]
    s.set_tokens([1, 7, 13, 17])
    assert s.evaluated_len() == 3
    assert not s.distribution_valid()
    s.evaluate(None)
    s.set_tokens([1, 7])
    assert s.evaluated_len() == 1
    s.evaluate(None)
    s.reset()
    assert s.history() == [] and not s.distribution_valid()
    assert s.evaluate_next_chunk(None) == 0
    s.set_tokens([11])
    s.evaluate(None)
    assert s.distribution_valid()
    s.set_tokens([])
    assert not s.distribution_valid()


def test_requests_are_admitted_before_mutation():
    """tests/session.rs:504-583: capacity and vocabulary errors change nothing."""
    s = host_session(4, 2, vocab=64)
    s.set_tokens([1, 2, 3])
    s.evaluate(None)
    before = (s.history(), s.evaluated_len(), s.distribution_valid())
    with pytest.raises(TkhError) as e:
        s.set_tokens([64])
    assert e.value.code == _lib.TOKEN and e.value.index == 0
    with pytest.raises(TkhError) as e:
        s.set_tokens([1, 2, 3, 4, 5])
    assert e.value.code == _lib.CAPACITY
    with pytest.raises(TkhError) as e:
        s.append([5, 6])
    assert e.value.code == _lib.CAPACITY
    with pytest.raises(TkhError) as e:
        s.append([64])
    assert e.value.code == _lib.TOKEN and e.value.index == 3
    assert (s.history(), s.evaluated_len(), s.distribution_valid()) == before


def test_evaluate_with_chunk_limit_walks_decode_steps():
    """Teacher-forced decode: pending tokens evaluated one position at a time."""
    s = host_session(16, 8)
    s.set_tokens(list(range(1, 11)))
    assert s.evaluate(None) == 10 and s.evaluated_len() == 10
    s.append([5, 6, 7])
    assert s.next_chunk() == (10, 3)
    assert s.evaluate(None, chunk_limit=1) == 3
    assert (s.evaluated_len(), s.pending_len()) == (13, 0)


def test_invalid_options_are_rejected():
    with pytest.raises(TkhError) as e:
        Session(None, Options(capacity=0))
    assert e.value.code == _lib.ZERO_DIMENSION
    with pytest.raises(TkhError) as e:
        Session(None, Options(capacity=8, query_heads=6, kv_heads=4))
    assert e.value.code == _lib.INVALID_PARAMETER
    with pytest.raises(TkhError):
        Session(None, Options(capacity=8, layers=2, layer_windows=[4, 0]))  # needs a score scale
    with pytest.raises(TkhError) as e:  # attention_cached semantics have no softcap
        Session(None, Options(capacity=8, softcap=50.0))
    assert e.value.code == _lib.INVALID_CONFIG


def test_llama3_rotary_options_are_validated():
    """Llama3Scaling::new's rules (src/cpu/llama3_rotary.rs:14-37, tests.rs:207-221)
    hold for the session's rotary options: factor >= 1, low > 0, high > low, the
    original context length in 1..2^53, theta finite and positive."""
    from toklet_amd.ops import ROTARY_LLAMA3

    def opts(**kw):
        base = dict(capacity=8, query_heads=4, kv_heads=2, head_dim=8, rotary=ROTARY_LLAMA3,
                    theta=500000.0, factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0,
                    original_max_positions=8192)
        base.update(kw)
        return Options(**base)

    Session(None, opts()).close()
    Session(None, opts(factor=1.0)).close()
    nan, inf = float("nan"), float("inf")
    bad = [dict(factor=v) for v in (0.0, -1.0, 0.5, nan, inf)]
    bad += [dict(low_freq_factor=v) for v in (0.0, -1.0, nan, inf)]
    bad += [dict(high_freq_factor=v) for v in (0.0, -1.0, nan, inf)]
    bad += [dict(low_freq_factor=4.0), dict(low_freq_factor=5.0), dict(original_max_positions=0),
            dict(original_max_positions=(1 << 53) + 1), dict(theta=0.0), dict(theta=nan)]
    for kw in bad:
        with pytest.raises(TkhError) as e:
            Session(None, opts(**kw))
        assert e.value.code == _lib.INVALID_PARAMETER, kw
    with pytest.raises(TkhError) as e:
        Session(None, opts(rotary=4))
    assert e.value.code == _lib.INVALID_PARAMETER


def _shared_fixture():
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemma_shared_kv_v1.json")
    return json.load(open(path))


def test_shared_kv_routing_matches_gemma_shared_kv_fixture():
    """Every case of gemma-shared-kv-v1 (35 layers with 20 shared, alternating, no
    sharing, irregular kinds): each layer's KV producer is the fixture's
    (SharedKvPlan::new / producer_for, src/model/shared_kv.rs:50-146), the KV bytes
    count the owners only, and the chunk steps commit as the fixture's do."""
    data = _shared_fixture()
    assert len(data["cases"]) == 4
    for case in data["cases"]:
        kinds, W = case["kinds"], case["window"]
        total = sum(case["chunks"])
        windows = [W if k == "S" else 0 for k in kinds]
        s = Session(None, Options(capacity=max(total, W), prefill_chunk_size=max(case["chunks"]),
                                  vocab_size=64, layers=len(kinds), query_heads=2, kv_heads=1,
                                  head_dim=8, score_scale=0.125, layer_windows=windows,
                                  shared_layers=case["shared"]))
        assert [s.kv_producer(l) for l in range(len(kinds))] == case["producer_map"], case["name"]
        producers = len(kinds) - case["shared"]
        for step in case["steps"]:
            for layer, producer, key_start, key_end, produces in step["layers"]:
                assert s.kv_producer(layer) == producer
                assert bool(produces) == (layer < producers)
                assert key_end == step["after"]
                w = W if kinds[layer] == "S" else None
                assert key_start == (max(0, step["before"] - w + 1) if w else 0)
        for step in case["steps"]:
            s.append([1] * step["count"])
            assert s.next_chunk() == (step["before"], step["count"])
            assert s.evaluate(None) == step["count"]
            assert s.evaluated_len() == step["after"]
        with pytest.raises(IndexError):
            s.kv_producer(len(kinds))
        s.close()


def test_shared_kv_routing_rejections():
    """SharedKvPlan::new's refusals (src/model/shared_kv.rs:57-87): no producer left,
    no earlier owner of the shared layer's kind, a different window."""
    def opts(windows, shared):
        return Options(capacity=16, layers=len(windows), query_heads=2, kv_heads=1, head_dim=8,
                       score_scale=0.125, layer_windows=windows, shared_layers=shared)

    for windows, shared in [([3, 0], 2), ([3, 0], 3), ([3, 3], 1 << 40)]:
        with pytest.raises(TkhError) as e:
            Session(None, opts(windows, shared))
        assert e.value.code == _lib.INVALID_CONFIG
    for windows, shared in [([3, 0], 1), ([3, 3, 0], 1), ([3, 4], 1), ([0, 3, 0, 5], 1)]:
        with pytest.raises(TkhError) as e:
            Session(None, opts(windows, shared))
        assert e.value.code == _lib.INVALID_CONFIG, (windows, shared)
    s = Session(None, opts([3, 0, 3, 0], 2))
    assert [s.kv_producer(l) for l in range(4)] == [0, 1, 0, 1]
    s.close()


def test_layer_by_layer_chunks_follow_the_whole_chunk_state_machine():
    """tkh_session_chunk_*: layers in order, the commit after the last layer commits
    the chunk as Session::evaluate_chunk does (src/session.rs:364-418); out-of-order
    layers are refused without dropping the chunk; an early commit, an abort or a
    state edit drops it and commits nothing."""
    s = Session(None, Options(capacity=32, prefill_chunk_size=4, vocab_size=64, layers=3,
                              query_heads=4, kv_heads=2, head_dim=8))
    s.set_tokens(list(range(1, 11)))
    assert s.chunk_begin() == (0, 4)
    s.chunk_layer(0, None)
    with pytest.raises(TkhError) as e:
        s.chunk_layer(2, None)
    assert e.value.code == _lib.INVALID_CONFIG
    s.chunk_layer(1, None)
    with pytest.raises(TkhError) as e:
        s.chunk_commit()  # two of three layers: dropped
    assert e.value.code == _lib.INVALID_CONFIG
    assert s.evaluated_len() == 0
    with pytest.raises(TkhError):
        s.chunk_layer(2, None)  # no chunk any more
    assert s.chunk_begin() == (0, 4)
    for layer in range(3):
        s.chunk_layer(layer, None)
    assert s.chunk_commit() == 4
    assert (s.evaluated_len(), s.pending_len()) == (4, 6)
    assert s.chunk_begin(chunk_limit=1) == (4, 1)
    s.chunk_layer(0, None)
    s.chunk_abort()
    with pytest.raises(TkhError):
        s.chunk_commit()
    assert s.evaluated_len() == 4
    assert s.chunk_begin(chunk_limit=2) == (4, 2)
    s.chunk_layer(0, None)
    s.set_tokens(list(range(1, 9)))  # a state edit drops the chunk
    with pytest.raises(TkhError):
        s.chunk_layer(1, None)
    assert s.evaluate(None) == 4 and s.evaluated_len() == 8
    assert s.chunk_begin() == (8, 0)
    with pytest.raises(TkhError):
        s.chunk_commit()
    assert s.distribution_valid() and s.pending_len() == 0
    s.close()
