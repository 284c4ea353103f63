"""The reference's Half staged-attention fixture sets on the CPU side:
staged-gqa-half-v1 (11 cases, src/metal/staged_gqa_fixture.rs:6-40) and
gemma3-staged-attention-v1 (8 cases, src/metal/staged_attention/tests.rs:9-60).

  * The physical input and after-commit arrays rebuilt from the fixtures'
    published recipe equal, word for word, the arrays the manifests hash.
  * The oracle's ring geometry (view start, old spans, copy runs;
    src/model/window_rows.rs:22-88) gives every case's recorded view and copy
    runs.

The device replay of the same cases is tests/test_gpu_staged_fixtures.py.
"""

import pytest

from goldens import Golden, staged_physical

FIXTURES = ("staged_gqa_half_v1", "gemma3_staged_attention_v1")


@pytest.mark.parametrize("fixture", FIXTURES)
def test_rebuilt_physical_arrays_match_manifest_hashes(fixture):
    g = Golden(fixture)
    assert len(g.meta["cases"]) == {"staged_gqa_half_v1": 11, "gemma3_staged_attention_v1": 8}[fixture]
    for case in g.meta["cases"]:
        arrays = staged_physical(g, fixture, case)  # asserts every SHA-256
        assert set(arrays) == set(case["input_sha256"])


@pytest.mark.parametrize("fixture", FIXTURES)
def test_views_and_copy_runs_match_oracle_ring_geometry(orc, fixture):
    g = Golden(fixture)
    for case in g.meta["cases"]:
        window = case["window"]
        retention = window or case["capacity"]
        committed, n = case["committed"], case["tokens"]
        view = case["view"]
        assert view["retention"] == retention
        assert orc.view_start(committed, window) == view["start"]
        spans = [(p, s, r) for p, s, r in orc.old_spans(retention, committed, window) if r]
        assert spans == [(s["absolute_start"], s["slot"], s["rows"]) for s in view["old_spans"]]
        runs = [(src, dst, r) for src, dst, r in orc.copy_runs(retention, committed, n, window is not None)
                if r]
        assert runs == [(r["source_row"], r["destination_row"], r["rows"]) for r in case["copy_runs"]]
