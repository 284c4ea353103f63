"""The reference's allocation-free steady state (tests/session.rs:715-744,
admitted_prefill_decode_and_reuse_allocate_no_buffers): after
tkh_session_create, prefill, re-prefill of a cached prompt, eight decode steps,
a discarded append, a shortened prompt, reset and a new prompt allocate no
host memory in the library and leave the device's free memory and the
session's memory accounting unchanged, on a synchronous and on a queued
context.

tests/native/session_allocations (built by __graft_entry__.build) runs the
sequence in a fresh process: it interposes malloc/calloc/realloc and operator
new and counts the calls made from libtokhip's code.
"""

import os
import subprocess

import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROGRAM = os.path.join(HERE, "native", "session_allocations")


def test_session_steady_state_allocates_nothing():
    assert os.path.exists(PROGRAM), "tests/native/session_allocations is not built (tests/native/build.py)"
    res = subprocess.run([PROGRAM], capture_output=True, text=True, timeout=120)
    for line in res.stdout.splitlines():
        log(line)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "OK: no allocation in the steady state" in res.stdout
