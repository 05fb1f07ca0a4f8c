"""Runs the C mirror of the reference's tests/check_fast.c (tests/c/), which
drives the fast.h drop-in from a C host exactly as the reference's callers do."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "check_fast_hip")


def test_check_fast_hip_binary():
    assert os.path.exists(BIN), "tests/c/check_fast_hip not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "0 failed" in r.stdout
