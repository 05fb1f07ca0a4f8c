"""Runs the C mirror of the reference's tests/check_fast.c (tests/c/), which
drives the fast.h drop-in from a C host exactly as the reference's callers do."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

CDIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c")


def _run(name):
    path = os.path.join(CDIR, name)
    assert os.path.exists(path), f"tests/c/{name} not built (run __graft_entry__.build())"
    r = subprocess.run([path], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    assert "0 failed" in r.stdout


def test_check_fast_hip_binary():
    _run("check_fast_hip")


def test_reference_layout_fastctx():
    """The library driven through the reference's 80-byte FastCtx
    (src/fast.h:35-45), guard bytes on both sides."""
    _run("check_refctx")


def test_training_step_from_c():
    """cngpt_hip_train_* in the reference's training-loop order from a C
    host (src/cngpt.c:150-165), against the oracle's step."""
    _run("check_train_hip")

