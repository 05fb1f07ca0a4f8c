"""The `cngpt` command (cngpt_amd/csrc/cngpt_cli.c) without a GPU: the
host-only sub-command and the error exits of the reference's CLI
(src/cngpt.c:440-454)."""
import os
import subprocess

import numpy as np
import pytest

import cngpt_amd
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cngpt_amd", "cngpt")


def run(*args):
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=120)


def test_create_tiny_matches_seeded_init(tmp_path):
    """create-tiny: 2L/4H/32C/V64/T8 after srand(seed) (src/cngpt.c:372-398)."""
    out = tmp_path / "tiny.bin"
    r = run("create-tiny", f"--out={out}", "--seed=99")
    assert r.returncode == 0, r.stderr
    assert "27776 params" in r.stdout
    cfg, params = cngpt_amd.load_weights(str(out))
    assert cfg == cngpt_amd.Config(2, 4, 32, 64, 8)
    ref = oracle.init_weights(oracle.Cfg(2, 4, 32, 64, 8), 99)
    assert np.array_equal(params, ref)
    # the space-separated flag form of arg_get (src/cngpt.c:35-50)
    out2 = tmp_path / "tiny2.bin"
    assert run("create-tiny", "--out", str(out2), "--seed", "99").returncode == 0
    assert out.read_bytes() == out2.read_bytes()


def test_usage_and_errors(tmp_path):
    r = run()
    assert r.returncode == 1 and "Usage" in r.stderr
    assert run("frobnicate").returncode == 1
    assert run("train", "--data=x").returncode == 1
    r = run("sample")
    assert r.returncode == 1 and "--weights is required" in r.stderr
    r = run("bench")
    assert r.returncode == 1 and "--weights is required" in r.stderr
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"\0" * 64)
    r = run("bench", f"--weights={bad}")
    assert r.returncode == 1 and "not a cngpt weight file" in r.stderr
    # sample validates the file header before it touches a device
    r = run("sample", f"--weights={bad}")
    assert r.returncode == 1 and "not a cngpt weight file" in r.stderr
    r = run("sample", f"--weights={tmp_path / 'missing.bin'}")
    assert r.returncode == 1 and "No such file" in r.stderr


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device path")
def test_sample_without_device_fails_cleanly(tmp_path):
    out = tmp_path / "tiny.bin"
    assert run("create-tiny", f"--out={out}").returncode == 0
    r = run("sample", f"--weights={out}", "--tokens=3", "--seed=1")
    assert r.returncode == 1
    assert "device" in r.stderr
