"""The library's CPU-only host paths built with AddressSanitizer and
UndefinedBehaviorSanitizer (tests/asan/, built by __graft_entry__.build()):
weight-file header validation on valid, truncated and corrupted files, the
seeded init, the model.h host API with a file round trip, and the error
paths of entry points called without a device or with bad arguments. Any
sanitizer report aborts the binary."""
import os
import subprocess

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "asan", "check_host_asan")


def test_host_paths_under_asan_and_ubsan():
    assert os.path.exists(BIN), "tests/asan not built (run __graft_entry__.build())"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
    assert "0 failed" in r.stdout
