"""cngpt_hip_forward_noalloc (the forward that allocates nothing: its
activations live in the library's per-device scratch array) against the
existing entry point cngpt_hip_forward_resident on the same handle.

Same kernels in the same order, so the logits must be bitwise equal; two
calls in a row, the second smaller (the scratch keeps the first call's
contents), in both modes; sizes beyond the scratch are refused; token ids
outside the vocabulary are clamped and flagged in the caller's error word.
Device buffers here are the test's own (hipMalloc through ctypes).
"""
import ctypes

import numpy as np
import pytest

import cngpt_amd
from test_parity_gpu import randomize, say

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


@pytest.fixture(scope="module")
def hip():
    h = ctypes.CDLL("libamdhip64.so.7")
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipFree.argtypes = [ctypes.c_void_p]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    for f in (h.hipMalloc, h.hipFree, h.hipMemcpy):
        f.restype = ctypes.c_int
    return h


class DevBuf:
    def __init__(self, hip, nbytes):
        self.hip, self.ptr = hip, ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.ptr), nbytes) == 0
        self.nbytes = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        assert self.hip.hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D) == 0

    def get(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        assert self.hip.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        self.hip.hipFree(self.ptr)


def reference(m, tokens, mode):
    """cngpt_hip_forward_resident on the handle's own arena."""
    B, T = tokens.shape
    V = m.cfg.vocab_size
    m.reserve(B, T, mode)
    m.upload_tokens(tokens)
    m.forward_resident(B, T, mode)
    m.synchronize()
    n = B * V if mode == cngpt_amd.LAST else B * T * V
    return m.read_logits(0, n)


def test_forward_noalloc_matches_forward_resident(hip):
    cfg = cngpt_amd.Config(2, 12, 768, 50257, 1024)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 31), 32)
    V = cfg.vocab_size
    rng = np.random.default_rng(33)
    tok_dev = DevBuf(hip, 4 * 1024 * 4)
    logit_dev = DevBuf(hip, 4 * 300 * V * 4)
    err_dev = DevBuf(hip, 4)
    try:
        with cngpt_amd.Model(cfg, params) as m:
            # 2 x 800 rows of width 768 take about 29.2 M of the scratch's 33.5 M
            # floats (16.8 M of them the split-K partials)
            for mode, shapes in ((cngpt_amd.LAST, [(2, 800), (1, 37)]),
                                 (cngpt_amd.ALL, [(1, 300), (2, 5)])):
                for B, T in shapes:  # the second call is smaller
                    say(f"noalloc mode={mode} B={B} T={T}")
                    tokens = rng.integers(0, V, size=(B, T), dtype=np.int32)
                    tok_dev.put(tokens)
                    err_dev.put(np.array([7], np.int32))  # the call zeroes it
                    m.forward_noalloc(tok_dev.ptr.value, B, T, mode, logit_dev.ptr.value,
                                      err_dev.ptr.value)
                    m.synchronize()
                    n = B * V if mode == cngpt_amd.LAST else B * T * V
                    got = logit_dev.get(n, np.float32)
                    assert err_dev.get(1, np.int32)[0] == 0
                    ref = reference(m, tokens, mode)
                    assert np.isfinite(got).all()
                    assert np.array_equal(got, ref), float(np.abs(got - ref).max())
            # beyond the scratch: refused with a message, nothing enqueued
            with pytest.raises(cngpt_amd.CngptError, match="scratch"):
                m.forward_noalloc(tok_dev.ptr.value, 3, 1024, cngpt_amd.LAST,
                                  logit_dev.ptr.value, None)
            # a token id outside [0, V) is clamped and flagged
            tokens = rng.integers(0, V, size=(1, 8), dtype=np.int32)
            tokens[0, 3] = V + 5
            tok_dev.put(tokens)
            m.forward_noalloc(tok_dev.ptr.value, 1, 8, cngpt_amd.LAST, logit_dev.ptr.value,
                              err_dev.ptr.value)
            m.synchronize()
            assert err_dev.get(1, np.int32)[0] & 1
    finally:
        for b in (tok_dev, logit_dev, err_dev):
            b.free()


def test_forward_noalloc_split_attention_on_a_small_handle(hip):
    """GPT-2 small's 12 heads, final-position mode, B=16 T=64: the last
    layer's 192 (sequence, head) pairs take the decode attention split over
    two workgroups per pair, whose tagged words and counters the no-alloc
    forward keeps in the scratch, while the handle's own arena is reserved
    for two sequences only. Two calls in a row (the counters go on from the
    first), each bitwise equal to the resident forward on a handle then
    reserved for all 16."""
    cfg = cngpt_amd.Config(2, 12, 768, 50257, 1024)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 41), 42)
    V = cfg.vocab_size
    B, T = 16, 64
    tokens = np.random.default_rng(43).integers(0, V, size=(B, T), dtype=np.int32)
    tok_dev = DevBuf(hip, tokens.nbytes)
    logit_dev = DevBuf(hip, B * V * 4)
    err_dev = DevBuf(hip, 4)
    try:
        with cngpt_amd.Model(cfg, params) as m:
            m.reserve(2, T, cngpt_amd.LAST)
            tok_dev.put(tokens)
            got = []
            for _ in range(2):
                say(f"noalloc split attention B={B} T={T} on a handle reserved for B=2")
                m.forward_noalloc(tok_dev.ptr.value, B, T, cngpt_amd.LAST, logit_dev.ptr.value,
                                  err_dev.ptr.value)
                m.synchronize()
                assert err_dev.get(1, np.int32)[0] == 0
                got.append(logit_dev.get(B * V, np.float32))
            ref = reference(m, tokens, cngpt_amd.LAST)
        for g in got:
            assert np.isfinite(g).all()
            assert np.array_equal(g, ref), float(np.abs(g - ref).max())
    finally:
        for b in (tok_dev, logit_dev, err_dev):
            b.free()


def test_forward_noalloc_capacity_boundary(hip):
    """The largest T the scratch takes at B=3 (found by halving the range
    between an accepted and a refused length; a refusal enqueues nothing)
    runs and matches the resident forward bitwise; one more position is
    refused with a message."""
    cfg = cngpt_amd.Config(2, 12, 768, 50257, 1024)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 51), 52)
    V = cfg.vocab_size
    B = 3
    rng = np.random.default_rng(53)
    tok_dev = DevBuf(hip, B * 1024 * 4)
    logit_dev = DevBuf(hip, B * V * 4)
    try:
        with cngpt_amd.Model(cfg, params) as m:
            tok_dev.put(rng.integers(0, V, size=(B, 1024), dtype=np.int32))

            def accepted(T):
                try:
                    m.forward_noalloc(tok_dev.ptr.value, B, T, cngpt_amd.LAST,
                                      logit_dev.ptr.value, None)
                except cngpt_amd.CngptError as e:
                    assert "scratch" in str(e)
                    return False
                m.synchronize()
                return True

            lo, hi = 1, 1024
            assert accepted(lo) and not accepted(hi)
            while hi - lo > 1:
                mid = (lo + hi) // 2
                if accepted(mid):
                    lo = mid
                else:
                    hi = mid
            say(f"noalloc capacity at B={B}: T={lo} accepted, T={lo + 1} refused")
            assert lo > 500
            tokens = rng.integers(0, V, size=(B, lo), dtype=np.int32)
            tok_dev.put(tokens)
            assert accepted(lo)
            got = logit_dev.get(B * V, np.float32)
            assert not accepted(lo + 1)
            ref = reference(m, tokens, cngpt_amd.LAST)
        assert np.isfinite(got).all()
        assert np.array_equal(got, ref), float(np.abs(got - ref).max())
    finally:
        for b in (tok_dev, logit_dev):
            b.free()
