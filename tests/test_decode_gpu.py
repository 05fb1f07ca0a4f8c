"""Incremental decode with the device KV cache vs the oracle.

The reference has no KV cache: gpt_sample (src/model.c:991-1016) reruns the
whole prefix for each token. Without window truncation (prompt + steps <=
block_size) the logits of step i equal the last-position logits of a
forward over the first prompt+i tokens, which by causality are row
prompt+i-1 of one all-positions forward over the final sequence; that is
the reference value each step is compared with.
"""
import numpy as np
import pytest

import cngpt_amd
import oracle
from test_parity_gpu import compare, ocfg, randomize, say

pytestmark = pytest.mark.gpu


def test_greedy_decode_gpt2_small():
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    prompt = oracle.lcg_tokens(32, cfg.vocab_size).reshape(1, 32)
    steps = 64
    with cngpt_amd.Model(cfg, params) as m:
        logits = [m.decode_begin(prompt, capacity=32 + steps)]
        toks = [int(logits[0].argmax())]
        for _ in range(steps - 1):
            logits.append(m.decode_step(np.array([toks[-1]], np.int32)))
            toks.append(int(logits[-1].argmax()))
        assert m.decode_length() == 32 + steps - 1
    seq = np.concatenate([prompt[0], np.array(toks[:-1], np.int32)]).reshape(1, -1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[0, 31:]
    got = np.stack([l[0] for l in logits])
    say(f"decode small: {steps} steps")
    compare(got, ref, what="greedy decode")


def test_device_argmax_feed_matches_host_feed():
    cfg = cngpt_amd.Config(2, 4, 256, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 5), 6)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=(3, 17), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        first = m.decode_begin(prompt, capacity=60)
        host = [first]
        for _ in range(20):
            host.append(m.decode_step(host[-1].argmax(-1).astype(np.int32)))
        m.decode_begin(prompt, capacity=60)
        dev = [first]
        for _ in range(20):
            dev.append(m.decode_step(None))   # argmax taken on the device
        for a, b in zip(host, dev):
            assert np.array_equal(a, b)
        toks = np.stack([h.argmax(-1) for h in host[:-1]], axis=1).astype(np.int32)
    seq = np.concatenate([prompt, toks], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 16:]
    got = np.stack(host, axis=1)
    say("decode B=3 (hs64)")
    compare(got, ref, what="B=3 decode")


def test_teacher_forced_decode_tiny_and_capacity():
    cfg = cngpt_amd.TINY
    params = cngpt_amd.init_weights(cfg, 42)
    rng = np.random.default_rng(2)
    seq = rng.integers(0, cfg.vocab_size, size=(2, 16), dtype=np.int32)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)
    with cngpt_amd.Model(cfg, params) as m:
        got = [m.decode_begin(seq[:, :4], capacity=16)]
        for t in range(4, 16):
            got.append(m.decode_step(seq[:, t]))
        # begin gives position 3, steps 4..15 give positions 4..15
        compare(np.stack(got, 1), ref[:, 3:], abs_tol=1e-4, what="tiny teacher-forced")
        # the cache is full at block_size positions
        with pytest.raises(cngpt_amd.CngptError, match="full"):
            m.decode_step(seq[:, 0])
        with pytest.raises(cngpt_amd.CngptError, match="capacity"):
            m.decode_begin(seq[:, :4], capacity=cfg.block_size + 1)
