"""GPT-2 medium and XL at full depth and width vs the oracle.

Weights: N(0, 0.02) from numpy's generator (seeded; the reference's rand()
stream would take minutes to draw 1.5 G values), LayerNorm gains and all
biases randomised. Both sides read the same parameter buffer, so the
comparison is the forward pass only.
"""
import numpy as np
import pytest

import cngpt_amd
import oracle
from test_parity_gpu import compare, ocfg, randomize, say

pytestmark = pytest.mark.gpu


def normal_params(cfg, seed):
    n = cngpt_amd.num_params(cfg)
    p = np.random.default_rng(seed).standard_normal(n, dtype=np.float32)
    p *= np.float32(0.02)
    return randomize(cfg, p, seed + 1)


def decode_vs_oracle(m, cfg, params, B, prompt_len, steps, seed, what):
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, size=(B, prompt_len),
                                                  dtype=np.int32)
    logits = [m.decode_begin(prompt, capacity=prompt_len + steps)]
    toks = [logits[0].argmax(-1).astype(np.int32)]
    for _ in range(steps):
        logits.append(m.decode_step(toks[-1]))
        toks.append(logits[-1].argmax(-1).astype(np.int32))
    seq = np.concatenate([prompt, np.stack(toks[:-1], 1)], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, prompt_len - 1:]
    compare(np.stack(logits, 1), ref, what=what)


@pytest.fixture(scope="module")
def medium():
    cfg = cngpt_amd.GPT2_MEDIUM
    params = normal_params(cfg, 101)
    with cngpt_amd.Model(cfg, params) as m:
        yield cfg, params, m


def test_medium_prefill(medium):
    cfg, params, m = medium
    rng = np.random.default_rng(3)
    tk = rng.integers(0, cfg.vocab_size, size=(2, 256), dtype=np.int32)
    say("medium LAST B=2 T=256")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
    tk = rng.integers(0, cfg.vocab_size, size=(1, 160), dtype=np.int32)
    say("medium ALL B=1 T=160")
    compare(m.forward(tk, cngpt_amd.ALL), oracle.forward(ocfg(cfg), params, tk, oracle.ALL),
            what="ALL")


def test_medium_decode_b8(medium):
    cfg, params, m = medium
    say("medium decode B=8")
    decode_vs_oracle(m, cfg, params, 8, 24, 16, 5, "medium decode B=8")


def test_xl_full_depth():
    """48 layers, 25 heads, C=1600: prefill (LAST and ALL) and batched decode
    at B=32 (the 16-column skinny products)."""
    cfg = cngpt_amd.GPT2_XL
    params = normal_params(cfg, 202)
    with cngpt_amd.Model(cfg, params) as m:
        tk = np.random.default_rng(4).integers(0, cfg.vocab_size, size=(2, 96), dtype=np.int32)
        say("xl LAST B=2 T=96")
        compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
        say("xl ALL B=1 T=40")
        compare(m.forward(tk[:1, :40], cngpt_amd.ALL),
                oracle.forward(ocfg(cfg), params, tk[:1, :40], oracle.ALL), what="ALL")
        say("xl decode B=32")
        decode_vs_oracle(m, cfg, params, 32, 8, 6, 6, "xl decode B=32")
