"""GPT-2 medium and XL at full depth and width vs the oracle, and the three
workloads of the benchmark configurations at their stated shapes:

- GPT-2 medium: prefill B=8, T=1024; decode B=8 for 256 steps;
- GPT-2 XL: prefill B=4, T=1024; decode B=32 for 128 steps;
- GPT-2 small: 512 greedy decode steps after a 32-token prompt as one
  generate call (one persistent launch), the benchmark's decode leg.

Weights (medium, XL): N(0, 0.02) from numpy's generator (seeded; the
reference's rand() stream would take minutes to draw 1.5 G values),
LayerNorm gains and all biases randomised. Both sides read the same
parameter buffer, so the comparison is the forward pass only.

Decode reference values: without window truncation the logits of decode
step i are row prompt+i-1 of one all-positions forward over the final
sequence (src/model.c:991-1016 reruns the prefix instead, which gives the
same values). Decode that starts after a 1024-token prefill would leave the
1024-position window, so the medium decode starts from a 768-token prompt
(768 + 256 = 1024 positions) and the XL decode from a 32-token prompt.
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


def greedy_decode(m, prompt, steps):
    """decode_begin + `steps` host-fed greedy steps; logits [B, steps+1, V]
    and the tokens fed after the prompt [B, steps]."""
    B, T0 = prompt.shape
    logits = [m.decode_begin(prompt, capacity=T0 + steps)]
    toks = [logits[0].argmax(-1).astype(np.int32)]
    for i in range(steps):
        logits.append(m.decode_step(toks[-1]))
        toks.append(logits[-1].argmax(-1).astype(np.int32))
        if (i + 1) % 64 == 0:
            say(f"  step {i + 1} of {steps}")
    return np.stack(logits, 1), np.stack(toks[:-1], 1)


def decode_vs_oracle(m, cfg, params, B, prompt_len, steps, seed, what):
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab_size, size=(B, prompt_len),
                                                  dtype=np.int32)
    got, fed = greedy_decode(m, prompt, steps)
    seq = np.concatenate([prompt, fed], axis=1)
    say(f"  oracle over [{B}, {seq.shape[1]}]")
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, prompt_len - 1:]
    compare(got, ref, what=what)


def prefill_vs_oracle(m, cfg, params, tokens, all_rows, what):
    """LAST logits of every sequence, and all-position logits of the
    sequences in all_rows read back from one resident ALL forward."""
    B, T = tokens.shape
    V = cfg.vocab_size
    say(f"{what}: LAST B={B} T={T}")
    got = m.forward(tokens, cngpt_amd.LAST)
    compare(got, oracle.forward(ocfg(cfg), params, tokens), what=f"{what} LAST")
    say(f"{what}: ALL B={B} T={T}, sequences {list(all_rows)} read back")
    m.reserve(B, T, cngpt_amd.ALL)
    m.upload_tokens(tokens)
    m.forward_resident(B, T, cngpt_amd.ALL)
    m.synchronize()
    got = np.stack([m.read_logits(b * T * V, T * V).reshape(T, V) for b in all_rows])
    ref = oracle.forward(ocfg(cfg), params, tokens[list(all_rows)], oracle.ALL)
    compare(got, ref, what=f"{what} ALL")


@pytest.fixture(scope="module")
def medium():
    cfg = cngpt_amd.GPT2_MEDIUM
    params = normal_params(cfg, 101)
    with cngpt_amd.Model(cfg, params) as m:
        yield cfg, params, m


@pytest.fixture(scope="module")
def xl():
    cfg = cngpt_amd.GPT2_XL
    say("xl: drawing 1.56 G parameters")
    params = normal_params(cfg, 202)
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


def test_medium_prefill_b8_t1024(medium):
    """The configuration's prefill: M = 8192 rows (GEMM variants by tile
    count), LAST for all 8 sequences, ALL read back for sequences 0 and 7."""
    cfg, params, m = medium
    tk = np.random.default_rng(41).integers(0, cfg.vocab_size, size=(8, 1024), dtype=np.int32)
    prefill_vs_oracle(m, cfg, params, tk, (0, 7), "medium B=8 T=1024")


def test_medium_decode_b8(medium):
    cfg, params, m = medium
    say("medium decode B=8, 16 steps")
    decode_vs_oracle(m, cfg, params, 8, 24, 16, 5, "medium decode B=8")


def test_medium_decode_b8_256_steps(medium):
    """The configuration's decode: B=8 for 256 steps from a 768-token
    prompt (keys up to 1023); over 2 rows the residual products form the
    next LayerNorm in their split-K sum (C = 1024)."""
    cfg, params, m = medium
    say("medium decode B=8, 256 steps after 768")
    decode_vs_oracle(m, cfg, params, 8, 768, 256, 42, "medium decode B=8 x 256")


def test_xl_full_depth(xl):
    """48 layers, 25 heads, C=1600: prefill (LAST and ALL) and batched decode
    at B=32 (the 16-column skinny products)."""
    cfg, params, m = xl
    tk = np.random.default_rng(4).integers(0, cfg.vocab_size, size=(2, 96), dtype=np.int32)
    say("xl LAST B=2 T=96")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
    say("xl ALL B=1 T=40")
    compare(m.forward(tk[:1, :40], cngpt_amd.ALL),
            oracle.forward(ocfg(cfg), params, tk[:1, :40], oracle.ALL), what="ALL")
    say("xl decode B=32, 6 steps")
    decode_vs_oracle(m, cfg, params, 32, 8, 6, 6, "xl decode B=32")


def test_xl_prefill_b4_t1024(xl):
    """The configuration's prefill: M = 4096 rows, LAST for all 4
    sequences, ALL read back for sequence 2."""
    cfg, params, m = xl
    tk = np.random.default_rng(43).integers(0, cfg.vocab_size, size=(4, 1024), dtype=np.int32)
    prefill_vs_oracle(m, cfg, params, tk, (2,), "xl B=4 T=1024")


def test_xl_decode_b32_128_steps(xl):
    """The configuration's decode: B=32 for 128 steps from a 32-token
    prompt; the 1600-wide residual rows take two float4 per thread in the
    LayerNorm formed by the split-K sum."""
    cfg, params, m = xl
    say("xl decode B=32, 128 steps after 32")
    decode_vs_oracle(m, cfg, params, 32, 32, 128, 44, "xl decode B=32 x 128")


def test_small_generate_512_steps():
    """The benchmark's decode leg: GPT-2 small with the seeded init (srand
    1234), a 32-token LCG prompt, 512 greedy steps as one generate call
    (one persistent launch). The tokens must equal 512 one-step launches
    (bitwise) and the oracle's argmax of the generated sequence up to
    near-ties; the per-step logits must match the oracle's."""
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    prompt = oracle.lcg_tokens(32, cfg.vocab_size, seed=777).reshape(1, 32)
    n = 513
    with cngpt_amd.Model(cfg, params) as m:
        say("small: generate 513 after 32, one launch")
        m.decode_begin(prompt, capacity=32 + n - 1)
        gen = m.generate(n)
        assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
        say("small: the same, one step per launch")
        first = m.decode_begin(prompt, capacity=32 + n - 1)
        steps = [first] + [m.decode_step(None) for _ in range(n - 1)]
    step_toks = np.stack([s.argmax(-1) for s in steps], 1)
    assert np.array_equal(gen, step_toks), "single-launch vs per-step tokens"
    seq = np.concatenate([prompt, gen[:, :-1]], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 31:]
    srt = np.sort(ref, axis=-1)
    tie = (srt[..., -1] - srt[..., -2]) < 1e-4
    say(f"  near-ties in the oracle's stream: {int(tie.sum())}")
    assert np.array_equal(np.where(tie, 0, ref.argmax(-1)), np.where(tie, 0, gen))
    compare(np.stack(steps, 1), ref, what="small 512-step decode logits")
