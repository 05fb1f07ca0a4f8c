"""Single-sequence decode as persistent launches (the stages of a step as
phases whose outputs travel as tagged words) vs the oracle and vs the
kernel-per-stage decode.

Reference values as in test_decode_gpu.py: without window truncation the
logits of decode step i are row prompt+i-1 of one all-positions forward
over the final sequence (src/model.c:991-1016 reruns the prefix instead).
"""
import numpy as np
import pytest

import cngpt_amd
import oracle
from test_parity_gpu import compare, ocfg, randomize, say

pytestmark = pytest.mark.gpu

# widths 256 / 512 / 768 take 1 / 2 / 3 float4 per lane per column
CASES = {
    "c256_v1000": cngpt_amd.Config(2, 4, 256, 1000, 128),
    "c512_v3000": cngpt_amd.Config(2, 8, 512, 3000, 256),
    "c768_v50257": cngpt_amd.Config(3, 12, 768, 50257, 1024),
}


def model(cfg, seed):
    params = randomize(cfg, cngpt_amd.init_weights(cfg, seed), seed + 1)
    return params, cngpt_amd.Model(cfg, params)


@pytest.mark.parametrize("name", list(CASES))
def test_persistent_teacher_forced(name):
    """Host-fed tokens, one launch per step; 70 steps cross the 64-key
    boundaries of the attention splits."""
    cfg = CASES[name]
    params, m = model(cfg, 7)
    T0, steps = 5, 70
    seq = np.random.default_rng(3).integers(0, cfg.vocab_size, size=(1, T0 + steps),
                                            dtype=np.int32)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, T0 - 1:]
    with m:
        m.set_decode_path(cngpt_amd.DECODE_PERSISTENT)
        say(f"{name}: persistent teacher-forced, {steps} steps")
        got = [m.decode_begin(seq[:, :T0], capacity=T0 + steps)]
        for t in range(T0, T0 + steps):
            got.append(m.decode_step(seq[:, t]))
            assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
        assert m.decode_length() == T0 + steps
    compare(np.stack(got, 1), ref, what=f"{name} persistent")


def test_persistent_generate_matches_steps_kernels_and_oracle():
    """GPT-2 small width at 3 layers, a 900-token prompt (16 attention
    splits): one launch of 99 steps = 99 launches of one step (bitwise),
    = the kernel-per-stage decode and the oracle up to near-ties."""
    cfg = CASES["c768_v50257"]
    params, m = model(cfg, 11)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, size=(1, 900), dtype=np.int32)
    n = 100
    with m:
        m.set_decode_path(cngpt_amd.DECODE_PERSISTENT)
        say("c768: generate 100 after a 900-token prompt, persistent")
        m.decode_begin(prompt, capacity=900 + n - 1)
        gen = m.generate(n)
        assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
        say("c768: the same, one step per launch")
        m.decode_begin(prompt, capacity=900 + n - 1)
        steps = [m.decode_step(None) for _ in range(n - 1)]
        step_toks = np.concatenate([np.stack([s.argmax(-1) for s in steps], 1)], axis=1)
        assert np.array_equal(gen[:, 1:], step_toks), "single-launch vs per-step tokens"
        say("c768: the same on the kernel-per-stage path")
        m.set_decode_path(cngpt_amd.DECODE_KERNELS)
        m.decode_begin(prompt, capacity=900 + n - 1)
        kern = m.generate(n)
        assert m.decode_path() == cngpt_amd.DECODE_KERNELS
    seq = np.concatenate([prompt, gen[:, :-1]], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 899:]
    srt = np.sort(ref, axis=-1)
    tie = (srt[..., -1] - srt[..., -2]) < 1e-4
    first = np.argmax(gen != kern) if not np.array_equal(gen, kern) else n
    # the streams agree up to the first near-tie (after one, they may diverge)
    assert first == n or tie[0, first], ("persistent vs kernels diverge without a tie", first)
    assert np.array_equal(np.where(tie, 0, ref.argmax(-1)), np.where(tie, 0, gen))
    compare(np.stack(steps, 1), ref[:, 1:], what="c768 per-step logits")


def test_persistent_sampled_generate():
    """Sampled generate on the persistent path (one launch per step, then
    the sampler): temp 0.8, top-k 40; every token is sample_top_k of the
    oracle's logits of the sequence generated so far (until a draw falls
    within the logits' error of a CDF boundary, after which the streams
    may part), and the same draws on the kernel path give the same tokens
    up to that point."""
    from test_decode_gpu import cdf_gap
    cfg = CASES["c768_v50257"]
    params, m = model(cfg, 13)
    prompt = np.random.default_rng(6).integers(0, cfg.vocab_size, size=(1, 40), dtype=np.int32)
    n = 60
    draws = np.random.default_rng(8).random(n).astype(np.float32)
    with m:
        say("c768: sampled generate, persistent")
        m.decode_begin(prompt, capacity=40 + n - 1)
        gen = m.generate(n, 0.8, 40, draws)[0]
        assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
        say("c768: sampled generate, kernel path")
        m.set_decode_path(cngpt_amd.DECODE_KERNELS)
        m.decode_begin(prompt, capacity=40 + n - 1)
        kern = m.generate(n, 0.8, 40, draws)[0]
        assert m.decode_path() == cngpt_amd.DECODE_KERNELS
    seq = np.concatenate([prompt[0], gen[:-1]]).reshape(1, -1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[0, 39:]
    for i in range(n):
        want = oracle.sample_top_k(ref[i], 0.8, 40, float(draws[i]))
        if want != gen[i]:
            assert cdf_gap(ref[i], 0.8, 40, float(draws[i])) < 1e-3, (i, gen[i], want)
            say(f"  diverged at a CDF boundary at token {i}")
            break
        assert kern[i] == gen[i] or cdf_gap(ref[i], 0.8, 40, float(draws[i])) < 1e-3, i
        if kern[i] != gen[i]:
            break


def test_persistent_in_launch_sampling_designed_rows():
    """Sampling inside the persistent launch on logits rows set exactly (the
    final LayerNorm outputs e_0, so every step's logits are wte[:, 0]):
    random values, 50 ties at the cut spread over the vocabulary, and a
    3000-way tie at the top, which overflows the workgroups' candidate
    slots so that each step ends the launch and the host draws its token.
    Every token is sample_top_k of the row with its draw, up to the
    rounding of the CDF's fp32 running sums."""
    from test_decode_gpu import consistent, designed_logits_model, survivors
    V = 50257
    cfg, params, w = designed_logits_model(V)
    rng = np.random.default_rng(31)
    base = (rng.standard_normal(V) * 3).astype(np.float32)
    rows = {"random": base}
    r = base.copy()
    r[rng.choice(V, 30, replace=False)] = 30 + rng.random(30).astype(np.float32)
    r[np.arange(50) * 1000 + 7] = np.float32(25.0)
    rows["tie_spread"] = r
    r = base.copy()
    r[5000:8000] = np.float32(12.5)
    rows["wide_tie"] = r
    n = 24
    prompt = oracle.lcg_tokens(8, V, seed=4).reshape(1, 8)
    with cngpt_amd.Model(cfg, params) as m:
        for name, row in rows.items():
            w["wte"][:, 0] = row
            m.load_params(params)
            for temp, k in ((1.0, 40), (0.7, 1), (1.2, 64)):
                draws = rng.random(n).astype(np.float32)
                say(f"in-launch sampling: {name}, temp {temp}, top-k {k}")
                m.decode_begin(prompt, capacity=8 + n)
                got = m.generate(n, temp, k, draws)[0]
                assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
                tol = 1e-5 + 2 * survivors(row, temp, k) * 2.0**-24
                for i in range(n):
                    ref = oracle.sample_top_k(row, temp, k, float(draws[i]))
                    assert got[i] == ref or consistent(row, temp, k, float(draws[i]), got[i],
                                                       tol), (name, temp, k, i, got[i], ref)


def test_persistent_gpt2_small_long_context():
    """GPT-2 small at full depth, the last 24 positions of the 1024-token
    window (keys up to 1023)."""
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    seq = oracle.lcg_tokens(1024, cfg.vocab_size, seed=21).reshape(1, 1024)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 999:]
    with cngpt_amd.Model(cfg, params) as m:
        m.set_decode_path(cngpt_amd.DECODE_PERSISTENT)
        say("small: persistent decode at positions 1000..1023")
        got = [m.decode_begin(seq[:, :1000], capacity=1024)]
        for t in range(1000, 1024):
            got.append(m.decode_step(seq[:, t]))
        assert m.decode_path() == cngpt_amd.DECODE_PERSISTENT
    compare(np.stack(got, 1), ref, what="small long context")


def test_persistent_refuses_batches():
    cfg = CASES["c256_v1000"]
    params, m = model(cfg, 3)
    prompt = np.zeros((2, 4), np.int32)
    with m:
        m.decode_begin(prompt, capacity=16)
        m.set_decode_path(cngpt_amd.DECODE_PERSISTENT)
        with pytest.raises(cngpt_amd.CngptError, match="persistent"):
            m.decode_step(None)
        m.set_decode_path(cngpt_amd.DECODE_AUTO)
        m.decode_step(None)
        assert m.decode_path() == cngpt_amd.DECODE_KERNELS
        with pytest.raises(cngpt_amd.CngptError):
            m.set_decode_path(7)
    # widths above 768 take the kernel-per-stage decode only
    cfg = cngpt_amd.Config(1, 16, 1024, 1000, 64)
    params, m = model(cfg, 4)
    with m:
        m.decode_begin(np.zeros((1, 4), np.int32), capacity=16)
        m.set_decode_path(cngpt_amd.DECODE_PERSISTENT)
        with pytest.raises(cngpt_amd.CngptError, match="persistent"):
            m.decode_step(None)
