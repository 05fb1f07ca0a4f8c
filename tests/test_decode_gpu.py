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


# ---------------------------------------------------------------- generate / sampling

def cdf_gap(logits, temp, top_k, r):
    """Distance from r to the nearest boundary of the sampling CDF that
    sample_top_k (src/model.c:927-989) builds from these logits (float64)."""
    x = logits.astype(np.float64) / (temp if temp > 0 else 1.0)
    p = np.exp(x - x.max())
    p /= p.sum()
    if 0 < top_k < p.size:
        thr = np.sort(p)[-top_k]
        p = np.where(p < thr, 0.0, p)
        p /= p.sum()
    c = np.cumsum(p)
    return float(np.abs(c - r).min())


def test_generate_greedy_matches_stepwise_and_oracle():
    cfg = cngpt_amd.Config(2, 4, 256, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 5), 6)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab_size, size=(3, 17), dtype=np.int32)
    n = 40
    with cngpt_amd.Model(cfg, params) as m:
        first = m.decode_begin(prompt, capacity=17 + n - 1)
        gen = m.generate(n)
        assert gen.shape == (3, n)
        assert m.decode_length() == 17 + n - 1
        m.decode_begin(prompt, capacity=17 + n - 1)
        toks = [first.argmax(-1).astype(np.int32)]
        for _ in range(n - 1):
            toks.append(m.decode_step(toks[-1]).argmax(-1).astype(np.int32))
    assert np.array_equal(gen, np.stack(toks, 1))
    seq = np.concatenate([prompt, gen[:, :-1]], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 16:]
    srt = np.sort(ref, axis=-1)
    tie = (srt[..., -1] - srt[..., -2]) < 1e-4
    assert np.array_equal(np.where(tie, 0, ref.argmax(-1)), np.where(tie, 0, gen))
    say("generate greedy B=3 n=40")


def test_decode_more_than_eight_sequences():
    """B > 8 takes the MFMA tile products and the row argmax kernel."""
    cfg = cngpt_amd.Config(2, 4, 256, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 8), 9)
    prompt = np.random.default_rng(12).integers(0, cfg.vocab_size, size=(12, 9), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        logits = [m.decode_begin(prompt, capacity=40)]
        toks = [logits[0].argmax(-1).astype(np.int32)]
        for _ in range(20):
            logits.append(m.decode_step(toks[-1]))
            toks.append(logits[-1].argmax(-1).astype(np.int32))
        m.decode_begin(prompt, capacity=40)
        gen = m.generate(21)
    assert np.array_equal(gen, np.stack(toks, 1))
    seq = np.concatenate([prompt, np.stack(toks[:-1], 1)], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 8:]
    say("decode B=12")
    compare(np.stack(logits, 1), ref, what="B=12 decode")


@pytest.mark.parametrize("C,H,B", [(128, 2, 5), (128, 4, 70)])
def test_decode_layernorm_formed_by_the_residual_products(C, H, B):
    """Over more than two sequences each residual product (c_proj, proj)
    also writes the next LayerNorm: in its split-K sum, or, where K is not
    split (width 128: one chunk) or the rows take MFMA tiles (70 > 64), by
    a LayerNorm launch right after it."""
    cfg = cngpt_amd.Config(2, H, C, 500, 64)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 21), 22)
    prompt = np.random.default_rng(13).integers(0, cfg.vocab_size, size=(B, 7), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        logits = [m.decode_begin(prompt, capacity=24)]
        toks = [logits[0].argmax(-1).astype(np.int32)]
        for _ in range(12):
            logits.append(m.decode_step(toks[-1]))
            toks.append(logits[-1].argmax(-1).astype(np.int32))
    seq = np.concatenate([prompt, np.stack(toks[:-1], 1)], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 6:]
    say(f"decode C={C} B={B}")
    compare(np.stack(logits, 1), ref, what=f"C={C} B={B} decode")


@pytest.mark.parametrize("C,H,B", [(256, 4, 5), (256, 8, 20), (256, 2, 3), (384, 6, 33),
                                   (256, 2, 64), (128, 16, 8), (256, 16, 24)])
def test_decode_split_products_widths(C, H, B):
    """Batched decode over widths whose products split K two or three ways
    (the in-order reduce of each split product writes row t of the cache,
    which every later step reads back), 3 to 64 sequences (one to four
    16-row blocks of the few-row products), head sizes 8 to 128; with at
    least 128 (sequence, head) pairs the attention runs in one pass (16
    wavefronts per pair, 8 from 384 pairs), below that split by keys and
    merged."""
    cfg = cngpt_amd.Config(2, H, C, 300, 48)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 31), 32)
    prompt = np.random.default_rng(17).integers(0, cfg.vocab_size, size=(B, 9), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        logits = [m.decode_begin(prompt, capacity=40)]
        toks = [logits[0].argmax(-1).astype(np.int32)]
        for _ in range(20):
            logits.append(m.decode_step(toks[-1]))
            toks.append(logits[-1].argmax(-1).astype(np.int32))
    seq = np.concatenate([prompt, np.stack(toks[:-1], 1)], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 8:]
    say(f"decode C={C} H={H} B={B}")
    compare(np.stack(logits, 1), ref, what=f"C={C} H={H} B={B} decode")


SAMPLE_CASES = [(0.8, 40), (1.0, 40), (0.0, 40), (1.0, 1), (1.3, 0), (0.7, 50257),
                (1.0, 5000)]


def test_device_sampling_matches_oracle():
    """cngpt_hip_sample vs the oracle's sample_top_k on the same logits and
    draws; a token may differ only when the draw sits within rounding of a
    CDF boundary. (1.0, 5000) keeps more than 2048 values and takes the
    blocked running-sum path; top_k 0 / >= V means no cut."""
    cfg = cngpt_amd.Config(1, 4, 256, 50257, 64)
    params = cngpt_amd.init_weights(cfg, 21)
    w = oracle.unpack(ocfg(cfg), params)
    w["wte"][:] *= 40.0          # logits with a realistic spread (sd ~ 3)
    prompt = np.tile(oracle.lcg_tokens(20, cfg.vocab_size, seed=3), (8, 1))
    rng = np.random.default_rng(4)
    with cngpt_amd.Model(cfg, params) as m:
        logits = m.decode_begin(prompt, capacity=32)
        row = logits[0]
        assert np.array_equal(logits, np.tile(row, (8, 1)))
        checked = skipped = 0
        for temp, k in SAMPLE_CASES:
            draws = rng.random(48).astype(np.float32)
            draws[:3] = [0.0, 0.5, np.float32(0.99999994)]
            for i in range(0, draws.size, 8):
                got = m.sample(8, temp, k, draws[i:i + 8])
                for r, g in zip(draws[i:i + 8], got):
                    ref = oracle.sample_top_k(row, temp, k, float(r))
                    if g != ref:
                        assert cdf_gap(row, temp, k, float(r)) < 1e-5, (temp, k, r, g, ref)
                        skipped += 1
                    checked += 1
        say(f"sampling: {checked} draws, {skipped} at a boundary")
        assert skipped <= 2
        # all-equal logits: every value ties at the threshold
        flat = np.zeros((8, 20), np.int32)
        params2 = params.copy()
        oracle.unpack(ocfg(cfg), params2)["wte"][:] = 0.0
        m.load_params(params2)
        row2 = m.decode_begin(flat, capacity=32)[0]
        assert np.all(row2 == row2[0])
        draws = np.array([0.0, 0.1, 0.25, 0.5, 0.75, 0.9, 0.999, 0.3333], np.float32)
        got = m.sample(8, 1.0, 40, draws)
        for r, g in zip(draws, got):
            ref = oracle.sample_top_k(row2, 1.0, 40, float(r))
            assert g == ref or cdf_gap(row2, 1.0, 40, float(r)) < 1e-5, (r, g, ref)


def survivors(logits, temp, top_k):
    """Number of values sample_top_k keeps (float64)."""
    x = logits.astype(np.float64) / (temp if temp > 0 else 1.0)
    if not 0 < top_k < x.size:
        return x.size
    return int((x >= np.sort(x)[-top_k]).sum())


def consistent(logits, temp, top_k, r, tok, tol):
    """tok is the token sample_top_k returns for draw r when its CDF is
    exact (float64) up to tol: r falls in tok's CDF step widened by tol."""
    x = logits.astype(np.float64) / (temp if temp > 0 else 1.0)
    p = np.exp(x - x.max())
    p /= p.sum()
    if 0 < top_k < p.size:
        p = np.where(p < np.sort(p)[-top_k], 0.0, p)
        p /= p.sum()
    c = np.cumsum(p)
    if tok == p.size - 1 and p[tok] == 0:
        return r >= c[-1] - tol  # the fallback when the running sum stays <= r
    return p[tok] > 0 and c[tok] - p[tok] - tol <= r < c[tok] + tol


def designed_logits_model(V=50257):
    """A model whose last-position logits are wte[:, 0] exactly, whatever
    the tokens: the final LayerNorm has gain 0 and bias e_0, so its output
    is e_0 and the lm_head row of token v is 1 * wte[v, 0] + 0 * ...."""
    cfg = cngpt_amd.Config(1, 4, 256, V, 64)
    params = cngpt_amd.init_weights(cfg, 5)
    w = oracle.unpack(ocfg(cfg), params)
    w["ln_f_w"][:] = 0.0
    w["ln_f_b"][:] = 0.0
    w["ln_f_b"][0] = 1.0
    return cfg, params, w


def test_split_sampling_designed_rows():
    """The split top-k path (top_k <= 64: chunk lists, then one pick per
    row) on logits rows built exactly (designed_logits_model): top values
    all in the first chunk (its list full, so the chunk is rescanned), exact
    ties at the cut inside one chunk and across chunks, a tie wider than
    the survivor list (blocked form), negative logits, top_k 1 / 40 / 64 and
    65 (the one-workgroup path), 8 rows at once."""
    V = 50257
    cfg, params, w = designed_logits_model(V)
    rng = np.random.default_rng(12)
    rows = {}
    base = (rng.standard_normal(V) * 3).astype(np.float32)
    rows["random"] = base
    r = base.copy()
    r[:100] = 20 + np.sort(rng.standard_normal(100)).astype(np.float32)  # all top-64 in chunk 0
    rows["first_chunk"] = r
    r = base.copy()
    r[:30] = 30 + rng.random(30).astype(np.float32)
    r[100:220] = np.float32(25.0)                 # 120 tied at the cut, one chunk
    rows["tie_one_chunk"] = r
    r = base.copy()
    r[rng.choice(V, 30, replace=False)] = 30 + rng.random(30).astype(np.float32)
    spread = np.arange(50) * 1000 + 7             # 50 tied at the cut, many chunks
    r[spread] = np.float32(25.0)
    rows["tie_spread"] = r
    r = base.copy()
    r[5000:8000] = np.float32(12.5)               # 3000 tied at the top: > 2048 survive
    rows["wide_tie"] = r
    rows["negative"] = (base - 200).astype(np.float32)
    prompt = np.tile(oracle.lcg_tokens(8, V, seed=3), (8, 1))
    checked = skipped = 0
    with cngpt_amd.Model(cfg, params) as m:
        for name, row in rows.items():
            near = 0
            w["wte"][:, 0] = row
            m.load_params(params)
            got_row = m.decode_begin(prompt, capacity=16)
            assert np.array_equal(got_row, np.tile(row, (8, 1))), name
            say(f"split sampling: {name}")
            for temp, k in ((1.0, 40), (0.8, 1), (1.3, 64), (1.0, 65), (0.0, 40)):
                draws = rng.random(16).astype(np.float32)
                draws[:2] = [0.0, np.float32(0.99999994)]
                for i in range(0, 16, 8):
                    got = m.sample(8, temp, k, draws[i:i + 8])
                    for rr, g in zip(draws[i:i + 8], got):
                        ref = oracle.sample_top_k(row, temp, k, float(rr))
                        checked += 1
                        if g != ref:
                            # both running sums are fp32: each is within n * 2^-24 of the
                            # exact CDF after n survivors (3000 tie in "wide_tie"), so
                            # the device token must be the exact CDF's token up to that
                            tol = 1e-5 + 2 * survivors(row, temp, k) * 2.0**-24
                            assert consistent(row, temp, k, float(rr), g, tol), (
                                name, temp, k, rr, g, ref)
                            near += rr < 0.9999  # draws next to 1 sit at the last step
            say(f"  {near} draws at a boundary")
            skipped += near
            # a 3000-way tie spaces the CDF steps 3.3e-4 apart: any draw is near one
            assert name == "wide_tie" or near <= 2, name
    say(f"split sampling: {checked} draws, {skipped} at a boundary")


def test_generate_sampling_gpt2_small_rand_stream():
    """The sampling loop of gpt_sample (src/model.c:991-1016) with the KV
    cache: draws from the reference's rand() stream after srand(7), temp 0.8,
    top-k 40. Each token is checked against sample_top_k over the oracle's
    logits of the sequence generated so far."""
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    prompt = oracle.lcg_tokens(32, cfg.vocab_size).reshape(1, 32)
    n = 48
    oracle.srand(7)
    draws = np.array([oracle.rand_uniform() for _ in range(n)], np.float32)
    with cngpt_amd.Model(cfg, params) as m:
        m.decode_begin(prompt, capacity=32 + n - 1)
        gen = m.generate(n, 0.8, 40, draws)[0]
    seq = np.concatenate([prompt[0], gen[:-1]]).reshape(1, -1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[0, 31:]
    for i in range(n):
        want = oracle.sample_top_k(ref[i], 0.8, 40, float(draws[i]))
        if want != gen[i]:
            # the device logits differ from the oracle's by <= 1e-3
            assert cdf_gap(ref[i], 0.8, 40, float(draws[i])) < 1e-3, (i, gen[i], want)
            say(f"  diverged at a CDF boundary at token {i}")
            break
    say(f"generate sampled small: {n} tokens")


def test_generate_sampling_gpt2_small_512_steps_teacher_forced():
    """The sampled decode leg as measured: GPT-2 small, the 32-token LCG
    prompt, 513 tokens at temp 0.8 / top-k 40 in one generate call (the
    whole run inside one persistent launch), fixed uniform draws. Every
    token is checked against sample_top_k over the oracle's logits of the
    sequence the device generated (teacher forcing: one oracle forward over
    all 544 positions), so a draw at a CDF boundary does not end the check."""
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    prompt = oracle.lcg_tokens(32, cfg.vocab_size, 777).reshape(1, 32)
    n = 513
    draws = np.random.default_rng(7).random(n).astype(np.float32)
    with cngpt_amd.Model(cfg, params) as m:
        m.decode_begin(prompt, capacity=32 + n - 1)
        gen = m.generate(n, 0.8, 40, draws)[0]
    seq = np.concatenate([prompt[0], gen[:-1]]).reshape(1, -1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[0, 31:]
    near = 0
    for i in range(n):
        want = oracle.sample_top_k(ref[i], 0.8, 40, float(draws[i]))
        if want != gen[i]:
            # the device logits differ from the oracle's by <= 1e-3
            assert cdf_gap(ref[i], 0.8, 40, float(draws[i])) < 1e-3, (i, gen[i], want)
            near += 1
    say(f"generate sampled small: {n} tokens, {near} at a CDF boundary")
    assert near <= 3


def test_packed_weights_bit_identical_to_row_major(monkeypatch):
    """A handle made with CNGPT_HIP_PACK=0 streams the row-major weights in
    its few-row products instead of their packed copy: the same values in
    the same order, so prefill and every batched decode step agree bit for
    bit (B=6 and a 40-row prompt put every product on the few-row kernel)."""
    cfg = cngpt_amd.Config(2, 4, 256, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 5), 6)
    prompt = oracle.lcg_tokens(6 * 40, cfg.vocab_size).reshape(6, 40) % cfg.vocab_size
    runs = []
    for pack in ("1", "0"):
        monkeypatch.setenv("CNGPT_HIP_PACK", pack)
        with cngpt_amd.Model(cfg, params) as m:
            got = [m.forward(prompt[:1, :40], cngpt_amd.ALL), m.decode_begin(prompt, capacity=60)]
            toks = got[-1].argmax(-1).astype(np.int32)
            for _ in range(12):
                got.append(m.decode_step(toks))
                toks = got[-1].argmax(-1).astype(np.int32)
        runs.append(got)
    for a, b in zip(*runs):
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_qkv_split_sum_in_attention_bit_identical(monkeypatch):
    """Batched decode steps whose QKV product splits K and whose attention
    runs one pass per (sequence, head): the attention sums the QKV partials
    of its head in split order plus the bias (the arithmetic of the sum
    launch it replaces) and writes row t of the cache, so every step's
    logits equal those of a handle made with CNGPT_HIP_QKVFOLD=0 bit for
    bit. GPT-2 small's width: B=12 (two workgroups per pair, the first
    writes the row) and B=24 (one per pair)."""
    cfg = cngpt_amd.Config(2, 12, 768, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 8), 9)
    for B in (12, 24):
        prompt = oracle.lcg_tokens(B * 9, cfg.vocab_size).reshape(B, 9) % cfg.vocab_size
        runs = []
        for fold in ("1", "0"):
            monkeypatch.setenv("CNGPT_HIP_QKVFOLD", fold)
            with cngpt_amd.Model(cfg, params) as m:
                got = [m.decode_begin(prompt, capacity=24)]
                toks = got[-1].argmax(-1).astype(np.int32)
                for _ in range(10):
                    got.append(m.decode_step(toks))
                    toks = got[-1].argmax(-1).astype(np.int32)
            runs.append(got)
        for a, b in zip(*runs):
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), B
        say(f"QKV sum in the attention, B={B}: 10 steps bit-identical")


def test_profiler_environment_turns_graph_replay_off(monkeypatch, capfd):
    """In rocprofv3's environment (it exports ROCPROF_OUTPUT_PATH to the
    program it profiles) a handle launches the batched decode step's kernels
    directly instead of replaying the captured step graph, and says so on
    stderr. The same kernels with the same arguments run either way, so
    every step agrees bit for bit with a handle that replays its graph."""
    cfg = cngpt_amd.Config(2, 4, 256, 1000, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 5), 6)
    prompt = oracle.lcg_tokens(6 * 20, cfg.vocab_size).reshape(6, 20) % cfg.vocab_size
    runs = []
    for profiled in (False, True):
        monkeypatch.delenv("ROCP_TOOL_LIBRARIES", raising=False)
        if profiled:
            monkeypatch.setenv("ROCPROF_OUTPUT_PATH", "/nonexistent-profile-output")
        else:
            monkeypatch.delenv("ROCPROF_OUTPUT_PATH", raising=False)
        capfd.readouterr()
        with cngpt_amd.Model(cfg, params) as m:
            got = [m.decode_begin(prompt, capacity=40)]
            toks = got[-1].argmax(-1).astype(np.int32)
            for _ in range(10):
                got.append(m.decode_step(toks))
                toks = got[-1].argmax(-1).astype(np.int32)
        noted = "profiler detected" in capfd.readouterr().err
        assert noted == profiled
        runs.append(got)
    for a, b in zip(*runs):
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    say("decode B=6 with the profiler environment: direct launches, bit-identical")


def test_prefill_of_four_sequences_on_whole_round_tiles():
    """A 4 x 300-token prompt (1200 rows): QKV and fc run 64 x 96 tiles
    that fill whole rounds of CUs, QKV writing each sequence's rows into its
    part of the KV cache (rows of 300 at a stride of the capacity); the
    prefill's logits and four greedy steps against the oracle."""
    cfg = cngpt_amd.Config(2, 12, 768, 50257, 512)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 9), 10)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab_size, size=(4, 300), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        got = [m.decode_begin(prompt, capacity=310)]
        for _ in range(4):
            got.append(m.decode_step(got[-1].argmax(-1).astype(np.int32)))
    toks = np.stack([g.argmax(-1) for g in got[:-1]], axis=1).astype(np.int32)
    seq = np.concatenate([prompt, toks], axis=1)
    ref = oracle.forward(ocfg(cfg), params, seq, oracle.ALL)[:, 299:]
    say("prefill 4 x 300 (whole-round tiles) + 4 steps")
    compare(np.stack(got, axis=1), ref, what="B=4 T=300 prefill and steps")
