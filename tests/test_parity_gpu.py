"""HIP forward pass vs the CPU oracle on the same seeded weights and tokens.

Bar: logits max|diff| <= 1e-3 and max|diff| / max|ref| <= 1e-4,
argmax identical. The tiny shapes of the reference's tests/check_fast.c use
that test's own tighter bound, max|diff| < 1e-4 (check_fast.c:62).
"""
import sys

import numpy as np
import pytest

import cngpt_amd
import oracle

pytestmark = pytest.mark.gpu

ABS_TOL = 1e-3
REL_TOL = 1e-4


def ocfg(cfg):
    return oracle.Cfg(cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def compare(got, ref, abs_tol=ABS_TOL, rel_tol=REL_TOL, check_argmax=True, what=""):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite logits"
    err = float(np.abs(got - ref).max())
    rel = err / float(np.abs(ref).max())
    say(f"  {what}: max|diff|={err:.3e} rel={rel:.3e}")
    assert err <= abs_tol and rel <= rel_tol, (what, err, rel)
    if check_argmax:
        ga, ra = got.argmax(-1), ref.argmax(-1)
        if not np.array_equal(ga, ra):
            # only a near-tie in the reference may flip the argmax
            srt = np.sort(ref, axis=-1)
            gap = (srt[..., -1] - srt[..., -2])[ga != ra]
            assert np.all(gap < 2 * err), (what, "argmax differs", gap)


def randomize(cfg, params, seed):
    """Non-trivial LayerNorm gains and biases (the seeded init has 1 / 0)."""
    rng = np.random.default_rng(seed)
    p = params.copy()
    w = oracle.unpack(ocfg(cfg), p)
    for L in w["layers"]:
        for k in ("ln1_w", "ln2_w"):
            L[k][:] = 1 + 0.1 * rng.standard_normal(L[k].shape)
        for k in ("ln1_b", "ln2_b", "c_attn_b", "c_proj_b", "mlp_fc_b", "mlp_proj_b"):
            L[k][:] = 0.05 * rng.standard_normal(L[k].shape)
    w["ln_f_w"][:] = 1 + 0.1 * rng.standard_normal(w["ln_f_w"].shape)
    w["ln_f_b"][:] = 0.05 * rng.standard_normal(w["ln_f_b"].shape)
    return p


# ---------------------------------------------------------------- check_fast mirror

def test_check_fast_shapes_tiny():
    """tests/check_fast.c: 3L/4H/32C/V70/T16 (head size 8), srand(42), shapes
    {1,1},{1,9},{2,6},{3,16},{1,16}, final-position logits, < 1e-4."""
    cfg = cngpt_amd.TINY
    params = cngpt_amd.init_weights(cfg, 42)
    rng = np.random.default_rng(42)
    with cngpt_amd.Model(cfg, params) as m:
        for B, T in [(1, 1), (1, 9), (2, 6), (3, 16), (1, 16)]:
            tk = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
            say(f"tiny B={B} T={T}")
            compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk),
                    abs_tol=1e-4, what="LAST")
            compare(m.forward(tk, cngpt_amd.ALL),
                    oracle.forward(ocfg(cfg), params, tk, oracle.ALL), abs_tol=1e-4, what="ALL")


HS_CASES = {
    "hs64": (cngpt_amd.Config(2, 4, 256, 1000, 256), [(1, 1), (1, 7), (2, 64), (3, 129), (2, 256)]),
    "hs32": (cngpt_amd.Config(2, 4, 128, 333, 96), [(1, 5), (2, 33), (1, 96)]),
    "hs16": (cngpt_amd.Config(1, 8, 128, 257, 70), [(2, 70)]),
    "hs128": (cngpt_amd.Config(1, 2, 256, 500, 160), [(2, 130), (1, 160)]),
    # widths that are not multiples of 32 (GEMM K steps of 16) or of 16
    # (register-staged tiles, zero-filled past K), more than 64 rows each
    "hs16_c48": (cngpt_amd.Config(1, 3, 48, 257, 40), [(2, 40), (3, 33)]),
    "hs8_c40": (cngpt_amd.Config(1, 5, 40, 101, 24), [(3, 24), (4, 19)]),
    # an all-position lm_head of 2 x 297 tiles: more than one round at 2
    # workgroups per CU, all in one at 4 (GEMM K steps of 16, two stages)
    "v38000": (cngpt_amd.Config(1, 4, 256, 38000, 64), [(4, 64)]),
}


@pytest.mark.parametrize("name", list(HS_CASES))
def test_head_sizes_and_ragged_shapes(name):
    cfg, shapes = HS_CASES[name]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 1234), 3)
    rng = np.random.default_rng(9)
    with cngpt_amd.Model(cfg, params) as m:
        for B, T in shapes:
            tk = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
            say(f"{name} B={B} T={T}")
            compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk),
                    what="LAST")
            compare(m.forward(tk, cngpt_amd.ALL),
                    oracle.forward(ocfg(cfg), params, tk, oracle.ALL), what="ALL")


# ---------------------------------------------------------------- GPT-2 sizes

@pytest.fixture(scope="module")
def small():
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    m = cngpt_amd.Model(cfg, params)
    yield cfg, params, m
    m.close()


def test_gpt2_small_b1_t64(small):
    """GPT-2 small, B=1, T=64 LCG tokens (cngpt.c:338-342), both modes."""
    cfg, params, m = small
    tk = oracle.lcg_tokens(64, cfg.vocab_size).reshape(1, 64)
    say("small B=1 T=64")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
    compare(m.forward(tk, cngpt_amd.ALL), oracle.forward(ocfg(cfg), params, tk, oracle.ALL),
            what="ALL")


def test_gpt2_small_zero_tokens_b2_t300(small):
    """All-zero tokens (the reference's timing input, cngpt.c:283) and a
    sequence length that is not a multiple of any tile."""
    cfg, params, m = small
    tk = np.zeros((2, 300), np.int32)
    tk[1] = oracle.lcg_tokens(300, cfg.vocab_size, seed=99)
    say("small B=2 T=300")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")


def test_gpt2_small_b16_t1024(small):
    """The B=16 T=1024 workload the bench times (16384 rows: 128-row tiles
    with the K=16 three-per-CU QKV variant): final-position logits of all 16
    sequences, then the all-position logits of sequences 0 and 15 read back
    from HBM at every position."""
    cfg, params, m = small
    V, T = cfg.vocab_size, 1024
    tk = oracle.lcg_tokens(16 * T, V, seed=12345).reshape(16, T)
    say("small B=16 T=1024 LAST")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
    m.reserve(16, T, cngpt_amd.ALL)
    m.upload_tokens(tk)
    m.forward_resident(16, T, cngpt_amd.ALL)
    m.synchronize()
    for b in (0, 15):
        say(f"small B=16 T=1024 ALL, sequence {b}")
        got = m.read_logits(b * T * V, T * V).reshape(1, T, V)
        compare(got, oracle.forward(ocfg(cfg), params, tk[b:b + 1], oracle.ALL),
                what=f"ALL seq {b}")


def test_gpt2_small_split_k_shapes(small):
    """Products with too few 128 x 128 tiles to fill the CUs split K and sum
    the partials in order (forming the next LayerNorm in the same pass for
    the residual products): the reference's own shape B=1 T=128 (M = 128:
    6 to 24 tiles per product), one GPU's share of the B=16 workload, B=2
    T=1024 (M = 2048: c_proj and proj 96 tiles), and B=3 T=200."""
    cfg, params, m = small
    V = cfg.vocab_size
    for B, T, seed in ((1, 128, 5), (3, 200, 6), (2, 1024, 7)):
        tk = oracle.lcg_tokens(B * T, V, seed=seed).reshape(B, T)
        say(f"small B={B} T={T} LAST")
        compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk),
                what=f"B={B} T={T} LAST")
        say(f"small B={B} T={T} ALL, last sequence")
        m.reserve(B, T, cngpt_amd.ALL)
        m.upload_tokens(tk)
        m.forward_resident(B, T, cngpt_amd.ALL)
        m.synchronize()
        got = m.read_logits((B - 1) * T * V, T * V).reshape(1, T, V)
        compare(got, oracle.forward(ocfg(cfg), params, tk[B - 1:], oracle.ALL),
                what=f"B={B} T={T} ALL")


def test_short_prefills_with_cproj_in_attention(small):
    """17 to 128 rows of 64-wide heads: the attention launch applies each
    head's 64 rows of the c_proj inner dimension to its output and writes
    per-head partials, which one launch sums in head order with the bias,
    the residual and LayerNorm 2. Ragged query blocks (T not a multiple of
    32), several sequences, both modes, the products on 32-row tiles (33 to
    128 rows) or weight-streaming (up to 32); GPT-2 medium's and large's
    widths (C = 1024 and 1280) on one layer."""
    cfg, params, m = small
    V = cfg.vocab_size
    for B, T, seed in ((1, 100, 11), (2, 50, 12), (4, 32, 13), (1, 65, 14), (1, 40, 16),
                       (3, 7, 17), (1, 17, 18), (2, 20, 19)):
        tk = oracle.lcg_tokens(B * T, V, seed=seed).reshape(B, T)
        say(f"small B={B} T={T} LAST and ALL")
        compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk),
                what=f"B={B} T={T} LAST")
        compare(m.forward(tk, cngpt_amd.ALL)[-1:],
                oracle.forward(ocfg(cfg), params, tk[-1:], oracle.ALL), what=f"B={B} T={T} ALL")
    # C = 1280, 20 heads (GPT-2 large's width): 80 query blocks take 4 column
    # blocks per wavefront over 5 slices, 400 workgroups at two per CU
    for C, H in ((1024, 16), (1280, 20)):
        mcfg = cngpt_amd.Config(1, H, C, 5000, 128)
        mp = randomize(mcfg, cngpt_amd.init_weights(mcfg, 77), 5)
        with cngpt_amd.Model(mcfg, mp) as mm:
            tk = oracle.lcg_tokens(128, mcfg.vocab_size, seed=15).reshape(1, 128)
            say(f"C={C} H={H} B=1 T=128 ALL")
            compare(mm.forward(tk, cngpt_amd.ALL),
                    oracle.forward(ocfg(mcfg), mp, tk, oracle.ALL), what=f"C={C} ALL")


def test_gpt2_small_b17_t512(small):
    """8704 rows: 68 row tiles leave the last round of the QKV (1224 tiles)
    and fc (1632 tiles) products under 90 % full at 4 and at 3 workgroups
    per CU, so both take the K=32 two-per-CU GEMM variant."""
    cfg, params, m = small
    tk = oracle.lcg_tokens(17 * 512, cfg.vocab_size, seed=777).reshape(17, 512)
    say("small B=17 T=512")
    compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk), what="LAST")
    say("small B=17 T=512 ALL, sequence 16")
    got = m.forward(tk, cngpt_amd.ALL)[16:]
    compare(got, oracle.forward(ocfg(cfg), params, tk[16:], oracle.ALL), what="ALL seq 16")


def test_resident_path_matches(small):
    cfg, params, m = small
    tk = oracle.lcg_tokens(2 * 128, cfg.vocab_size, seed=5).reshape(2, 128)
    ref = m.forward(tk, cngpt_amd.ALL)
    m.reserve(2, 128, cngpt_amd.ALL)
    m.upload_tokens(tk)
    m.forward_resident(2, 128, cngpt_amd.ALL)
    m.synchronize()
    got = m.read_logits(0, ref.size).reshape(ref.shape)
    assert np.array_equal(got, ref)


def test_xl_width_one_layer():
    """XL widths: C=1600 (K not a multiple of 128), 25 heads, N=4800/6400,
    ragged vocabulary 50257."""
    cfg = cngpt_amd.Config(1, 25, 1600, 50257, 128)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 77), 8)
    tk = np.random.default_rng(3).integers(0, cfg.vocab_size, size=(2, 100), dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        say("xl-width B=2 T=100")
        compare(m.forward(tk, cngpt_amd.ALL), oracle.forward(ocfg(cfg), params, tk, oracle.ALL),
                what="ALL")
        compare(m.forward(tk, cngpt_amd.LAST), oracle.forward(ocfg(cfg), params, tk),
                what="LAST")


# ---------------------------------------------------------------- errors

def test_errors_are_reported(small):
    cfg, params, m = small
    with pytest.raises(cngpt_amd.CngptError, match="token"):
        m.forward(np.array([[1, 2, cfg.vocab_size]], np.int32))
    with pytest.raises(cngpt_amd.CngptError, match="token"):
        m.forward(np.array([[-1]], np.int32))
    with pytest.raises(cngpt_amd.CngptError, match="block_size"):
        m.forward(np.zeros((1, cfg.block_size + 1), np.int32))
    with pytest.raises(cngpt_amd.CngptError, match="parameter count"):
        m.load_params(params[:-1])
    with pytest.raises(cngpt_amd.CngptError):
        cngpt_amd.Model(cfg, params, device=99)
    # the handle still works after the errors
    tk = np.zeros((1, 4), np.int32)
    compare(m.forward(tk), oracle.forward(ocfg(cfg), params, tk), what="after errors")


def test_forward_graph_replays_match_direct_launches(monkeypatch):
    """cngpt_hip_forward and cngpt_hip_forward_resident replay a captured
    graph per shape; a handle made with CNGPT_HIP_GRAPH=0 launches the same
    kernels directly. Every call agrees bit for bit: repeated shapes with new
    tokens (the replay reads the uploaded tokens), shape changes (a new
    capture), an arena growth, and a decode (eager launches) in between."""
    cfg = cngpt_amd.Config(2, 12, 768, 50257, 1024)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 61), 62)
    rng = np.random.default_rng(63)
    monkeypatch.setenv("CNGPT_HIP_GRAPH", "1")
    g = cngpt_amd.Model(cfg, params)
    monkeypatch.setenv("CNGPT_HIP_GRAPH", "0")
    d = cngpt_amd.Model(cfg, params)
    try:
        calls = [(1, 128, cngpt_amd.LAST), (1, 128, cngpt_amd.LAST), (2, 64, cngpt_amd.ALL),
                 (1, 128, cngpt_amd.LAST), (5, 200, cngpt_amd.LAST), (1, 128, cngpt_amd.LAST)]
        for i, (B, T, mode) in enumerate(calls):
            say(f"forward graph replay {i}: B={B} T={T} mode={mode}")
            tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
            a = g.forward(tokens, mode)
            b = d.forward(tokens, mode)
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
            # the resident entry point replays the same graph
            g.upload_tokens(tokens)
            g.forward_resident(B, T, mode)
            g.synchronize()
            n = B * cfg.vocab_size if mode == cngpt_amd.LAST else B * T * cfg.vocab_size
            c = g.read_logits(0, n)
            assert np.array_equal(c.view(np.uint32), b.reshape(-1).view(np.uint32)), i
            if i == 2:
                # eager work between replays: a few decode steps
                prompt = rng.integers(0, cfg.vocab_size, size=(2, 9), dtype=np.int32)
                l0 = g.decode_begin(prompt, capacity=20)
                g.decode_step(l0.argmax(-1).astype(np.int32))
    finally:
        g.close()
        d.close()
