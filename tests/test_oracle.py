"""Pins for the CPU oracle (oracle/cngpt_oracle.c) -- no GPU.

Each function of the oracle is checked against something it does not
compute itself: the hand-computed known answers of the reference's
tests/check_ops.c, float64 library routines (numpy, torch, scipy,
transformers' GPT2LMHeadModel), and invariants the mathematics fixes.
"""
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle

TOL_KAT = 1e-3


# ---------------------------------------------------------------- ops KATs
# Hand-computed values of tests/check_ops.c:69-182.

def test_linear_kat():                       # check_ops.c:69-82
    X = np.array([[1, 0], [0, 1]], np.float32)
    W = np.array([[2, 3], [4, 5]], np.float32)
    b = np.array([1, -1], np.float32)
    np.testing.assert_allclose(oracle.linear(X, W, b), [[3, 3], [4, 4]], atol=1e-5)


def test_layernorm_kat():                    # check_ops.c:118-136
    out, mean, rstd = oracle.layernorm(np.array([[1, 2, 3, 4]], np.float32),
                                       np.ones(4, np.float32), np.zeros(4, np.float32))
    assert abs(mean[0] - 2.5) < 1e-4
    np.testing.assert_allclose(out[0], [-1.3416, -0.4472, 0.4472, 1.3416], atol=TOL_KAT)
    assert abs(out.sum()) < 1e-4


def test_gelu_kat():                         # check_ops.c:146-157
    out = oracle.gelu(np.array([0, 1, -1, 2], np.float32))
    np.testing.assert_allclose(out, [0.0, 0.8413, -0.1587, 1.9545], atol=TOL_KAT)


def test_softmax_kat():                      # check_ops.c:165-182
    x = oracle.softmax(np.array([[1, 2, 3], [100, 100, 100]], np.float32))
    np.testing.assert_allclose(x[0], [0.0900, 0.2447, 0.6652], atol=TOL_KAT)
    assert abs(x[0].sum() - 1) < 1e-5
    np.testing.assert_allclose(x[1], [1 / 3] * 3, atol=1e-5)


# ---------------------------------------------------------------- float64 library pins

def test_linear_vs_float64_matmul_odd_shapes():
    rng = np.random.default_rng(1)
    for M, K, N in [(1, 4, 1), (37, 100, 53), (130, 1600, 81), (5, 768, 2304)]:
        X = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.standard_normal((N, K)).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        ref = X.astype(np.float64) @ W.astype(np.float64).T + b
        got = oracle.linear(X, W, b)
        assert np.abs(got - ref).max() <= 1e-5 * math.sqrt(K) * 4, (M, K, N)


def test_layernorm_vs_torch_float64():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((33, 768)) * 3 + 1.5).astype(np.float32)
    w = rng.standard_normal(768).astype(np.float32)
    b = rng.standard_normal(768).astype(np.float32)
    got, mean, rstd = oracle.layernorm(x, w, b)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,),
                                         torch.from_numpy(w).double(),
                                         torch.from_numpy(b).double(), eps=1e-5).numpy()
    assert np.abs(got - ref).max() < 2e-5
    np.testing.assert_allclose(mean, x.astype(np.float64).mean(1), rtol=1e-5, atol=1e-6)
    # invariant with unit gain / zero bias: each row has mean 0 and variance 1
    z, _, _ = oracle.layernorm(x, np.ones(768, np.float32), np.zeros(768, np.float32))
    assert np.abs(z.mean(1)).max() < 1e-5
    assert np.abs(z.var(1) - 1).max() < 1e-3


def test_gelu_vs_torch_tanh_float64():
    x = np.linspace(-12, 12, 10001).astype(np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    assert np.abs(oracle.gelu(x) - ref).max() < 2e-6


def test_softmax_and_mask():
    rng = np.random.default_rng(3)
    s = (rng.standard_normal((17, 17)) * 4).astype(np.float32)
    m = oracle.causal_mask(s)
    upper = np.triu_indices(17, 1)
    assert np.all(m[upper] == np.float32(-1e9))
    assert np.array_equal(np.tril(m), np.tril(s))
    p = oracle.softmax(m)
    assert np.all(p[upper] == 0.0)                # masked probability is exactly 0
    assert p[0, 0] == 1.0                         # a one-key row
    np.testing.assert_allclose(p.sum(1), 1, atol=1e-6)
    ref = scipy.special.softmax(np.where(np.triu(np.ones_like(s), 1) > 0, -np.inf,
                                         s.astype(np.float64)), axis=1)
    assert np.abs(p - ref).max() < 1e-6


# ---------------------------------------------------------------- cross-entropy

def test_cross_entropy_kat():                # check_ops.c:191-210
    tg = np.array([0, 1], np.int32)
    loss, rows, probs = oracle.cross_entropy(np.array([[10, 0], [0, 10]], np.float32), tg, True)
    assert abs(loss) < 0.01
    assert abs(probs[0, 0] - 1) < 0.01 and abs(probs[1, 1] - 1) < 0.01
    loss2, _, _ = oracle.cross_entropy(np.array([[0, 10], [10, 0]], np.float32), tg)
    assert loss2 > 5.0
    # the closed forms of both cases: log(1 + e^-10) and log(1 + e^10)
    assert abs(loss - math.log1p(math.exp(-10))) < 1e-6
    assert abs(loss2 - math.log1p(math.exp(10))) < 1e-5


def test_cross_entropy_vs_torch_float64():
    """torch's cross_entropy in float64, the loss verify_forward.py:110-112
    checks cngpt against; per row against scipy's logsumexp."""
    rng = np.random.default_rng(4)
    for rows, V, scale in [(1, 2, 1.0), (37, 1000, 5.0), (6, 50257, 3.0)]:
        lg = (rng.standard_normal((rows, V)) * scale + 40).astype(np.float32)
        tg = rng.integers(0, V, size=rows, dtype=np.int32)
        loss, per_row, probs = oracle.cross_entropy(lg, tg, True)
        l64 = lg.astype(np.float64)
        ref = float(torch.nn.functional.cross_entropy(torch.from_numpy(l64),
                                                      torch.from_numpy(tg.astype(np.int64))))
        # a running fp32 sum of V positive terms is within V * 2^-24 of the
        # exact one, relatively, which bounds the error of log(sum)
        tol = 4e-6 * abs(ref) + V * 2.0**-24
        assert abs(loss - ref) <= tol, (rows, V, loss, ref)
        ref_rows = scipy.special.logsumexp(l64, axis=1) - l64[np.arange(rows), tg]
        assert np.abs(per_row - ref_rows).max() <= tol
        np.testing.assert_allclose(probs, scipy.special.softmax(l64, axis=1),
                                   rtol=4e-6 + V * 2.0**-24, atol=1e-9)
        assert np.array_equal(probs, oracle.softmax(lg))  # same arithmetic as ops.c:424-482


def test_cross_entropy_closed_forms():
    # V equal logits: log V whatever the level (expf(125) overflows without
    # the max subtraction)
    for V in (1, 7, 50257):
        for c in (0.0, 125.0, -300.0):
            loss, _, _ = oracle.cross_entropy(np.full((3, V), c, np.float32),
                                              np.array([0, V // 2, V - 1], np.int32))
            assert abs(loss - math.log(V)) <= 1e-6 * max(1.0, math.log(V)), (V, c, loss)
    # the mean is over all B*T rows: rows with losses log(1+e^-d) for d = 0..5
    d = np.arange(6, dtype=np.float32)
    lg = np.stack([d, np.zeros(6, np.float32)], 1).reshape(2, 3, 2)
    loss, per_row, _ = oracle.cross_entropy(lg, np.zeros((2, 3), np.int32))
    want = np.log1p(np.exp(-d.astype(np.float64)))
    np.testing.assert_allclose(per_row, want, rtol=1e-6, atol=1e-7)
    assert abs(loss - want.mean()) < 1e-6
    # a per-row shift leaves the loss unchanged; the target's logit enters
    # with a minus sign
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((4, 300)).astype(np.float32)
    tg = rng.integers(0, 300, size=4, dtype=np.int32)
    base, _, _ = oracle.cross_entropy(lg, tg)
    shifted, _, _ = oracle.cross_entropy(lg + np.float32(64), tg)
    assert abs(base - shifted) < 1e-5
    up = lg.copy()
    up[np.arange(4), tg] += 1
    assert oracle.cross_entropy(up, tg)[0] < base


# ---------------------------------------------------------------- whole forward

def _hf_logits(cfg: oracle.Cfg, params: np.ndarray, tokens: np.ndarray) -> np.ndarray:
    """transformers' GPT2LMHeadModel, built from a local config in float64,
    with the flat cngpt weights copied in (Conv1D weights are [in, out])."""
    from transformers import GPT2Config, GPT2LMHeadModel

    hc = GPT2Config(vocab_size=cfg.vocab_size, n_positions=cfg.block_size, n_embd=cfg.n_embd,
                    n_layer=cfg.n_layer, n_head=cfg.n_head, resid_pdrop=0.0, embd_pdrop=0.0,
                    attn_pdrop=0.0, layer_norm_epsilon=1e-5, activation_function="gelu_new",
                    bos_token_id=0, eos_token_id=0)
    hc._attn_implementation = "eager"
    model = GPT2LMHeadModel(hc).double().eval()
    w = oracle.unpack(cfg, params)
    t = lambda a: torch.from_numpy(np.array(a, dtype=np.float64))  # noqa: E731
    sd = {"transformer.wte.weight": t(w["wte"]), "transformer.wpe.weight": t(w["wpe"]),
          "transformer.ln_f.weight": t(w["ln_f_w"]), "transformer.ln_f.bias": t(w["ln_f_b"])}
    for l, L in enumerate(w["layers"]):
        p = f"transformer.h.{l}."
        sd[p + "ln_1.weight"] = t(L["ln1_w"])
        sd[p + "ln_1.bias"] = t(L["ln1_b"])
        sd[p + "attn.c_attn.weight"] = t(L["c_attn_w"].T)
        sd[p + "attn.c_attn.bias"] = t(L["c_attn_b"])
        sd[p + "attn.c_proj.weight"] = t(L["c_proj_w"].T)
        sd[p + "attn.c_proj.bias"] = t(L["c_proj_b"])
        sd[p + "ln_2.weight"] = t(L["ln2_w"])
        sd[p + "ln_2.bias"] = t(L["ln2_b"])
        sd[p + "mlp.c_fc.weight"] = t(L["mlp_fc_w"].T)
        sd[p + "mlp.c_fc.bias"] = t(L["mlp_fc_b"])
        sd[p + "mlp.c_proj.weight"] = t(L["mlp_proj_w"].T)
        sd[p + "mlp.c_proj.bias"] = t(L["mlp_proj_b"])
    sd["lm_head.weight"] = sd["transformer.wte.weight"]
    model.load_state_dict(sd, strict=False)
    with torch.no_grad():
        return model(torch.from_numpy(tokens.astype(np.int64))).logits.numpy()


def _randomize_ln_and_biases(cfg, params, seed):
    """The seeded init leaves LN gains 1 and biases 0; randomize them so a
    dropped or misplaced bias / gain cannot pass."""
    rng = np.random.default_rng(seed)
    p = params.copy()
    w = oracle.unpack(cfg, p)
    for L in w["layers"]:
        for k in ("ln1_w", "ln2_w"):
            L[k][:] = 1 + 0.1 * rng.standard_normal(L[k].shape)
        for k in ("ln1_b", "ln2_b", "c_attn_b", "c_proj_b", "mlp_fc_b", "mlp_proj_b"):
            L[k][:] = 0.05 * rng.standard_normal(L[k].shape)
    w["ln_f_w"][:] = 1 + 0.1 * rng.standard_normal(w["ln_f_w"].shape)
    w["ln_f_b"][:] = 0.05 * rng.standard_normal(w["ln_f_b"].shape)
    return p


HF_CASES = [oracle.TINY, oracle.Cfg(2, 2, 128, 300, 64)]


@pytest.mark.parametrize("cfg", HF_CASES, ids=["tiny_hs8", "hs64"])
def test_forward_all_vs_transformers_float64(cfg):
    params = _randomize_ln_and_biases(cfg, oracle.init_weights(cfg, 42), 5)
    rng = np.random.default_rng(11)
    B, T = 3, cfg.block_size
    tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    got = oracle.forward(cfg, params, tokens, oracle.ALL)
    ref = _hf_logits(cfg, params, tokens)
    err = np.abs(got - ref).max()
    assert err < 1e-4, err
    last = oracle.forward(cfg, params, tokens, oracle.LAST)
    assert np.abs(last - ref[:, -1]).max() < 1e-4


def test_forward_last_matches_all_check_fast_shapes():
    """check_fast.c:88-94 shapes: LAST (fast.c) vs ALL's final rows."""
    cfg = oracle.TINY
    params = oracle.init_weights(cfg, 42)
    rng = np.random.default_rng(0)
    for B, T in [(1, 1), (1, 9), (2, 6), (3, 16), (1, 16)]:
        tk = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
        for threads in (1, 2, 3):
            oracle.set_threads(threads)
            last = oracle.forward(cfg, params, tk, oracle.LAST)
            full = oracle.forward(cfg, params, tk, oracle.ALL)
            assert np.abs(last - full[:, -1]).max() < 1e-5, (B, T, threads)
    oracle.set_threads(0)


def test_forward_causal_and_batch_invariants():
    cfg = oracle.Cfg(2, 2, 64, 97, 32)
    params = _randomize_ln_and_biases(cfg, oracle.init_weights(cfg, 3), 4)
    rng = np.random.default_rng(5)
    tk = rng.integers(0, cfg.vocab_size, size=(3, 32), dtype=np.int32)
    full = oracle.forward(cfg, params, tk, oracle.ALL)
    # positions <= t do not see tokens after t
    tk2 = tk.copy()
    tk2[:, 20:] = rng.integers(0, cfg.vocab_size, size=(3, 12))
    full2 = oracle.forward(cfg, params, tk2, oracle.ALL)
    assert np.abs(full[:, :20] - full2[:, :20]).max() < 1e-6
    assert np.abs(full[:, 20:] - full2[:, 20:]).max() > 1e-3
    # sequences are independent
    one = oracle.forward(cfg, params, tk[1:2], oracle.ALL)
    assert np.abs(one[0] - full[1]).max() < 1e-6


def test_forward_rejects_bad_input():
    cfg = oracle.TINY
    params = oracle.init_weights(cfg, 1)
    with pytest.raises(ValueError):
        oracle.forward(cfg, params, np.full((1, 4), cfg.vocab_size, np.int32))
    with pytest.raises(ValueError):
        oracle.forward(cfg, params, np.zeros((1, cfg.block_size + 1), np.int32))


# ---------------------------------------------------------------- init and layout

def test_param_counts():
    # model.c:20-48 for the GPT-2 sizes (124.4M / 354.8M / 1557.6M)
    assert oracle.num_params(oracle.GPT2_SMALL) == 124_439_808
    assert oracle.num_params(oracle.GPT2_MEDIUM) == 354_823_168
    assert oracle.num_params(oracle.GPT2_XL) == 1_557_611_200
    off = oracle.offsets(oracle.GPT2_SMALL)
    assert off[1] == 50257 * 768 and off[2] == off[1] + 1024 * 768
    assert off[-1] + 768 == oracle.num_params(oracle.GPT2_SMALL)


def test_init_statistics():
    cfg = oracle.Cfg(4, 4, 128, 1000, 64)
    p = oracle.init_weights(cfg, 1234)
    w = oracle.unpack(cfg, p)
    assert abs(w["wte"].std() - 0.02) < 0.0005 and abs(w["wte"].mean()) < 0.0005
    res = 0.02 / math.sqrt(2 * cfg.n_layer)
    for L in w["layers"]:
        assert np.all(L["ln1_w"] == 1) and np.all(L["ln1_b"] == 0)
        assert np.all(L["c_attn_b"] == 0) and np.all(L["mlp_proj_b"] == 0)
        assert abs(L["c_attn_w"].std() - 0.02) < 0.001
        assert abs(L["c_proj_w"].std() - res) < 0.0006
        assert abs(L["mlp_proj_w"].std() - res) < 0.0003
    assert np.all(w["ln_f_w"] == 1) and np.all(w["ln_f_b"] == 0)
    # same seed, same stream; different seed, different stream
    assert np.array_equal(p, oracle.init_weights(cfg, 1234))
    assert not np.array_equal(p[:100], oracle.init_weights(cfg, 1235)[:100])


def test_lcg_tokens():
    # cngpt.c:338-342 recurrence, first values worked by hand
    s = 12345
    s = (s * 1664525 + 1013904223) % 2**32
    first = (s >> 8) % 50257
    t = oracle.lcg_tokens(3, 50257)
    assert t[0] == first and np.all((t >= 0) & (t < 50257))


# ---------------------------------------------------------------- sampling

def test_sample_top_k_cdf():
    logits = np.log(np.array([1, 2, 3, 4], np.float32))   # p = .1 .2 .3 .4
    for r, want in [(0.05, 0), (0.15, 1), (0.35, 2), (0.65, 3), (0.9999, 3)]:
        assert oracle.sample_top_k(logits, 1.0, 0, r) == want
    # top-2 keeps .3 and .4, renormalised to 3/7 and 4/7
    assert oracle.sample_top_k(logits, 1.0, 2, 0.1) == 2
    assert oracle.sample_top_k(logits, 1.0, 2, 3 / 7 + 0.01) == 3
    # temp <= 0 is treated as 1 (model.c:934)
    assert oracle.sample_top_k(logits, 0.0, 0, 0.15) == 1
    # a high temperature flattens the distribution: r=0.3 then lands earlier
    assert oracle.sample_top_k(logits, 100.0, 0, 0.3) == 1


def test_sample_top_k_ties_and_greedy():
    logits = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    # top_k=1 keeps every entry tied with the maximum (model.c:970-972)
    assert oracle.sample_top_k(logits, 1.0, 1, 0.25) == 1
    assert oracle.sample_top_k(logits, 1.0, 1, 0.75) == 2
    rng = np.random.default_rng(9)
    v = rng.standard_normal(1000).astype(np.float32)
    for r in (0.0, 0.5, 0.999):
        assert oracle.sample_top_k(v, 0.8, 1, r) == int(np.argmax(v))
