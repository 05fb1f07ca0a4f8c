"""The training step on the device (cngpt_hip_train_*) against the oracle's
restatement of gpt_forward with targets, gpt_backward and gpt_adamw
(src/model.c:442-921), itself pinned against float64 autograd through
transformers' GPT2LMHeadModel and torch.optim.AdamW (test_oracle_train.py).

Tolerances: both sides compute in fp32 with different summation orders
(MFMA tiles and fixed-order partial sums here, BLAS and row loops in the
oracle), so each parameter's gradient is compared per tensor within
2e-4 of that tensor's largest reference magnitude (plus 1e-6 absolute),
the loss within 1e-5 relative, AdamW results within a few ulp.
"""
import numpy as np
import pytest

import cngpt_amd
import oracle
from test_parity_gpu import ocfg, randomize, say

pytestmark = pytest.mark.gpu

LAYER_NAMES = ("ln1_w", "ln1_b", "attn_w", "attn_b", "proj_w", "proj_b",
               "ln2_w", "ln2_b", "fc_w", "fc_b", "mlp_w", "mlp_b")


def tensors(cfg):
    """(name, offset, size) of every parameter tensor in the flat layout."""
    off = [int(o) for o in oracle.offsets(ocfg(cfg))]
    names = ["wte", "wpe"] + [f"h{l}.{n}" for l in range(cfg.n_layer) for n in LAYER_NAMES]
    names += ["ln_f_w", "ln_f_b"]
    ends = off[1:len(names)] + [cngpt_amd.num_params(cfg)]
    return [(n, o, e - o) for n, o, e in zip(names, off, ends)]


def compare_grads(cfg, got, ref, rel=2e-4, what=""):
    worst = 0.0
    for name, o, n in tensors(cfg):
        g, r = got[o:o + n], ref[o:o + n]
        assert np.isfinite(g).all(), (what, name, "non-finite")
        err = float(np.abs(g - r).max())
        scale = float(np.abs(r).max())
        assert err <= rel * scale + 1e-6, (what, name, err, scale)
        worst = max(worst, err / (scale + 1e-30))
    say(f"  {what}: worst per-tensor relative gradient error {worst:.2e}")


def batch(cfg, B, T, seed):
    rng = np.random.default_rng(seed)
    tok = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    tgt = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    return tok, tgt


CASES = {
    # head size 8, three layers
    "tiny": (cngpt_amd.TINY, 2, 16),
    # head size 64 (the GPT-2 head), ragged rows: 3 x 37 = 111, padded to 128
    "hs64": (cngpt_amd.Config(2, 2, 128, 300, 64), 3, 37),
    # head size 128; width 48 with head size 16 (products with K = 48, 144, 192)
    "hs128": (cngpt_amd.Config(1, 2, 256, 500, 160), 2, 130),
    "c48": (cngpt_amd.Config(1, 3, 48, 257, 40), 3, 33),
    # GPT-2 small's width, heads and vocabulary (V = 50257: the padded
    # lm_head products) at two layers
    "gpt2_width": (cngpt_amd.Config(2, 12, 768, 50257, 128), 2, 64),
}


@pytest.mark.parametrize("name", list(CASES))
def test_forward_backward_vs_oracle(name):
    cfg, B, T = CASES[name]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 11), 12)
    tok, tgt = batch(cfg, B, T, 13)
    say(f"{name}: B={B} T={T}")
    ref = oracle.Trainer(ocfg(cfg), params, B, T)
    ref.zero_grad()
    ref_loss = ref.forward(tok, tgt)
    ref.backward()
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        loss = tr.forward(tok, tgt)
        tr.backward()
        grads = tr.grads
        assert np.array_equal(tr.params, params)   # the forward and backward change no weight
    say(f"  loss {loss:.6f} vs {ref_loss:.6f}")
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    compare_grads(cfg, grads, ref.grads, what=name)
    ref.close()


def test_attention_backward_whole_walks():
    """With at least 1024 causal walks (here 8 x 32 heads x 4 key blocks of
    128) the attention backward keeps each walk in one workgroup and stores
    the gradient; below that (every other case here) the walks are split in
    halves that add into a zeroed gradient."""
    cfg, B, T = cngpt_amd.Config(1, 32, 256, 97, 512), 8, 512
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 71), 72)
    tok, tgt = batch(cfg, B, T, 73)
    ref = oracle.Trainer(ocfg(cfg), params, B, T)
    ref.zero_grad()
    ref_loss = ref.forward(tok, tgt)
    ref.backward()
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        loss = tr.forward(tok, tgt)
        tr.backward()
        grads = tr.grads
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    compare_grads(cfg, grads, ref.grads, what="whole walks (hs 8)")
    ref.close()


def test_gpt2_small_full_depth_step():
    """GPT-2 small at full depth and width (the bench's training model),
    B=2 T=128, seeded weights with LayerNorm gains and biases randomised:
    loss and every parameter's gradient, then one AdamW step."""
    cfg, B, T = cngpt_amd.GPT2_SMALL, 2, 128
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 1234), 5)
    tok, tgt = batch(cfg, B, T, 17)
    say("gpt2 small full depth: oracle step")
    ref = oracle.Trainer(ocfg(cfg), params, B, T)
    ref.zero_grad()
    ref_loss = ref.forward(tok, tgt)
    ref.backward()
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        loss = tr.forward(tok, tgt)
        tr.backward()
        grads = tr.grads
        norm = tr.adamw(3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
        p = tr.params
    say(f"  loss {loss:.6f} vs {ref_loss:.6f}")
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    compare_grads(cfg, grads, ref.grads, what="gpt2 small")
    want = float(np.sqrt((ref.grads.astype(np.float64) ** 2).sum()))
    assert abs(norm - want) <= 1e-4 * want
    ref.adamw(3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
    err = np.abs(p - ref.params)
    say(f"  after AdamW: max|dparam| {err.max():.2e}, {int((err > 1e-5).sum())} above 1e-5")
    assert err.max() <= 2 * 3e-4 and np.mean(err > 1e-5) < 1e-3
    ref.close()


def test_gradients_accumulate_reproducibly_and_zero_grad_clears():
    cfg, B, T = CASES["hs64"]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 21), 22)
    tok, tgt = batch(cfg, B, T, 23)
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        tr.forward(tok, tgt)
        tr.backward()
        once = tr.grads
        tr.forward(tok, tgt)
        tr.backward()
        twice = tr.grads
        tr.zero_grad()
        assert not tr.grads.any()
        tr.forward(tok, tgt)
        tr.backward()
        # fixed-order sums: the same step gives the same bits
        assert np.array_equal(tr.grads, once)
    np.testing.assert_allclose(twice, 2 * once, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("clip", [0.0, 1.0, 1e-3])
def test_adamw_vs_oracle(clip):
    """Three gpt_adamw steps on the same gradients: clipping by the global
    norm, bias correction, decay only on matrices and embeddings."""
    cfg = cngpt_amd.Config(2, 2, 32, 50, 16)
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 31), 32)
    rng = np.random.default_rng(33)
    ref = oracle.Trainer(ocfg(cfg), params, 1, 4)
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, 1, 4) as tr:
        for step in range(3):
            g = (rng.standard_normal(params.size) * 0.05).astype(np.float32)
            tr.write(cngpt_amd.TRAIN_GRADS, g)
            ref.grads[:] = g
            norm = tr.adamw(3e-3, 0.9, 0.95, 1e-8, 0.1, clip)
            ref.adamw(3e-3, 0.9, 0.95, 1e-8, 0.1, clip)
            want = float(np.sqrt((g.astype(np.float64) ** 2).sum()))
            assert abs(norm - want) <= 1e-6 * want
            assert tr.steps == step + 1
            for which, r in ((cngpt_amd.TRAIN_PARAMS, ref.params),
                             (cngpt_amd.TRAIN_GRADS, ref.grads),
                             (cngpt_amd.TRAIN_M, ref.m), (cngpt_amd.TRAIN_V, ref.v)):
                got = tr.read(which)
                # a weight that the update nearly cancels keeps the rounding
                # of terms of size lr = 3e-3 (ulp 2.3e-10): atol 1e-8
                np.testing.assert_allclose(got, r, rtol=4e-6, atol=1e-8)
    ref.close()


def test_training_steps_vs_oracle():
    """Four full steps (zero_grad, forward, backward, adamw with clipping)
    from the same weights: losses and weights track the oracle's."""
    cfg, B, T = cngpt_amd.Config(2, 4, 64, 97, 32), 4, 32
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 41), 42)
    ref = oracle.Trainer(ocfg(cfg), params, B, T)
    losses, ref_losses = [], []
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        for step in range(4):
            tok, tgt = batch(cfg, B, T, 100 + step)
            tr.zero_grad()
            losses.append(tr.forward(tok, tgt))
            tr.backward()
            tr.adamw(1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
            ref.zero_grad()
            ref_losses.append(ref.forward(tok, tgt))
            ref.backward()
            ref.adamw(1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
            p = tr.params
            err = float(np.abs(p - ref.params).max())
            moved = float(np.abs(ref.params - params).max())
            say(f"  step {step}: loss {losses[-1]:.6f} vs {ref_losses[-1]:.6f}, "
                f"max|dparam| {err:.2e} of {moved:.2e} moved")
            # Adam's update is lr * m_hat / (sqrt(v_hat) + eps): a gradient
            # element near zero can flip the sign of its step, so weights may
            # differ by up to ~2 lr per step on such elements
            assert err <= 2 * 1e-3 * (step + 1)
            assert np.mean(np.abs(p - ref.params) > 1e-5) < 1e-2
        # the updated weights serve the inference path of the same handle
        # (its 16-row products read the packed weight copies, which the
        # updates marked stale and the forward packs again)
        tok, _ = batch(cfg, 1, 16, 7)
        got = m.forward(tok, cngpt_amd.ALL)
    np.testing.assert_allclose(losses, ref_losses, rtol=1e-4)
    want = oracle.forward(ocfg(cfg), p, tok, oracle.ALL)
    assert float(np.abs(got - want).max()) < 1e-4
    ref.close()


def test_loss_falls_on_a_fixed_batch():
    cfg, B, T = cngpt_amd.TINY, 2, 16
    params = cngpt_amd.init_weights(cfg, 51)
    tok, tgt = batch(cfg, B, T, 52)
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        first = None
        for _ in range(30):
            tr.zero_grad()
            loss = tr.forward(tok, tgt)
            first = loss if first is None else first
            tr.backward()
            tr.adamw(1e-2, 0.9, 0.95, 1e-8, 0.0, 1.0)
    say(f"  loss {first:.4f} -> {loss:.4f}")
    assert loss < 0.5 * first


def test_errors():
    cfg = cngpt_amd.TINY
    params = cngpt_amd.init_weights(cfg, 61)
    with cngpt_amd.Model(cfg, params) as m:
        with pytest.raises(cngpt_amd.CngptError, match="positions"):
            cngpt_amd.Trainer(m, 1, cfg.block_size + 1)
        with cngpt_amd.Trainer(m, 1, 8) as tr:
            with pytest.raises(cngpt_amd.CngptError, match="no training forward"):
                tr.backward()
            tok = np.zeros(8, np.int32)
            bad = tok.copy()
            bad[3] = cfg.vocab_size
            with pytest.raises(cngpt_amd.CngptError, match="token"):
                tr.forward(bad, tok)
            with pytest.raises(cngpt_amd.CngptError, match="target"):
                tr.forward(tok, bad)
            with pytest.raises(cngpt_amd.CngptError, match="load_params"):
                tr.write(cngpt_amd.TRAIN_PARAMS, params)


@pytest.mark.parametrize("name,p", [("tiny", 0.1), ("hs64", 0.3), ("gpt2_width", 0.1)])
def test_dropout_vs_oracle(name, p):
    """GPTConfig.dropout: the same rand() stream (srand before each side)
    gives the device and the oracle the same keep masks at model.c's three
    sites; two steps, so the second forward's masks continue the stream."""
    cfg, B, T = CASES[name]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 31), 32)
    ref = oracle.Trainer(ocfg(cfg), params, B, T)
    ref.set_dropout(p)
    batches = [batch(cfg, B, T, 40 + i) for i in range(2)]
    oracle.srand(2024)
    ref_losses = []
    for tok, tgt in batches:
        ref.zero_grad()
        ref_losses.append(ref.forward(tok, tgt))
        ref.backward()
        ref.adamw(3e-3)
    with cngpt_amd.Model(cfg, params) as m, cngpt_amd.Trainer(m, B, T) as tr:
        tr.set_dropout(p)
        oracle.srand(2024)
        for i, (tok, tgt) in enumerate(batches):
            say(f"{name}: dropout {p}, step {i}")
            tr.zero_grad()
            loss = tr.forward(tok, tgt)
            tr.backward()
            # step 1 starts from weights updated on both sides (Adam may flip
            # the sign of a near-zero gradient element's step: see above)
            assert abs(loss - ref_losses[i]) <= (1e-5 if i == 0 else 1e-4) * abs(ref_losses[i]), \
                (i, loss, ref_losses[i])
            if i == 0:
                # the first step's gradients against a fresh oracle step
                chk = oracle.Trainer(ocfg(cfg), params, B, T)
                chk.set_dropout(p)
                oracle.srand(2024)
                chk.zero_grad()
                chk.forward(*batches[0])
                chk.backward()
                compare_grads(cfg, tr.grads, chk.grads, what=f"{name} dropout {p}")
                chk.close()   # its forward left the stream where step 0 left it
            tr.adamw(3e-3)
        params_dev = tr.params
    err = np.abs(params_dev - ref.params)
    assert float(err.max()) <= 2 * 3e-3 * 2
    assert np.mean(err > 1e-5) < 1e-2
    ref.close()


def test_dropout_rate_outside_range_is_refused():
    cfg, B, T = CASES["tiny"]
    with cngpt_amd.Model(cfg, cngpt_amd.init_weights(cfg, 1)) as m, cngpt_amd.Trainer(m, B, T) as tr:
        for p in (1.0, -0.1, float("nan")):
            with pytest.raises(cngpt_amd.CngptError):
                tr.set_dropout(p)
        tr.set_dropout(0.0)
