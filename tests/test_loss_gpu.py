"""Cross-entropy over the logits held on the device vs the oracle's
cross_entropy_fwd restatement (src/ops.c:499-574) and float64 log-sum-exp.

Tolerances, written per check:
  * device row terms vs float64 on the same logits: 1e-5 + 2e-6 |ref|
    (the device sums each row in short runs and trees);
  * device vs the oracle on the same logits: the oracle's own rounding,
    a running fp32 sum of V terms (V * 2^-24 relative) per row and of B*T
    rows for the mean;
  * the whole chain (forward + loss) vs the oracle's chain: the above plus
    2 max|logit diff| (a row term moves by at most twice the largest change
    of a logit).
The loss bar of the reference's scripts/verify_forward.py:279-281 is
|diff| < 5e-4; every comparison here is tighter.
"""
import numpy as np
import pytest
import scipy.special

import cngpt_amd
import oracle
from test_parity_gpu import ocfg, randomize, say

pytestmark = pytest.mark.gpu


def f64_rows(logits, targets):
    l64 = logits.reshape(-1, logits.shape[-1]).astype(np.float64)
    t = targets.reshape(-1)
    return scipy.special.logsumexp(l64, axis=1) - l64[np.arange(t.size), t]


def check_same_logits(logits, targets, loss, rows, what):
    """Device loss / row terms vs float64 and vs the oracle on the logits the
    device held."""
    V = logits.shape[-1]
    n = targets.size
    ref = f64_rows(logits, targets)
    err = np.abs(rows.reshape(-1) - ref)
    say(f"  {what}: rows vs float64 max|diff|={err.max():.2e}, loss={loss:.6f}")
    assert np.all(err <= 1e-5 + 2e-6 * np.abs(ref)), (what, err.max())
    assert abs(loss - ref.mean()) <= 1e-6 * max(1.0, abs(ref.mean())), (what, loss, ref.mean())
    o_loss, o_rows, _ = oracle.cross_entropy(logits, targets)
    row_tol = 1e-5 + 4e-6 * np.abs(ref) + V * 2.0**-24 * np.maximum(1.0, np.abs(o_rows))
    assert np.all(np.abs(rows.reshape(-1) - o_rows) <= row_tol), what
    mean_tol = 1e-5 + (n + V) * 2.0**-24 * max(1.0, abs(o_loss))
    assert abs(loss - o_loss) <= mean_tol, (what, loss, o_loss)


CASES = {
    # tiny (check_fast.c's shape): V = 70, rows start at every other float
    "tiny": (cngpt_amd.TINY, 3, 16, 1.0),
    # V = 333: rows start at every alignment
    "v333": (cngpt_amd.Config(2, 4, 128, 333, 96), 2, 96, 1.0),
    # LayerNorm gain x 400: logits in the hundreds (expf overflows without
    # the max subtraction)
    "large_logits": (cngpt_amd.Config(1, 4, 256, 1000, 64), 2, 64, 400.0),
}


@pytest.mark.parametrize("name", list(CASES))
def test_loss_chain_vs_oracle(name):
    cfg, B, T, gain = CASES[name]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 5), 6)
    oracle.unpack(ocfg(cfg), params)["ln_f_w"][:] *= gain
    rng = np.random.default_rng(17)
    tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    targets = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    ref_logits = oracle.forward(ocfg(cfg), params, tokens, oracle.ALL)
    ref_loss, ref_rows, ref_probs = oracle.cross_entropy(ref_logits, targets, True)
    with cngpt_amd.Model(cfg, params) as m:
        say(f"{name}: forward + loss B={B} T={T} V={cfg.vocab_size}")
        loss, logits = m.loss(tokens, targets, copy_logits=True)
        loss2, rows = m.cross_entropy(targets, rows=True)
        assert loss2 == loss  # the held logits are unchanged by the loss
        check_same_logits(logits, targets, loss, rows, name)
        dl = float(np.abs(logits - ref_logits).max())
        tol = 2 * dl + 1e-5 + cfg.vocab_size * 2.0**-24 * np.maximum(1.0, np.abs(ref_rows))
        assert np.all(np.abs(rows.reshape(-1) - ref_rows) <= tol), name
        assert abs(loss - ref_loss) <= 2 * dl + 1e-4, (name, loss, ref_loss)
        say(f"  chain: loss {loss:.6f} vs oracle {ref_loss:.6f}, max|logit diff|={dl:.2e}")
        # probs_out: the softmax replaces the held logits
        loss3 = m.cross_entropy(targets, probs=True)
        assert loss3 == loss
        probs = m.read_logits(0, B * T * cfg.vocab_size).reshape(B * T, cfg.vocab_size)
    own = scipy.special.softmax(logits.reshape(B * T, -1).astype(np.float64), axis=1)
    np.testing.assert_allclose(probs, own, rtol=2e-5, atol=1e-12)
    np.testing.assert_allclose(probs.sum(1), 1.0, atol=1e-5)
    # vs the oracle's probs of its own logits: as above plus exp(2 dl)
    np.testing.assert_allclose(probs, ref_probs,
                               rtol=2e-5 + 2.5 * dl + cfg.vocab_size * 2.0**-24, atol=1e-9)


def test_loss_last_positions_and_decode():
    """[B, V] logits (LAST forward, decode step) take targets [B] (T = 1)."""
    cfg = CASES["v333"][0]
    params = randomize(cfg, cngpt_amd.init_weights(cfg, 9), 10)
    rng = np.random.default_rng(2)
    tokens = rng.integers(0, cfg.vocab_size, size=(3, 20), dtype=np.int32)
    tg = rng.integers(0, cfg.vocab_size, size=3, dtype=np.int32)
    with cngpt_amd.Model(cfg, params) as m:
        say("v333: loss of LAST logits")
        lg = m.forward(tokens, cngpt_amd.LAST)
        loss, rows = m.cross_entropy(tg, rows=True)
        check_same_logits(lg, tg, loss, rows, "LAST")
        with pytest.raises(cngpt_amd.CngptError, match="logits are held"):
            m.cross_entropy(np.zeros((3, 20), np.int32))
        say("v333: loss of decode-step logits")
        m.decode_begin(tokens, capacity=24)
        lg = m.decode_step(tg)
        loss, rows = m.cross_entropy(tg, rows=True)
        check_same_logits(lg, tg, loss, rows, "decode")


def test_loss_errors():
    cfg = CASES["tiny"][0]
    params = cngpt_amd.init_weights(cfg, 1)
    with cngpt_amd.Model(cfg, params) as m:
        with pytest.raises(cngpt_amd.CngptError, match="no cross-entropy"):
            m.read_loss()
        tk = np.zeros((2, 8), np.int32)
        m.forward(tk, cngpt_amd.ALL, copy=False)
        for bad in (-1, cfg.vocab_size):
            tg = np.zeros((2, 8), np.int32)
            tg[1, 3] = bad
            with pytest.raises(cngpt_amd.CngptError, match="target"):
                m.cross_entropy(tg)
        with pytest.raises(cngpt_amd.CngptError, match="logits are held"):
            m.cross_entropy(np.zeros((2, 7), np.int32))
        # the handle still works after the errors
        say("tiny: loss after errors")
        tg = np.arange(16, dtype=np.int32).reshape(2, 8)
        loss = m.cross_entropy(tg)
        m.upload_targets(tg)
        m.cross_entropy_resident(2, 8)
        loss2, rows = m.read_loss(rows=True)
        assert loss2 == loss and rows.shape == (16,)


def test_loss_gpt2_small_b16_t1024():
    """The B=16 T=1024 all-position logits (16384 rows x 50257, 3.29 GB)
    stay in HBM; the loss is read back, then every logit row, sequence by
    sequence, for the float64 check (and the oracle on sequences 0 and 15)."""
    cfg = cngpt_amd.GPT2_SMALL
    V, B, T = cfg.vocab_size, 16, 1024
    params = cngpt_amd.init_weights(cfg, 1234)
    tokens = oracle.lcg_tokens(B * T, V, seed=12345).reshape(B, T)
    targets = np.roll(tokens.reshape(-1), -1).reshape(B, T)  # next-token targets
    with cngpt_amd.Model(cfg, params) as m:
        say("small B=16 T=1024: forward ALL + loss on the device")
        m.reserve(B, T, cngpt_amd.ALL)
        m.upload_tokens(tokens)
        m.forward_resident(B, T, cngpt_amd.ALL)
        m.upload_targets(targets)
        m.cross_entropy_resident(B, T)
        loss, rows = m.read_loss(rows=True)
        rows = rows.reshape(B, T)
        ref_rows = np.empty((B, T))
        for b in range(B):
            lg = m.read_logits(b * T * V, T * V).reshape(T, V)
            ref_rows[b] = f64_rows(lg, targets[b])
            if b in (0, B - 1):
                say(f"  sequence {b}: oracle cross-entropy on the device's logits")
                check_same_logits(lg, targets[b], float(rows[b].astype(np.float64).mean()),
                                  rows[b], f"seq {b}")
    err = np.abs(rows - ref_rows)
    say(f"  loss {loss:.6f} vs float64 {ref_rows.mean():.6f}; rows max|diff|={err.max():.2e}")
    assert np.all(err <= 1e-5 + 2e-6 * np.abs(ref_rows))
    assert abs(loss - ref_rows.mean()) <= 1e-6 * abs(ref_rows.mean())
    # seeded N(0, 0.02) weights give near-uniform predictions: loss ~ log V
    assert abs(loss - np.log(V)) < 0.5
