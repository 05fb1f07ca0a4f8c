"""Pins for the oracle's training step (gpt_forward with targets,
gpt_backward, gpt_adamw: src/model.c:442-921) -- no GPU.

Each piece is checked against something it does not compute itself: the
hand-worked known answers of the reference's tests/check_ops.c (linear_bwd_dx
:84-105, the layernorm_bwd finite-difference check :212-245), float64 torch
autograd per op, float64 autograd through transformers' GPT2LMHeadModel built
from a local config with the same weights (every parameter's gradient and the
loss), and torch.optim.AdamW in float64 for the update (decoupled weight decay
on the tensors with two or more dimensions, nanoGPT's rule that
src/model.c:143-172 follows).
"""
import numpy as np
import pytest
import torch

import oracle
from test_oracle import _randomize_ln_and_biases


def test_linear_bwd_dx_kat():                 # check_ops.c:84-105
    dX = oracle.linear_bwd_dx(np.eye(2, dtype=np.float32), np.array([[2, 3], [4, 5]], np.float32))
    np.testing.assert_allclose(dX, [[2, 3], [4, 5]], atol=1e-5)


def test_layernorm_bwd_finite_difference_kat():   # check_ops.c:212-245
    x = np.array([[0.5, -0.3, 1.2, -0.8]], np.float32)
    w = np.array([1.0, 2.0, 0.5, 1.5], np.float32)
    b = np.array([0.1, -0.1, 0.2, -0.2], np.float32)
    dout = np.array([[0.3, -0.5, 0.7, -0.2]], np.float32)
    _, mean, rstd = oracle.layernorm(x, w, b)
    dx, _, _ = oracle.layernorm_bwd(dout, x, w, mean, rstd)
    eps = 1e-4
    xp, xm = x.copy(), x.copy()
    xp[0, 0] += eps
    xm[0, 0] -= eps
    num = ((dout * oracle.layernorm(xp, w, b)[0]).sum() -
           (dout * oracle.layernorm(xm, w, b)[0]).sum()) / (2 * eps)
    assert abs(dx[0, 0] - num) < 1e-3


def test_linear_bwd_dw_vs_float64():
    rng = np.random.default_rng(2)
    dY = rng.standard_normal((37, 53)).astype(np.float32)
    X = rng.standard_normal((37, 100)).astype(np.float32)
    dW0 = rng.standard_normal((53, 100)).astype(np.float32)
    dW, db = oracle.linear_bwd_dw(dY, X, dW0)
    ref = dW0 + dY.astype(np.float64).T @ X.astype(np.float64)
    assert np.abs(dW - ref).max() < 1e-4
    assert np.abs(db - dY.astype(np.float64).sum(0)).max() < 1e-5


def test_layernorm_and_gelu_bwd_vs_torch_float64():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((9, 64)) * 2 + 0.5).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    b = (0.1 * rng.standard_normal(64)).astype(np.float32)
    dout = rng.standard_normal((9, 64)).astype(np.float32)
    _, mean, rstd = oracle.layernorm(x, w, b)
    dx, dw, db = oracle.layernorm_bwd(dout, x, w, mean, rstd)
    tx, tw, tb = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w, b))
    torch.nn.functional.layer_norm(tx, (64,), tw, tb, 1e-5).backward(
        torch.tensor(dout, dtype=torch.float64))
    for got, ref in ((dx, tx.grad), (dw, tw.grad), (db, tb.grad)):
        assert np.abs(got - ref.numpy()).max() < 2e-5 * max(1.0, np.abs(ref.numpy()).max())
    g = np.linspace(-8, 8, 2001).astype(np.float32)
    d = rng.standard_normal(g.size).astype(np.float32)
    tg = torch.tensor(g, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.gelu(tg, approximate="tanh").backward(torch.tensor(d, dtype=torch.float64))
    assert np.abs(oracle.gelu_bwd(d, g) - tg.grad.numpy()).max() < 1e-5


def _hf_model(cfg, params):
    """float64 GPT2LMHeadModel with the flat cngpt weights copied in, and the
    (name, flat offset, transpose) map from its parameters back to the flat
    layout (Conv1D weights are [in, out])."""
    from transformers import GPT2Config, GPT2LMHeadModel
    hc = GPT2Config(vocab_size=cfg.vocab_size, n_positions=cfg.block_size, n_embd=cfg.n_embd,
                    n_layer=cfg.n_layer, n_head=cfg.n_head, resid_pdrop=0.0, embd_pdrop=0.0,
                    attn_pdrop=0.0, layer_norm_epsilon=1e-5, activation_function="gelu_new",
                    bos_token_id=0, eos_token_id=0)
    hc._attn_implementation = "eager"
    model = GPT2LMHeadModel(hc).double().train()
    off = oracle.offsets(cfg)
    names = [("transformer.wte.weight", False), ("transformer.wpe.weight", False)]
    for l in range(cfg.n_layer):
        p = f"transformer.h.{l}."
        names += [(p + "ln_1.weight", False), (p + "ln_1.bias", False),
                  (p + "attn.c_attn.weight", True), (p + "attn.c_attn.bias", False),
                  (p + "attn.c_proj.weight", True), (p + "attn.c_proj.bias", False),
                  (p + "ln_2.weight", False), (p + "ln_2.bias", False),
                  (p + "mlp.c_fc.weight", True), (p + "mlp.c_fc.bias", False),
                  (p + "mlp.c_proj.weight", True), (p + "mlp.c_proj.bias", False)]
    names += [("transformer.ln_f.weight", False), ("transformer.ln_f.bias", False)]
    sd = dict(model.named_parameters())
    layout = []
    with torch.no_grad():
        for (name, tr), o in zip(names, off):
            prm = sd[name]
            n = prm.numel()
            flat = torch.from_numpy(params[o:o + n].astype(np.float64))
            if tr:
                prm.copy_(flat.reshape(prm.shape[1], prm.shape[0]).T)
            else:
                prm.copy_(flat.reshape(prm.shape))
            layout.append((name, int(o), tr, prm))
    assert model.lm_head.weight.data_ptr() == sd["transformer.wte.weight"].data_ptr()
    return model, layout


def _hf_grads(cfg, params, tokens, targets):
    model, layout = _hf_model(cfg, params)
    logits = model(torch.from_numpy(tokens.astype(np.int64))).logits
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, cfg.vocab_size),
                                             torch.from_numpy(targets.reshape(-1).astype(np.int64)))
    loss.backward()
    flat = np.zeros(params.size, np.float64)
    for name, o, tr, prm in layout:
        g = prm.grad.T if tr else prm.grad
        flat[o:o + prm.numel()] = g.contiguous().reshape(-1).numpy()
    return float(loss.detach()), flat, layout


@pytest.mark.parametrize("cfg", [oracle.TINY, oracle.Cfg(2, 2, 128, 300, 64)],
                         ids=["tiny_hs8", "hs64"])
def test_backward_vs_transformers_float64(cfg):
    """Every parameter's gradient (wte gets the lm_head's and the
    embedding's) and the loss, against float64 autograd."""
    params = _randomize_ln_and_biases(cfg, oracle.init_weights(cfg, 42), 6)
    rng = np.random.default_rng(12)
    B, T = 3, min(cfg.block_size, 24)
    tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    targets = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    tr = oracle.Trainer(cfg, params, B, T)
    tr.zero_grad()
    loss = tr.forward(tokens, targets)
    tr.backward()
    ref_loss, ref, layout = _hf_grads(cfg, params, tokens, targets)
    assert abs(loss - ref_loss) < 1e-5 * max(1.0, abs(ref_loss))
    for name, o, _, prm in layout:
        n = prm.numel()
        g, r = tr.grads[o:o + n], ref[o:o + n]
        err = np.abs(g - r).max()
        assert err <= 1e-4 * np.abs(r).max() + 1e-7, (name, err, np.abs(r).max())
    tr.close()


def test_gradient_accumulates_and_zero_grad():
    cfg = oracle.TINY
    params = oracle.init_weights(cfg, 3)
    tok = np.arange(16, dtype=np.int32).reshape(2, 8) % cfg.vocab_size
    tgt = (tok + 1) % cfg.vocab_size
    tr = oracle.Trainer(cfg, params, 2, 8)
    tr.zero_grad()
    tr.forward(tok, tgt)
    tr.backward()
    once = tr.grads.copy()
    tr.forward(tok, tgt)
    tr.backward()
    # (BLAS folds the existing gradient into its own accumulation order)
    np.testing.assert_allclose(tr.grads, 2 * once, rtol=1e-5, atol=1e-6)
    tr.zero_grad()
    assert not tr.grads.any()
    tr.close()


@pytest.mark.parametrize("clip", [0.0, 1.0, 1e-3])
def test_adamw_vs_torch_adamw_float64(clip):
    """Three steps of gpt_adamw against torch.optim.AdamW (float64) on the
    same gradients: decay groups by tensor dimension, bias corrections, the
    global-norm clip (applied to the gradients first, as
    src/model.c:893-900 does)."""
    cfg = oracle.Cfg(2, 2, 32, 50, 16)
    rng = np.random.default_rng(4)
    params = _randomize_ln_and_biases(cfg, oracle.init_weights(cfg, 9), 10)
    model, layout = _hf_model(cfg, params)
    decay = [p for name, o, tr, p in layout if p.dim() >= 2]
    nodecay = [p for name, o, tr, p in layout if p.dim() < 2]
    opt = torch.optim.AdamW([{"params": decay, "weight_decay": 0.1},
                             {"params": nodecay, "weight_decay": 0.0}],
                            lr=3e-3, betas=(0.9, 0.95), eps=1e-8)
    tr = oracle.Trainer(cfg, params, 1, 4)
    for step in range(3):
        g = (rng.standard_normal(params.size) * 0.05).astype(np.float32)
        tr.grads[:] = g
        tr.adamw(3e-3, 0.9, 0.95, 1e-8, 0.1, clip)
        g64 = g.astype(np.float64)
        norm = np.sqrt((g64 ** 2).sum())
        if clip > 0 and norm > clip:
            g64 = g64 * (clip / norm)
        for name, o, trn, prm in layout:
            gg = torch.from_numpy(g64[o:o + prm.numel()].copy())
            prm.grad = (gg.reshape(prm.shape[1], prm.shape[0]).T if trn
                        else gg.reshape(prm.shape)).contiguous()
        opt.step()
    got = tr.params
    for name, o, trn, prm in layout:
        ref = (prm.detach().T if trn else prm.detach()).contiguous().reshape(-1).numpy()
        err = np.abs(got[o:o + prm.numel()] - ref).max()
        assert err < 2e-6, (name, err)
    tr.close()
