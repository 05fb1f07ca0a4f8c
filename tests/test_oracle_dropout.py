"""Pins for the oracle's training dropout (GPTConfig.dropout: dropout_fwd /
dropout_bwd of src/ops.c:603-625 on the residual stream at src/model.c:471-472,
572-574, 597-599 and backward at :699-700, :732-733, :849-850) -- no GPU.

The masks are checked against the C library's rand() called directly (the
draw order of model.c: the embedding, then res1 and res2 of each layer), and
the loss and every parameter's gradient against float64 autograd through a
torch restatement of model.c's forward that multiplies the same masks in at
the same three places (and, with no masks, agrees with the oracle's
dropout-free step, itself pinned against transformers' GPT2LMHeadModel).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from test_oracle import _randomize_ln_and_biases

LIBC = ctypes.CDLL(None)
LIBC.rand.restype = ctypes.c_int
RAND_MAX = 2147483647


def _libc_masks(seed, n, p):
    """srand(seed), then n draws kept when rand() > (unsigned)(p * RAND_MAX)
    with the product in float (ops.c:611-613)."""
    LIBC.srand(seed)
    thr = int(np.float32(p) * np.float32(RAND_MAX))
    return np.array([LIBC.rand() > thr for _ in range(n)], np.uint8)


def _torch_step(cfg, params, tokens, targets, masks, p):
    """Loss and flat float64 gradients of model.c's forward, the keep masks
    (keep ? 1 / (1 - p) : 0) multiplied into the embedding, res1 and res2."""
    C, H, L, V = cfg.n_embd, cfg.n_head, cfg.n_layer, cfg.vocab_size
    hs = C // H
    B, T = tokens.shape
    off = oracle.offsets(cfg)
    shapes = [(C,), (C,), (3 * C, C), (3 * C,), (C, C), (C,), (C,), (C,),
              (4 * C, C), (4 * C,), (C, 4 * C), (C,)]
    leaves = []

    def leaf(o, shape):
        n = int(np.prod(shape))
        t = torch.tensor(params[o:o + n].astype(np.float64).reshape(shape), requires_grad=True)
        leaves.append((int(o), t))
        return t

    wte, wpe = leaf(off[0], (V, C)), leaf(off[1], (cfg.block_size, C))
    layers = [[leaf(off[2 + 12 * l + i], shapes[i]) for i in range(12)] for l in range(L)]
    lnf_w, lnf_b = leaf(off[2 + 12 * L], (C,)), leaf(off[3 + 12 * L], (C,))
    scale = 1.0 / (1.0 - np.float64(np.float32(p))) if masks is not None else 1.0

    def drop(x, i):
        if masks is None:
            return x
        m = torch.from_numpy(masks[i].reshape(B, T, C).astype(np.float64)) * scale
        return x * m

    def ln(x, w, b):
        return torch.nn.functional.layer_norm(x, (C,), w, b, 1e-5)

    tok = torch.from_numpy(tokens.astype(np.int64))
    x = drop(wte[tok] + wpe[:T], 0)
    causal = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    for l, (l1w, l1b, aw, ab, pw, pb, l2w, l2b, fw, fb, mw, mb) in enumerate(layers):
        qkv = ln(x, l1w, l1b) @ aw.T + ab
        q, k, v = (qkv[..., i * C:(i + 1) * C].reshape(B, T, H, hs).transpose(1, 2)
                   for i in range(3))
        att = (q @ k.transpose(-1, -2)) / np.sqrt(hs)
        att = torch.softmax(att.masked_fill(causal, float("-inf")), -1)
        o = (att @ v).transpose(1, 2).reshape(B, T, C)
        res1 = drop(x + (o @ pw.T + pb), 1 + 2 * l)
        f = torch.nn.functional.gelu(ln(res1, l2w, l2b) @ fw.T + fb, approximate="tanh")
        x = drop(res1 + (f @ mw.T + mb), 2 + 2 * l)
    logits = ln(x, lnf_w, lnf_b) @ wte.T
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, V),
                                             torch.from_numpy(targets.reshape(-1).astype(np.int64)))
    loss.backward()
    flat = np.zeros(params.size, np.float64)
    for o, t in leaves:
        flat[o:o + t.numel()] = t.grad.reshape(-1).numpy()
    return float(loss.detach()), flat, leaves


def test_dropout_masks_are_the_rand_draws_in_model_order():
    """The masks of a training forward are libc rand() draws after srand,
    in model.c's order, and the forward scales kept values by 1 / (1 - p)."""
    cfg = oracle.TINY
    params = oracle.init_weights(cfg, 5)
    B, T, p = 2, 8, 0.25
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    targets = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    tr = oracle.Trainer(cfg, params, B, T)
    tr.set_dropout(p)
    oracle.srand(123)
    tr.forward(tokens, targets)
    masks = tr.masks()
    n = masks.size
    ref = _libc_masks(123, n, p).reshape(masks.shape)
    assert np.array_equal(masks, ref)
    assert abs(masks.mean() - (1 - p)) < 0.05
    # a forward without targets draws nothing and applies no dropout
    LIBC.srand(9)
    before = LIBC.rand()
    LIBC.srand(9)
    tr.forward(tokens, None)
    assert LIBC.rand() == before
    tr.close()


@pytest.mark.parametrize("p", [0.0, 0.1, 0.5])
def test_dropout_backward_vs_torch_float64(p):
    """Loss and every parameter's gradient of the step with dropout against
    float64 autograd with the oracle's masks at model.c's three sites."""
    cfg = oracle.Cfg(2, 2, 32, 50, 16)
    params = _randomize_ln_and_biases(cfg, oracle.init_weights(cfg, 21), 8)
    rng = np.random.default_rng(17)
    B, T = 3, 12
    tokens = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    targets = rng.integers(0, cfg.vocab_size, size=(B, T), dtype=np.int32)
    tr = oracle.Trainer(cfg, params, B, T)
    tr.set_dropout(p)
    tr.zero_grad()
    oracle.srand(77)
    loss = tr.forward(tokens, targets)
    tr.backward()
    masks = tr.masks() if p > 0 else None
    ref_loss, ref, leaves = _torch_step(cfg, params, tokens, targets, masks, p)
    assert abs(loss - ref_loss) < 1e-5 * max(1.0, abs(ref_loss))
    for o, t in leaves:
        n = t.numel()
        g, r = tr.grads[o:o + n], ref[o:o + n]
        err = np.abs(g - r).max()
        assert err <= 1e-4 * np.abs(r).max() + 1e-7, (o, err, np.abs(r).max())
    tr.close()
