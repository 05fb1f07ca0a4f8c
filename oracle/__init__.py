"""CPU oracle for cngpt's inference forward pass -- TEST INFRASTRUCTURE ONLY.

The C library built from ``oracle/cngpt_oracle.c`` restates the reference's
``gpt_forward_fast`` (src/fast.c:227-333), its all-rows variant (the
semantics of ``gpt_forward``, src/model.c:442-625), the forward ops of
src/ops.c, the seeded init (src/model.c:275-331) and ``sample_top_k``
(src/model.c:927-989). This module is a ctypes front end to it.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline; the product (``cngpt_amd``) never does.
"""
from __future__ import annotations

import ctypes
import glob
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcngpt_oracle.so")

LAST, ALL = 0, 1


class OrcCfg(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_embd", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("block_size", ctypes.c_int)]


@dataclass(frozen=True)
class Cfg:
    n_layer: int
    n_head: int
    n_embd: int
    vocab_size: int
    block_size: int

    def c(self) -> OrcCfg:
        return OrcCfg(self.n_layer, self.n_head, self.n_embd, self.vocab_size,
                      self.block_size)


# Model shapes: the tiny model of tests/check_fast.c:29-33 and GPT-2 sizes.
TINY = Cfg(3, 4, 32, 70, 16)
GPT2_SMALL = Cfg(12, 12, 768, 50257, 1024)
GPT2_MEDIUM = Cfg(24, 16, 1024, 50257, 1024)
GPT2_XL = Cfg(48, 25, 1600, 50257, 1024)

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)
_L = ctypes.POINTER(ctypes.c_long)
_lib = None


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_I)


def find_openblas() -> str | None:
    """Path of a CBLAS-compatible OpenBLAS on this host: the one bundled in
    scipy's wheel, else a system libopenblas."""
    try:
        import scipy
        d = os.path.join(os.path.dirname(os.path.dirname(scipy.__file__)), "scipy.libs")
        hits = sorted(glob.glob(os.path.join(d, "libscipy_openblas*.so")))
        if hits:
            return hits[0]
    except ImportError:
        pass
    for p in ("/usr/lib/x86_64-linux-gnu/libopenblas.so.0", "/usr/lib/libopenblas.so"):
        if os.path.exists(p):
            return p
    return None


def lib():
    """Load the oracle library (built by oracle/Makefile) and bind a CBLAS."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library not built: {LIB_PATH} (run make -C oracle)")
    L = ctypes.CDLL(LIB_PATH)
    L.orc_num_params.argtypes = [ctypes.POINTER(OrcCfg)]
    L.orc_num_params.restype = ctypes.c_long
    L.orc_offsets.argtypes = [ctypes.POINTER(OrcCfg), _L]
    L.orc_init_weights.argtypes = [ctypes.POINTER(OrcCfg), _F, ctypes.c_uint]
    L.orc_use_blas.argtypes = [ctypes.c_char_p]
    L.orc_use_blas.restype = ctypes.c_int
    L.orc_blas_info.restype = ctypes.c_char_p
    L.orc_set_threads.argtypes = [ctypes.c_int]
    L.orc_set_threads.restype = ctypes.c_int
    L.orc_physical_cores.restype = ctypes.c_int
    L.orc_layernorm.argtypes = [_F, _F, _F, _F, _F, _F, ctypes.c_int, ctypes.c_int]
    L.orc_gelu.argtypes = [_F, _F, ctypes.c_int]
    L.orc_softmax_inplace.argtypes = [_F, ctypes.c_int, ctypes.c_int]
    L.orc_causal_mask.argtypes = [_F, ctypes.c_int]
    L.orc_linear.argtypes = [_F, _F, _F, _F, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.orc_forward.argtypes = [ctypes.POINTER(OrcCfg), _F, _I, ctypes.c_int,
                              ctypes.c_int, ctypes.c_int, _F]
    L.orc_forward.restype = ctypes.c_int
    L.orc_sample_top_k.argtypes = [_F, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                   ctypes.c_float]
    L.orc_sample_top_k.restype = ctypes.c_int
    L.orc_cross_entropy.argtypes = [_F, _I, _F, _F, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int]
    L.orc_cross_entropy.restype = ctypes.c_float
    L.orc_srand.argtypes = [ctypes.c_uint]
    L.orc_rand_uniform.restype = ctypes.c_float
    i = ctypes.c_int
    L.orc_linear_bwd_dx.argtypes = [_F, _F, _F, i, i, i]
    L.orc_linear_bwd_dw.argtypes = [_F, _F, _F, _F, i, i, i]
    L.orc_layernorm_bwd.argtypes = [_F, _F, _F, _F, _F, _F, _F, _F, i, i]
    L.orc_gelu_bwd.argtypes = [_F, _F, _F, i]
    L.orc_train_new.argtypes = [ctypes.POINTER(OrcCfg), i, i]
    L.orc_train_new.restype = ctypes.c_void_p
    L.orc_train_free.argtypes = [ctypes.c_void_p]
    L.orc_train_forward.argtypes = [ctypes.c_void_p, _F, _I, _I]
    L.orc_train_forward.restype = ctypes.c_float
    L.orc_train_backward.argtypes = [ctypes.c_void_p, _F, _I, _I, _F]
    L.orc_train_set_dropout.argtypes = [ctypes.c_void_p, ctypes.c_float]
    L.orc_train_masks.argtypes = [ctypes.c_void_p]
    L.orc_train_masks.restype = ctypes.POINTER(ctypes.c_ubyte)
    L.orc_dropout_fwd.argtypes = [_F, ctypes.POINTER(ctypes.c_ubyte), ctypes.c_long, ctypes.c_float]
    L.orc_adamw.argtypes = [ctypes.POINTER(OrcCfg), _F, _F, _F, _F, i, ctypes.c_float,
                            ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                            ctypes.c_float]
    blas = os.environ.get("CNGPT_ORACLE_BLAS") or find_openblas()
    if blas and blas != "builtin":
        L.orc_use_blas(blas.encode())
    _lib = L
    return L


def blas_info() -> str:
    return lib().orc_blas_info().decode()


def set_threads(n: int = 0) -> int:
    return lib().orc_set_threads(n)


def physical_cores() -> int:
    return lib().orc_physical_cores()


def num_params(cfg: Cfg) -> int:
    return lib().orc_num_params(ctypes.byref(cfg.c()))


def offsets(cfg: Cfg) -> np.ndarray:
    off = np.zeros(4 + 12 * cfg.n_layer, dtype=np.int64)
    lib().orc_offsets(ctypes.byref(cfg.c()), off.ctypes.data_as(_L))
    return off


def init_weights(cfg: Cfg, seed: int) -> np.ndarray:
    p = np.zeros(num_params(cfg), dtype=np.float32)
    lib().orc_init_weights(ctypes.byref(cfg.c()), _fp(p), seed)
    return p


def unpack(cfg: Cfg, params: np.ndarray) -> dict:
    """Named views into the flat buffer (layout of src/model.c:54-83)."""
    C, V, T = cfg.n_embd, cfg.vocab_size, cfg.block_size
    off = offsets(cfg)
    shapes = [(C,), (C,), (3 * C, C), (3 * C,), (C, C), (C,), (C,), (C,),
              (4 * C, C), (4 * C,), (C, 4 * C), (C,)]
    names = ["ln1_w", "ln1_b", "c_attn_w", "c_attn_b", "c_proj_w", "c_proj_b",
             "ln2_w", "ln2_b", "mlp_fc_w", "mlp_fc_b", "mlp_proj_w", "mlp_proj_b"]

    def view(o, shape):
        n = int(np.prod(shape))
        return params[o:o + n].reshape(shape)

    d = {"wte": view(off[0], (V, C)), "wpe": view(off[1], (T, C)), "layers": []}
    for l in range(cfg.n_layer):
        o = off[2 + 12 * l: 2 + 12 * (l + 1)]
        d["layers"].append({n: view(o[i], s) for i, (n, s) in enumerate(zip(names, shapes))})
    of = off[2 + 12 * cfg.n_layer:]
    d["ln_f_w"] = view(of[0], (C,))
    d["ln_f_b"] = view(of[1], (C,))
    return d


def forward(cfg: Cfg, params: np.ndarray, tokens: np.ndarray, mode: int = LAST) -> np.ndarray:
    """LAST: logits [B, V] (gpt_forward_fast); ALL: logits [B, T, V]."""
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    B, T = tokens.shape
    shape = (B, cfg.vocab_size) if mode == LAST else (B, T, cfg.vocab_size)
    out = np.empty(shape, dtype=np.float32)
    rc = lib().orc_forward(ctypes.byref(cfg.c()), _fp(params), _ip(tokens), B, T, mode, _fp(out))
    if rc != 0:
        raise ValueError(f"orc_forward failed (B={B}, T={T})")
    return out


def layernorm(x, w, b):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, C = x.shape
    out = np.empty_like(x)
    mean = np.empty(T, np.float32)
    rstd = np.empty(T, np.float32)
    lib().orc_layernorm(_fp(x), _fp(np.ascontiguousarray(w, np.float32)),
                        _fp(np.ascontiguousarray(b, np.float32)), _fp(out), _fp(mean),
                        _fp(rstd), T, C)
    return out, mean, rstd


def gelu(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_gelu(_fp(x), _fp(out), x.size)
    return out


def softmax(x):
    x = np.array(x, dtype=np.float32, order="C")
    rows, cols = x.shape
    lib().orc_softmax_inplace(_fp(x), rows, cols)
    return x


def causal_mask(s):
    s = np.array(s, dtype=np.float32, order="C")
    lib().orc_causal_mask(_fp(s), s.shape[0])
    return s


def linear(X, W, b=None):
    X = np.ascontiguousarray(X, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, K = X.shape
    N = W.shape[0]
    Y = np.empty((M, N), np.float32)
    bp = _fp(np.ascontiguousarray(b, np.float32)) if b is not None else None
    lib().orc_linear(_fp(X), _fp(W), bp, _fp(Y), M, K, N)
    return Y


def sample_top_k(logits, temp: float, top_k: int, r: float) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().orc_sample_top_k(_fp(logits), logits.size, temp, top_k, r)


def cross_entropy(logits, targets, want_probs: bool = False):
    """cross_entropy_fwd (src/ops.c:499-574) over logits [..., V] and
    targets [...]: (mean loss, per-row loss, probs or None)."""
    logits = np.ascontiguousarray(logits, np.float32)
    V = logits.shape[-1]
    rows = logits.size // V
    targets = np.ascontiguousarray(targets, np.int32).reshape(-1)
    assert targets.size == rows and (rows == 0 or (targets.min() >= 0 and targets.max() < V))
    row_loss = np.empty(rows, np.float32)
    probs = np.empty((rows, V), np.float32) if want_probs else None
    loss = lib().orc_cross_entropy(_fp(logits), _ip(targets),
                                   _fp(probs) if want_probs else None, _fp(row_loss), 1, rows, V)
    return float(loss), row_loss, probs


def srand(seed: int) -> None:
    lib().orc_srand(seed)


def rand_uniform() -> float:
    return lib().orc_rand_uniform()


def lcg_tokens(n: int, vocab: int, seed: int = 12345) -> np.ndarray:
    """Token ids from the LCG of src/cngpt.c:338-342."""
    out = np.empty(n, dtype=np.int32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (s >> 8) % vocab
    return out


# ---------------------------------------------------------------- training

def linear_bwd_dx(dY, W, dX=None):
    """linear_bwd_dx (src/ops.c:125-133): dX [M,K] += dY [M,N] . W [N,K]."""
    dY = np.ascontiguousarray(dY, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, N = dY.shape
    K = W.shape[1]
    dX = np.zeros((M, K), np.float32) if dX is None else np.array(dX, np.float32, order="C")
    lib().orc_linear_bwd_dx(_fp(dY), _fp(W), _fp(dX), M, K, N)
    return dX


def linear_bwd_dw(dY, X, dW=None, db=None):
    """linear_bwd_dw (src/ops.c:135-153): dW [N,K] += dY^T X, db += sum_rows dY."""
    dY = np.ascontiguousarray(dY, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    M, N = dY.shape
    K = X.shape[1]
    dW = np.zeros((N, K), np.float32) if dW is None else np.array(dW, np.float32, order="C")
    db = np.zeros(N, np.float32) if db is None else np.array(db, np.float32, order="C")
    lib().orc_linear_bwd_dw(_fp(dY), _fp(X), _fp(dW), _fp(db), M, K, N)
    return dW, db


def layernorm_bwd(dout, x, w, mean, rstd):
    """layernorm_bwd (src/ops.c:250-331) into zeroed dx, dw, db."""
    dout = np.ascontiguousarray(dout, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    T, C = x.shape
    dx = np.zeros_like(x)
    dw = np.zeros(C, np.float32)
    db = np.zeros(C, np.float32)
    lib().orc_layernorm_bwd(_fp(dout), _fp(x), _fp(np.ascontiguousarray(w, np.float32)),
                            _fp(np.ascontiguousarray(mean, np.float32)),
                            _fp(np.ascontiguousarray(rstd, np.float32)), _fp(dx), _fp(dw),
                            _fp(db), T, C)
    return dx, dw, db


def gelu_bwd(dout, x):
    """gelu_bwd (src/ops.c:382-422) into a zeroed dx."""
    dout = np.ascontiguousarray(dout, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    dx = np.zeros_like(x)
    lib().orc_gelu_bwd(_fp(dout), _fp(x), _fp(dx), x.size)
    return dx


class Trainer:
    """The reference's training step on the CPU: gpt_forward with targets,
    gpt_backward and gpt_adamw (src/model.c:442-921), over params, grads, m,
    v arrays of the flat layout."""

    def __init__(self, cfg: Cfg, params: np.ndarray, B: int, T: int):
        self.cfg, self.B, self.T = cfg, B, T
        self.params = np.array(params, np.float32, order="C")
        n = self.params.size
        self.grads = np.zeros(n, np.float32)
        self.m = np.zeros(n, np.float32)
        self.v = np.zeros(n, np.float32)
        self.step = 0
        self._t = lib().orc_train_new(ctypes.byref(cfg.c()), B, T)
        if not self._t:
            raise ValueError("orc_train_new failed")

    def close(self):
        if getattr(self, "_t", None):
            lib().orc_train_free(self._t)
            self._t = None

    def __del__(self):
        self.close()

    def zero_grad(self):                                # model.c:879-886
        self.grads[:] = 0

    def set_dropout(self, p: float) -> None:
        """GPTConfig.dropout: the residual-stream dropout of the training
        forwards (model.c:450-472, 572-599), rand() draws in model.c's order."""
        if lib().orc_train_set_dropout(self._t, p) != 0:
            raise ValueError(f"dropout rate {p} outside [0, 1)")
        self.dropout = p

    def masks(self) -> np.ndarray:
        """The last forward's keep masks, [1 + 2 L, B T C] (the embedding,
        then res1 and res2 of each layer)."""
        n = (1 + 2 * self.cfg.n_layer) * self.B * self.T * self.cfg.n_embd
        return np.ctypeslib.as_array(lib().orc_train_masks(self._t), shape=(n,)).reshape(
            1 + 2 * self.cfg.n_layer, -1).copy()

    def forward(self, tokens, targets) -> float:        # model.c:442-625
        """The loss, or 0 with targets None (no loss, no dropout)."""
        tokens = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        if targets is not None:
            targets = np.ascontiguousarray(targets, np.int32).reshape(-1)
        self._tok, self._tgt = tokens, targets
        tp = _ip(targets) if targets is not None else None
        return float(lib().orc_train_forward(self._t, _fp(self.params), _ip(tokens), tp))

    def backward(self):                                 # model.c:634-877
        lib().orc_train_backward(self._t, _fp(self.params), _ip(self._tok), _ip(self._tgt),
                                 _fp(self.grads))

    def adamw(self, lr, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1, grad_clip=1.0):
        self.step += 1                                  # model.c:888-921
        lib().orc_adamw(ctypes.byref(self.cfg.c()), _fp(self.params), _fp(self.grads),
                        _fp(self.m), _fp(self.v), self.step, lr, beta1, beta2, eps, wd,
                        grad_clip)
