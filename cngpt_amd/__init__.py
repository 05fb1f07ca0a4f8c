"""cngpt_amd: GPT-2 inference forward pass on an MI355X (gfx950).

Python front end over the C ABI of ``libcngpt_hip.so`` (declared in
``include/cngpt_hip.h``). The compute path is the hand-written HIP kernels in
``cngpt_amd/csrc``; this module only moves host arrays across the boundary.
There is no CPU fallback: if the library is missing, loading it raises.

Mirrors the reference's inference interface:
  ``Model.forward(tokens)``           gpt_forward_fast (src/fast.c:227-333)
  ``Model.forward(tokens, ALL)``      all-position logits (src/model.c:612-614)
  ``Model.loss(tokens, targets)``     gpt_forward with targets: logits and the
                                      cross_entropy_fwd loss (src/model.c:617-623)
  ``init_weights(cfg, seed)``         gpt_init_weights after srand(seed)
  ``load_weights / save_weights``     the weight file of src/model.c:177-231
"""
from __future__ import annotations

import ctypes
import os
import struct
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcngpt_hip.so")

LAST, ALL = 0, 1
(K_GEMM, K_GEMV, K_ATTN, K_ATTN_ROW, K_LAYERNORM, K_EMBED, K_GATHER, K_ARGMAX,
 K_SAMPLE, K_STEP, K_LOSS) = range(11)
KERNEL_CLASSES = ["gemm", "gemv", "attn", "attn_row", "layernorm", "embed", "gather", "argmax",
                  "sample", "step", "loss"]
# decode paths (include/cngpt_hip.h)
DECODE_AUTO, DECODE_KERNELS, DECODE_PERSISTENT = 0, 1, 2

MAGIC = 0x434E4750
VERSION = 1


class CngptError(RuntimeError):
    pass


class _Cfg(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_embd", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("block_size", ctypes.c_int)]


@dataclass(frozen=True)
class Config:
    n_layer: int
    n_head: int
    n_embd: int
    vocab_size: int
    block_size: int

    def _c(self) -> _Cfg:
        return _Cfg(self.n_layer, self.n_head, self.n_embd, self.vocab_size, self.block_size)


# GPT-2 shapes and the tiny model of the reference's tests/check_fast.c:29-33.
TINY = Config(3, 4, 32, 70, 16)
GPT2_SMALL = Config(12, 12, 768, 50257, 1024)
GPT2_MEDIUM = Config(24, 16, 1024, 50257, 1024)
GPT2_XL = Config(48, 25, 1600, 50257, 1024)

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)
_D = ctypes.POINTER(ctypes.c_double)
_Lp = ctypes.POINTER(ctypes.c_long)
_VP = ctypes.c_void_p

# Every symbol include/cngpt_hip.h, fast.h and model.h declare.
EXPORTS = [
    "cngpt_hip_last_error", "cngpt_hip_create", "cngpt_hip_destroy", "cngpt_hip_num_params",
    "cngpt_hip_load_params", "cngpt_hip_file_config", "cngpt_hip_load_file",
    "cngpt_hip_reserve", "cngpt_hip_forward",
    "cngpt_hip_upload_tokens", "cngpt_hip_forward_resident", "cngpt_hip_forward_noalloc",
    "cngpt_hip_synchronize",
    "cngpt_hip_read_logits", "cngpt_hip_logits_device", "cngpt_hip_cross_entropy",
    "cngpt_hip_upload_targets", "cngpt_hip_cross_entropy_resident", "cngpt_hip_read_loss",
    "cngpt_hip_decode_begin",
    "cngpt_hip_decode_step", "cngpt_hip_generate", "cngpt_hip_argmax", "cngpt_hip_sample",
    "cngpt_hip_decode_length", "cngpt_hip_set_decode_path", "cngpt_hip_decode_path",
    "cngpt_hip_profile_enable", "cngpt_hip_profile_reset", "cngpt_hip_profile_read",
    "cngpt_hip_host_alloc", "cngpt_hip_host_free", "cngpt_hip_init_weights",
    "cngpt_hip_train_create", "cngpt_hip_train_destroy", "cngpt_hip_train_forward",
    "cngpt_hip_train_backward", "cngpt_hip_train_zero_grad", "cngpt_hip_train_adamw",
    "cngpt_hip_train_read", "cngpt_hip_train_write", "cngpt_hip_train_steps",
    "cngpt_hip_train_set_dropout",
    "fast_init", "fast_free", "fast_set_threads", "gpt_forward_fast", "gpt_forward_fast_all",
    "fast_params_changed", "fast_last_error",
    "gpt_num_params", "gpt_init", "gpt_init_weights", "gpt_load", "gpt_save", "gpt_free",
]

_lib = None


def lib():
    """Load libcngpt_hip.so (built by __graft_entry__.build()); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise CngptError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    L.cngpt_hip_last_error.restype = ctypes.c_char_p
    L.cngpt_hip_create.argtypes = [ctypes.c_int, ctypes.POINTER(_VP)]
    L.cngpt_hip_destroy.argtypes = [_VP]
    L.cngpt_hip_destroy.restype = None
    L.cngpt_hip_num_params.argtypes = [ctypes.POINTER(_Cfg)]
    L.cngpt_hip_num_params.restype = ctypes.c_long
    L.cngpt_hip_load_params.argtypes = [_VP, ctypes.POINTER(_Cfg), _F, ctypes.c_long]
    L.cngpt_hip_file_config.argtypes = [ctypes.c_char_p, ctypes.POINTER(_Cfg), _Lp]
    L.cngpt_hip_load_file.argtypes = [_VP, ctypes.c_char_p, ctypes.POINTER(_Cfg)]
    L.cngpt_hip_reserve.argtypes = [_VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.cngpt_hip_forward.argtypes = [_VP, _I, ctypes.c_int, ctypes.c_int, ctypes.c_int, _F]
    L.cngpt_hip_upload_tokens.argtypes = [_VP, _I, ctypes.c_int, ctypes.c_int]
    L.cngpt_hip_forward_resident.argtypes = [_VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.cngpt_hip_forward_noalloc.argtypes = [_VP, _VP, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            _VP, _VP]
    L.cngpt_hip_synchronize.argtypes = [_VP]
    L.cngpt_hip_read_logits.argtypes = [_VP, ctypes.c_size_t, ctypes.c_size_t, _F]
    L.cngpt_hip_logits_device.argtypes = [_VP]
    L.cngpt_hip_logits_device.restype = _VP
    L.cngpt_hip_cross_entropy.argtypes = [_VP, _I, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          _F, _F]
    L.cngpt_hip_upload_targets.argtypes = [_VP, _I, ctypes.c_int, ctypes.c_int]
    L.cngpt_hip_cross_entropy_resident.argtypes = [_VP, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_int]
    L.cngpt_hip_read_loss.argtypes = [_VP, _F, _F]
    L.cngpt_hip_decode_begin.argtypes = [_VP, _I, ctypes.c_int, ctypes.c_int, ctypes.c_int, _F]
    L.cngpt_hip_decode_step.argtypes = [_VP, _I, _F]
    L.cngpt_hip_generate.argtypes = [_VP, ctypes.c_int, ctypes.c_float, ctypes.c_int, _F, _I]
    L.cngpt_hip_argmax.argtypes = [_VP, _I]
    L.cngpt_hip_sample.argtypes = [_VP, ctypes.c_float, ctypes.c_int, _F, _I]
    L.cngpt_hip_decode_length.argtypes = [_VP]
    L.cngpt_hip_set_decode_path.argtypes = [_VP, ctypes.c_int]
    L.cngpt_hip_decode_path.argtypes = [_VP]
    L.cngpt_hip_profile_enable.argtypes = [_VP, ctypes.c_int]
    L.cngpt_hip_profile_reset.argtypes = [_VP]
    L.cngpt_hip_profile_read.argtypes = [_VP, ctypes.c_int, _D, _Lp, _D, _D]
    L.cngpt_hip_host_alloc.argtypes = [ctypes.c_size_t]
    L.cngpt_hip_host_alloc.restype = _VP
    L.cngpt_hip_host_free.argtypes = [_VP]
    L.cngpt_hip_host_free.restype = None
    L.cngpt_hip_init_weights.argtypes = [ctypes.POINTER(_Cfg), _F, ctypes.c_uint]
    L.cngpt_hip_train_create.argtypes = [_VP, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_VP)]
    L.cngpt_hip_train_destroy.argtypes = [_VP]
    L.cngpt_hip_train_destroy.restype = None
    L.cngpt_hip_train_forward.argtypes = [_VP, _I, _I, _F]
    L.cngpt_hip_train_backward.argtypes = [_VP]
    L.cngpt_hip_train_zero_grad.argtypes = [_VP]
    L.cngpt_hip_train_set_dropout.argtypes = [_VP, ctypes.c_float]
    L.cngpt_hip_train_adamw.argtypes = [_VP] + [ctypes.c_float] * 6 + [_F]
    L.cngpt_hip_train_read.argtypes = [_VP, ctypes.c_int, _F, ctypes.c_long]
    L.cngpt_hip_train_write.argtypes = [_VP, ctypes.c_int, _F, ctypes.c_long]
    L.cngpt_hip_train_steps.argtypes = [_VP]
    _lib = L
    return L


def _err() -> str:
    return lib().cngpt_hip_last_error().decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise CngptError(f"{what}: {_err()}")


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_I)


def num_params(cfg: Config) -> int:
    n = lib().cngpt_hip_num_params(ctypes.byref(cfg._c()))
    if n < 0:
        raise CngptError(f"invalid shape {cfg}")
    return n


def init_weights(cfg: Config, seed: int) -> np.ndarray:
    """Seeded synthetic weights (srand(seed); gpt_init_weights order)."""
    p = np.empty(num_params(cfg), dtype=np.float32)
    _check(lib().cngpt_hip_init_weights(ctypes.byref(cfg._c()), _fp(p), seed), "init_weights")
    return p


def save_weights(path: str, cfg: Config, params: np.ndarray) -> None:
    """Write the reference's weight file: 7 int32 header + flat fp32."""
    with open(path, "wb") as f:
        f.write(struct.pack("<7i", MAGIC, VERSION, cfg.n_layer, cfg.n_head, cfg.n_embd,
                            cfg.vocab_size, cfg.block_size))
        f.write(np.ascontiguousarray(params, np.float32).tobytes())


def load_weights(path: str) -> tuple[Config, np.ndarray]:
    """Read a weight file (memory-mapped), checking magic and length."""
    with open(path, "rb") as f:
        hdr = f.read(28)
    if len(hdr) < 28:
        raise CngptError(f"{path}: file ends inside its 28-byte header")
    magic, _ver, L, H, C, V, T = struct.unpack("<7i", hdr)
    if magic != MAGIC:
        raise CngptError(f"{path}: not a cngpt weight file (first word 0x{magic & 0xFFFFFFFF:X})")
    cfg = Config(L, H, C, V, T)
    n = num_params(cfg)
    p = np.memmap(path, dtype=np.float32, mode="r", offset=28)
    if p.size < n:
        raise CngptError(f"{path}: file ends before its parameters ({p.size} of {n} floats)")
    return cfg, np.ascontiguousarray(p[:n])


def file_config(path: str) -> tuple[Config, int]:
    """Shape and parameter count of a weight file, validated without a GPU
    (cngpt_hip_file_config)."""
    c = _Cfg()
    n = ctypes.c_long()
    _check(lib().cngpt_hip_file_config(os.fsencode(path), ctypes.byref(c), ctypes.byref(n)),
           "file_config")
    return Config(c.n_layer, c.n_head, c.n_embd, c.vocab_size, c.block_size), n.value


class Model:
    """One device handle: parameters in one allocation, activations in another."""

    def __init__(self, cfg: Config | None, params: np.ndarray | None, device: int = 0):
        L = lib()
        h = _VP()
        _check(L.cngpt_hip_create(device, ctypes.byref(h)), "create")
        self._h = h
        self.cfg = cfg
        self.decode_batch = 0
        if params is not None:
            self.load_params(params)

    @classmethod
    def from_file(cls, path: str, device: int = 0) -> "Model":
        """A handle whose parameters are streamed from a weight file straight
        to the device (cngpt_hip_load_file; no host copy of the buffer)."""
        m = cls(None, None, device)
        try:
            m.load_file(path)
        except Exception:
            m.close()
            raise
        return m

    def load_file(self, path: str) -> Config:
        c = _Cfg()
        _check(lib().cngpt_hip_load_file(self._h, os.fsencode(path), ctypes.byref(c)),
               "load_file")
        self.cfg = Config(c.n_layer, c.n_head, c.n_embd, c.vocab_size, c.block_size)
        return self.cfg

    def load_params(self, params: np.ndarray) -> None:
        params = np.ascontiguousarray(params, dtype=np.float32)
        _check(lib().cngpt_hip_load_params(self._h, ctypes.byref(self.cfg._c()), _fp(params),
                                           params.size), "load_params")

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().cngpt_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- forward --------------------------------------------------------
    def forward(self, tokens, mode: int = LAST, copy: bool = True):
        """tokens [B, T] -> logits [B, V] (LAST) or [B, T, V] (ALL).
        With copy=False (ALL) the logits stay on the device."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, T = tokens.shape
        V = self.cfg.vocab_size
        out = None
        if copy:
            out = np.empty((B, V) if mode == LAST else (B, T, V), dtype=np.float32)
        _check(lib().cngpt_hip_forward(self._h, _ip(tokens), B, T, mode,
                                       _fp(out) if out is not None else None), "forward")
        return out

    def reserve(self, B: int, T: int, mode: int = LAST, kv_capacity: int = 0) -> None:
        _check(lib().cngpt_hip_reserve(self._h, B, T, mode, kv_capacity), "reserve")

    def upload_tokens(self, tokens) -> None:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        _check(lib().cngpt_hip_upload_tokens(self._h, _ip(tokens), *tokens.shape), "upload")

    def forward_resident(self, B: int, T: int, mode: int = LAST) -> None:
        _check(lib().cngpt_hip_forward_resident(self._h, B, T, mode), "forward_resident")

    def forward_noalloc(self, tokens_dev: int, B: int, T: int, mode: int, logits_dev: int,
                        err_dev: int | None = None) -> None:
        """cngpt_hip_forward_noalloc: device tokens [B, T] -> device logits,
        activations in the library's scratch (no allocation); enqueued."""
        _check(lib().cngpt_hip_forward_noalloc(self._h, tokens_dev, B, T, mode, logits_dev,
                                               err_dev), "forward_noalloc")

    def synchronize(self) -> None:
        _check(lib().cngpt_hip_synchronize(self._h), "synchronize")

    def read_logits(self, offset: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        _check(lib().cngpt_hip_read_logits(self._h, offset, count, _fp(out)), "read_logits")
        return out

    # -- loss -----------------------------------------------------------
    def cross_entropy(self, targets, probs: bool = False, rows: bool = False):
        """Cross-entropy of the held logits against targets [B, T] ([B] after a
        LAST forward or a decode step): the mean loss, and with rows=True also
        the [B, T] row terms. probs=True replaces the held logits by their
        softmax (cross_entropy_fwd's probs_out, src/ops.c:499-574)."""
        targets = np.ascontiguousarray(targets, dtype=np.int32)
        if targets.ndim == 1:
            targets = targets.reshape(-1, 1)
        B, T = targets.shape
        loss = ctypes.c_float()
        per_row = np.empty((B, T), np.float32) if rows else None
        _check(lib().cngpt_hip_cross_entropy(self._h, _ip(targets), B, T, int(probs),
                                             ctypes.byref(loss),
                                             _fp(per_row) if rows else None), "cross_entropy")
        return (loss.value, per_row) if rows else loss.value

    def loss(self, tokens, targets, copy_logits: bool = False):
        """gpt_forward(m, tokens, targets, B, T) (src/model.c:442-625): the
        all-position forward, then the mean cross-entropy over its logits,
        which stay on the device unless copy_logits. Returns the loss, or
        (loss, logits [B, T, V])."""
        logits = self.forward(tokens, ALL, copy=copy_logits)
        loss = self.cross_entropy(targets)
        return (loss, logits) if copy_logits else loss

    def upload_targets(self, targets) -> None:
        targets = np.ascontiguousarray(targets, dtype=np.int32)
        _check(lib().cngpt_hip_upload_targets(self._h, _ip(targets), *targets.shape),
               "upload_targets")

    def cross_entropy_resident(self, B: int, T: int, probs: bool = False) -> None:
        _check(lib().cngpt_hip_cross_entropy_resident(self._h, B, T, int(probs)),
               "cross_entropy_resident")
        self._loss_rows = B * T

    def read_loss(self, rows: bool = False):
        """Mean of the last cross_entropy_resident, and with rows=True its
        B*T row terms."""
        loss = ctypes.c_float()
        per_row = np.empty(getattr(self, "_loss_rows", 0), np.float32) if rows else None
        _check(lib().cngpt_hip_read_loss(self._h, ctypes.byref(loss),
                                         _fp(per_row) if rows else None), "read_loss")
        return (loss.value, per_row) if rows else loss.value

    # -- decode ---------------------------------------------------------
    def decode_begin(self, prompt, capacity: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        B, T = prompt.shape
        out = np.empty((B, self.cfg.vocab_size), dtype=np.float32)
        _check(lib().cngpt_hip_decode_begin(self._h, _ip(prompt), B, T, capacity, _fp(out)),
               "decode_begin")
        self.decode_batch = B
        return out

    def decode_step(self, tokens=None, copy: bool = True):
        """Append one token per sequence (None: the device argmax of the
        previous logits). Returns the new [B, V] logits if copy."""
        tk = None
        if tokens is not None:
            tk = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        out = None
        if copy:
            out = np.empty((self.decode_batch, self.cfg.vocab_size), dtype=np.float32)
        _check(lib().cngpt_hip_decode_step(self._h, _ip(tk) if tk is not None else None,
                                           _fp(out) if out is not None else None), "decode_step")
        return out

    def generate(self, n_new: int, temperature: float = 1.0, top_k: int = 0,
                 draws=None) -> np.ndarray:
        """n_new tokens per sequence after decode_begin, [B, n_new]. draws
        None: greedy; else [n_new, B] uniform draws for sample_top_k."""
        B = self.decode_batch
        out = np.empty((B, n_new), dtype=np.int32)
        dp = None
        if draws is not None:
            draws = np.ascontiguousarray(draws, dtype=np.float32).reshape(n_new, B)
            dp = _fp(draws)
        _check(lib().cngpt_hip_generate(self._h, n_new, temperature, top_k, dp, _ip(out)),
               "generate")
        return out

    def argmax(self, B: int) -> np.ndarray:
        out = np.empty(B, dtype=np.int32)
        _check(lib().cngpt_hip_argmax(self._h, _ip(out)), "argmax")
        return out

    def sample(self, B: int, temperature: float, top_k: int, draws) -> np.ndarray:
        """One token per row of the current last-position logits."""
        draws = np.ascontiguousarray(draws, dtype=np.float32).reshape(B)
        out = np.empty(B, dtype=np.int32)
        _check(lib().cngpt_hip_sample(self._h, temperature, top_k, _fp(draws), _ip(out)),
               "sample")
        return out

    def decode_length(self) -> int:
        return lib().cngpt_hip_decode_length(self._h)

    def set_decode_path(self, path: int) -> None:
        """DECODE_AUTO, DECODE_KERNELS or DECODE_PERSISTENT for later steps."""
        _check(lib().cngpt_hip_set_decode_path(self._h, path), "set_decode_path")

    def decode_path(self) -> int:
        """Path of the last decode step (DECODE_KERNELS / DECODE_PERSISTENT)."""
        return lib().cngpt_hip_decode_path(self._h)

    # -- timing ---------------------------------------------------------
    def profile(self, on: bool) -> None:
        _check(lib().cngpt_hip_profile_enable(self._h, int(on)), "profile_enable")

    def profile_reset(self) -> None:
        _check(lib().cngpt_hip_profile_reset(self._h), "profile_reset")

    def profile_read(self) -> dict:
        res = {}
        for k, name in enumerate(KERNEL_CLASSES):
            ms, n = ctypes.c_double(), ctypes.c_long()
            fl, by = ctypes.c_double(), ctypes.c_double()
            _check(lib().cngpt_hip_profile_read(self._h, k, ctypes.byref(ms), ctypes.byref(n),
                                                ctypes.byref(fl), ctypes.byref(by)),
                   "profile_read")
            res[name] = {"ms": ms.value, "launches": n.value, "flops": fl.value,
                         "bytes": by.value}
        return res


# ---------------------------------------------------------------- training

TRAIN_PARAMS, TRAIN_GRADS, TRAIN_M, TRAIN_V = 0, 1, 2, 3


class Trainer:
    """The reference's training step on the device (cngpt_hip_train_*):
    gpt_forward with targets, gpt_backward, gpt_zero_grad and gpt_adamw
    (src/model.c:442-921) over a Model's parameters, which adamw updates in
    place, for one batch shape B x T."""

    def __init__(self, model: Model, B: int, T: int):
        self.model, self.B, self.T = model, B, T
        self.n = num_params(model.cfg)
        t = _VP()
        _check(lib().cngpt_hip_train_create(model._h, B, T, ctypes.byref(t)), "train_create")
        self._t = t

    def close(self) -> None:
        if getattr(self, "_t", None):
            lib().cngpt_hip_train_destroy(self._t)
            self._t = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def forward(self, tokens, targets) -> float:       # model.c:442-625
        tokens = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        targets = np.ascontiguousarray(targets, np.int32).reshape(-1)
        if tokens.size != self.B * self.T or targets.size != self.B * self.T:
            raise CngptError(f"tokens and targets must hold {self.B} x {self.T} ids")
        loss = ctypes.c_float()
        _check(lib().cngpt_hip_train_forward(self._t, _ip(tokens), _ip(targets),
                                             ctypes.byref(loss)), "train_forward")
        return float(loss.value)

    def backward(self) -> None:                         # model.c:634-877
        _check(lib().cngpt_hip_train_backward(self._t), "train_backward")

    def set_dropout(self, p: float) -> None:
        """GPTConfig.dropout (model.h:43): with p > 0 each forward draws its
        keep masks with the process's rand() in model.c's order and applies
        the residual-stream dropout of model.c:471-599 (and its backward)."""
        _check(lib().cngpt_hip_train_set_dropout(self._t, ctypes.c_float(p)), "train_set_dropout")

    def zero_grad(self) -> None:                        # model.c:879-886
        _check(lib().cngpt_hip_train_zero_grad(self._t), "train_zero_grad")

    def adamw(self, lr, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1, grad_clip=1.0) -> float:
        """model.c:888-921; returns the gradient norm before clipping."""
        norm = ctypes.c_float()
        _check(lib().cngpt_hip_train_adamw(self._t, lr, beta1, beta2, eps, wd, grad_clip,
                                           ctypes.byref(norm)), "train_adamw")
        return float(norm.value)

    def read(self, which: int) -> np.ndarray:
        out = np.empty(self.n, np.float32)
        _check(lib().cngpt_hip_train_read(self._t, which, _fp(out), self.n), "train_read")
        return out

    def write(self, which: int, values) -> None:
        values = np.ascontiguousarray(values, np.float32)
        _check(lib().cngpt_hip_train_write(self._t, which, _fp(values), values.size),
               "train_write")

    @property
    def params(self) -> np.ndarray:
        return self.read(TRAIN_PARAMS)

    @property
    def grads(self) -> np.ndarray:
        return self.read(TRAIN_GRADS)

    @property
    def steps(self) -> int:
        return lib().cngpt_hip_train_steps(self._t)

