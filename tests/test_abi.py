"""The C-ABI library without a GPU: it loads, exports every symbol the
headers declare, and its host-only entry points (seeded init, parameter
count, weight file) behave; compute entry points fail cleanly."""
import ctypes
import os
import re
import struct

import numpy as np
import pytest

import cngpt_amd
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in ("cngpt_hip.h", "fast.h", "model.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name.startswith(("cngpt_hip_", "fast_", "gpt_")):
                names.add(name)
    return names


def test_library_exports_every_declared_symbol():
    lib = cngpt_amd.lib()
    declared = _declared_functions()
    assert len(declared) >= 30
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    assert declared == set(cngpt_amd.EXPORTS)


def test_init_weights_matches_oracle_bitwise():
    for cfg in (cngpt_amd.TINY, cngpt_amd.Config(2, 2, 128, 300, 64)):
        got = cngpt_amd.init_weights(cfg, 42)
        ref = oracle.init_weights(oracle.Cfg(cfg.n_layer, cfg.n_head, cfg.n_embd,
                                             cfg.vocab_size, cfg.block_size), 42)
        assert np.array_equal(got, ref)


def test_num_params():
    assert cngpt_amd.num_params(cngpt_amd.GPT2_SMALL) == 124_439_808
    assert cngpt_amd.num_params(cngpt_amd.GPT2_XL) == 1_557_611_200
    with pytest.raises(cngpt_amd.CngptError):
        cngpt_amd.num_params(cngpt_amd.Config(1, 3, 32, 10, 8))  # 32 % 3 != 0


def test_weight_file_roundtrip_and_errors(tmp_path):
    cfg = cngpt_amd.TINY
    p = cngpt_amd.init_weights(cfg, 7)
    f = tmp_path / "tiny.bin"
    cngpt_amd.save_weights(str(f), cfg, p)
    assert f.stat().st_size == 28 + 4 * p.size
    cfg2, p2 = cngpt_amd.load_weights(str(f))
    assert cfg2 == cfg and np.array_equal(p, p2)
    raw = f.read_bytes()
    bad = tmp_path / "bad.bin"
    bad.write_bytes(struct.pack("<i", 0x12345678) + raw[4:])
    with pytest.raises(cngpt_amd.CngptError, match="not a cngpt weight file"):
        cngpt_amd.load_weights(str(bad))
    short = tmp_path / "short.bin"
    short.write_bytes(raw[:-8])
    with pytest.raises(cngpt_amd.CngptError, match="ends before its parameters"):
        cngpt_amd.load_weights(str(short))


def test_file_config_validates_header_without_gpu(tmp_path):
    """cngpt_hip_file_config: the header checks cngpt_hip_load_file makes
    before any device work (GPTHeader, src/model.h:19-30; gpt_load's magic
    and length checks, src/model.c:185-207)."""
    cfg = cngpt_amd.Config(2, 4, 64, 97, 32)
    p = cngpt_amd.init_weights(cfg, 3)
    f = tmp_path / "m.bin"
    cngpt_amd.save_weights(str(f), cfg, p)
    assert cngpt_amd.file_config(str(f)) == (cfg, p.size)
    raw = f.read_bytes()
    # trailing bytes are ignored, as gpt_load reads exactly n_params floats
    (tmp_path / "long.bin").write_bytes(raw + b"\0" * 12)
    assert cngpt_amd.file_config(str(tmp_path / "long.bin")) == (cfg, p.size)

    def bad(name, data, match):
        g = tmp_path / name
        g.write_bytes(data)
        with pytest.raises(cngpt_amd.CngptError, match=match):
            cngpt_amd.file_config(str(g))

    hdr = list(struct.unpack("<7i", raw[:28]))

    def with_hdr(**kw):
        h = hdr.copy()
        for i, k in enumerate(("magic", "version", "L", "H", "C", "V", "T")):
            h[i] = kw.get(k, h[i])
        return struct.pack("<7i", *h) + raw[28:]

    bad("empty.bin", b"", "ends inside its 28-byte header")
    bad("hdr.bin", raw[:27], "ends inside its 28-byte header")
    bad("magic.bin", with_hdr(magic=0x12345678), "not a cngpt weight file \\(first word 0x12345678\\)")
    bad("version.bin", with_hdr(version=2), "unsupported version 2")
    bad("heads.bin", with_hdr(H=5), "invalid shape")          # 64 % 5 != 0
    bad("zero.bin", with_hdr(L=0), "invalid shape")
    bad("huge.bin", with_hdr(C=1 << 30, H=1), "invalid shape")
    bad("short.bin", raw[:-4], "ends before its parameters")
    bad("bigger.bin", with_hdr(L=3), "ends before its parameters")      # header promises more
    with pytest.raises(cngpt_amd.CngptError, match="No such file"):
        cngpt_amd.file_config(str(tmp_path / "missing.bin"))


class _GPTConfig(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("n_head", ctypes.c_int),
                ("n_embd", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("block_size", ctypes.c_int), ("dropout", ctypes.c_float)]


_PP = ctypes.POINTER(ctypes.c_void_p)


class _GPTWeights(ctypes.Structure):
    _fields_ = ([("wte", ctypes.c_void_p), ("wpe", ctypes.c_void_p)]
                + [(n, _PP) for n in ("ln1_w", "ln1_b", "c_attn_w", "c_attn_b", "c_proj_w",
                                      "c_proj_b", "ln2_w", "ln2_b", "mlp_fc_w", "mlp_fc_b",
                                      "mlp_proj_w", "mlp_proj_b")]
                + [("ln_f_w", ctypes.c_void_p), ("ln_f_b", ctypes.c_void_p)])


class _GPTActivations(ctypes.Structure):
    # 25 pointer members (include/model.h, src/model.h:86-115)
    _fields_ = [(f"p{i}", ctypes.c_void_p) for i in range(25)]


class _GPT(ctypes.Structure):
    _fields_ = [("cfg", _GPTConfig), ("params", _GPTWeights), ("grads", _GPTWeights),
                ("acts", _GPTActivations), ("param_buf", ctypes.POINTER(ctypes.c_float)),
                ("grad_buf", ctypes.c_void_p), ("act_buf", ctypes.c_void_p),
                ("mask_buf", ctypes.c_void_p), ("m_buf", ctypes.c_void_p),
                ("v_buf", ctypes.c_void_p), ("decay_buf", ctypes.c_void_p),
                ("n_params", ctypes.c_int), ("step", ctypes.c_int)]


def test_c_model_api_reads_the_same_file(tmp_path):
    """gpt_load / gpt_num_params / gpt_init_weights (model.h) agree with the
    Python weight file and the seeded init."""
    lib = cngpt_amd.lib()
    cfg = cngpt_amd.TINY
    c = _GPTConfig(cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size, 0.0)
    lib.gpt_num_params.argtypes = [ctypes.POINTER(_GPTConfig)]
    assert lib.gpt_num_params(ctypes.byref(c)) == cngpt_amd.num_params(cfg)
    p = cngpt_amd.init_weights(cfg, 3)
    f = tmp_path / "m.bin"
    cngpt_amd.save_weights(str(f), cfg, p)
    m = _GPT()
    lib.gpt_load.argtypes = [ctypes.POINTER(_GPT), ctypes.c_char_p]
    lib.gpt_free.argtypes = [ctypes.POINTER(_GPT)]
    assert lib.gpt_load(ctypes.byref(m), str(f).encode()) == 0
    assert m.n_params == p.size and m.cfg.n_embd == cfg.n_embd
    got = np.ctypeslib.as_array(m.param_buf, (m.n_params,))
    assert np.array_equal(got, p)
    # wpe sits right after wte (src/model.c:63-64)
    assert m.params.wpe - m.params.wte == 4 * cfg.vocab_size * cfg.n_embd
    lib.gpt_free(ctypes.byref(m))
    # gpt_init + srand + gpt_init_weights == the seeded init
    lib.gpt_init.argtypes = [ctypes.POINTER(_GPT), _GPTConfig]
    lib.gpt_init_weights.argtypes = [ctypes.POINTER(_GPT)]
    m2 = _GPT()
    assert lib.gpt_init(ctypes.byref(m2), c) == 0
    ctypes.CDLL(None).srand(3)
    lib.gpt_init_weights(ctypes.byref(m2))
    assert np.array_equal(np.ctypeslib.as_array(m2.param_buf, (m2.n_params,)), p)
    lib.gpt_free(ctypes.byref(m2))
    # a header of the wrong shape is refused when the model already exists
    m3 = _GPT()
    assert lib.gpt_init(ctypes.byref(m3), _GPTConfig(1, 1, 8, 5, 4, 0.0)) == 0
    assert lib.gpt_load(ctypes.byref(m3), str(f).encode()) == -1
    lib.gpt_free(ctypes.byref(m3))


def test_create_without_gpu_fails_cleanly():
    lib = cngpt_amd.lib()
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    assert lib.cngpt_hip_create(0, ctypes.byref(h)) == -1
    assert b"device" in lib.cngpt_hip_last_error() or lib.cngpt_hip_last_error()
    assert not h.value
