"""Weight file -> device streaming loader (cngpt_hip_load_file) vs the
host-buffer upload (cngpt_hip_load_params) of the same parameters.

The file is the reference's format (src/model.c:177-231): a 7 x int32
header and the flat fp32 parameters. Loading it through pinned chunks must
leave the device buffer byte-identical to uploading the host array, which
the forward shows bitwise: every parameter takes part in a last-position
forward over a full block_size window (wpe rows 0..block_size-1, every
layer, the weight-tied lm_head over all of wte).
"""
import numpy as np
import pytest

import cngpt_amd
import oracle
from test_parity_gpu import compare, ocfg, randomize, say

pytestmark = pytest.mark.gpu


def window(cfg, B=1, seed=5):
    T = cfg.block_size
    return oracle.lcg_tokens(B * T, cfg.vocab_size, seed=seed).reshape(B, T)


def test_gpt2_small_file_matches_host_upload(tmp_path):
    """498 MB: 30 chunks of 16 MB over 4 reader threads, the last partial."""
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    path = tmp_path / "small.bin"
    cngpt_amd.save_weights(str(path), cfg, params)
    tk = window(cfg)
    say("small: host upload")
    with cngpt_amd.Model(cfg, params) as m:
        want = m.forward(tk)
    say("small: streamed from the file")
    with cngpt_amd.Model.from_file(str(path)) as m:
        assert m.cfg == cfg
        got = m.forward(tk)
    assert np.array_equal(got, want)
    compare(got, oracle.forward(ocfg(cfg), params, tk), what="small from file vs oracle")


def test_reload_shapes_and_failures(tmp_path):
    """One handle: tiny -> other shape -> same shape with other weights; files
    rejected at their header leave the loaded parameters in place."""
    tiny = cngpt_amd.TINY
    mid = cngpt_amd.Config(2, 4, 256, 1000, 256)
    files = {}
    for name, cfg, seed in (("tiny", tiny, 1), ("mid", mid, 2), ("mid2", mid, 3)):
        p = randomize(cfg, cngpt_amd.init_weights(cfg, seed), seed + 10)
        f = tmp_path / f"{name}.bin"
        cngpt_amd.save_weights(str(f), cfg, p)
        files[name] = (cfg, p, f)
    with cngpt_amd.Model.from_file(str(files["tiny"][2])) as m:
        for name in ("tiny", "mid", "mid2", "tiny"):
            cfg, p, f = files[name]
            say(f"load {name}")
            assert m.load_file(str(f)) == cfg
            tk = window(cfg, B=2)
            compare(m.forward(tk), oracle.forward(ocfg(cfg), p, tk), what=name)
        # rejected before any device work
        cfg, p, f = files["mid"]
        cut = tmp_path / "cut.bin"
        cut.write_bytes(f.read_bytes()[:-100])
        with pytest.raises(cngpt_amd.CngptError, match="ends before its parameters"):
            m.load_file(str(cut))
        with pytest.raises(cngpt_amd.CngptError, match="not a cngpt weight file"):
            bad = tmp_path / "bad.bin"
            bad.write_bytes(b"\0" * 64)
            m.load_file(str(bad))
        say("tiny still loaded after the failures")
        tcfg, tp, _ = files["tiny"]
        tk = window(tcfg, B=1)
        compare(m.forward(tk), oracle.forward(ocfg(tcfg), tp, tk), what="kept")
        say("load mid after the failures")
        m.load_file(str(f))
        tk = window(cfg, B=1)
        compare(m.forward(tk), oracle.forward(ocfg(cfg), p, tk), what="after failures")
        # decode on streamed weights
        say("decode on streamed weights")
        m.decode_begin(tk[:, :10], capacity=40)
        gen = m.generate(20)
        ref = oracle.forward(ocfg(cfg), p, np.concatenate([tk[:, :10], gen[:, :-1]], 1),
                             oracle.ALL)[:, 9:]
        srt = np.sort(ref, -1)
        tie = (srt[..., -1] - srt[..., -2]) < 1e-4
        assert np.array_equal(np.where(tie, 0, ref.argmax(-1)), np.where(tie, 0, gen))
