"""`cngpt sample` and `cngpt bench` on the device, checked with the oracle.

sample: the tokens the command prints are replayed through the oracle:
token i is sample_top_k (src/model.c:927-989) over the oracle's logits of
the context gpt_sample would use (src/model.c:991-1016: the last block_size
tokens, positions from 0), with the i-th rand() draw after srand(seed).
"""
import os
import re
import subprocess

import numpy as np
import pytest

import cngpt_amd
import oracle
from test_decode_gpu import cdf_gap
from test_parity_gpu import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "cngpt_amd", "cngpt")


def run(*args):
    say("cngpt " + " ".join(args))
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=120)


def parse_sample(out):
    line = [l for l in out.splitlines() if "|" in l][0]
    prompt, gen = line.split("|")
    return ([int(x) for x in prompt.strip().split(",")], [int(x) for x in gen.strip().split(",")])


def replay(cfg, params, prompt, gen, seed, temp, top_k, what):
    oracle.srand(seed)
    draws = [oracle.rand_uniform() for _ in gen]
    seq = list(prompt)
    ocfg = oracle.Cfg(cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size)
    for i, g in enumerate(gen):
        ctx = np.array(seq[-cfg.block_size:], np.int32).reshape(1, -1)
        logits = oracle.forward(ocfg, params, ctx, oracle.LAST)[0]
        want = oracle.sample_top_k(logits, temp, top_k, draws[i])
        if want != g:
            assert cdf_gap(logits, temp, top_k, draws[i]) < 1e-4, (what, i, g, want)
            say(f"  {what}: stopped at a CDF boundary at token {i}")
            return
        seq.append(g)


def test_sample_tiny_with_sliding_window(tmp_path):
    """Tiny model, block_size 8: 3 prompt tokens + 20 new ones, so tokens
    past the 6th come from the sliding window (positions re-based)."""
    w = tmp_path / "tiny.bin"
    assert run("create-tiny", f"--out={w}", "--seed=5").returncode == 0
    cfg, params = cngpt_amd.load_weights(str(w))
    for temp, k, seed in [(0.8, 10, 7), (1.0, 0, 11), (1.5, 1, 3)]:
        r = run("sample", f"--weights={w}", "--prompt=1,2,3", "--tokens=20", f"--temp={temp}",
                f"--topk={k}", f"--seed={seed}")
        assert r.returncode == 0, r.stderr
        prompt, gen = parse_sample(r.stdout)
        assert prompt == [1, 2, 3] and len(gen) == 20
        assert all(0 <= g < cfg.vocab_size for g in gen)
        replay(cfg, params, prompt, gen, seed, temp, k, f"tiny temp={temp} k={k}")
    # same seed, same tokens
    a = run("sample", f"--weights={w}", "--tokens=12", "--seed=42")
    b = run("sample", f"--weights={w}", "--tokens=12", "--seed=42")
    assert a.returncode == 0 and a.stdout == b.stdout
    # prompt tokens outside the vocabulary are rejected
    r = run("sample", f"--weights={w}", "--prompt=1,64", "--tokens=2", "--seed=1")
    assert r.returncode == 1 and "bad prompt token" in r.stderr


def test_sample_and_bench_gpt2_small(tmp_path):
    cfg = cngpt_amd.GPT2_SMALL
    params = cngpt_amd.init_weights(cfg, 1234)
    w = tmp_path / "small.bin"
    cngpt_amd.save_weights(str(w), cfg, params)
    prompt = ",".join(str(t) for t in oracle.lcg_tokens(16, cfg.vocab_size))
    r = run("sample", f"--weights={w}", f"--prompt={prompt}", "--tokens=24", "--temp=0.8",
            "--topk=40", "--seed=7")
    assert r.returncode == 0, r.stderr
    p, gen = parse_sample(r.stdout)
    replay(cfg, params, p, gen, 7, 0.8, 40, "small")
    r = run("bench", f"--weights={w}", "--fast", "--seq=128", "--iters=5")
    assert r.returncode == 0, r.stderr
    d = float(re.search(r"fast vs all-positions : ([0-9.e+-]+)", r.stdout).group(1))
    assert d < 1e-4
    # the independent route (prefill of 127 tokens, then one KV-cache decode
    # step), as the reference's bench compares gpt_forward_fast with gpt_forward
    d = float(re.search(r"fast vs KV-cache decode : ([0-9.e+-]+)", r.stdout).group(1))
    say(f"  bench --fast seq 128: fast vs KV-cache decode {d:.3e}")
    assert d < 1e-3
    tps = float(re.search(r"tok/s\s*:\s*([0-9.]+)", r.stdout).group(1))
    assert tps > 0
    say(f"  bench --fast seq 128: {tps} tok/s")
    r = run("bench", f"--weights={w}", "--seq=64", "--batch=2", "--iters=3")
    assert r.returncode == 0, r.stderr
