"""Benchmark: GPT-2 fp32 batched forward with full logits, and batched decode.

Default workload (the headline): GPT-2 small, B=16, T=1024, all-position
logits [16, 1024, 50257] left in HBM. Prints one JSON line:
  value     forward tokens/s over the timed steps (tokens already in HBM);
  roofline  the MFMA GEMM kernels (all linear layers and the lm_head), each
            launch timed with a HIP event pair on the library's stream during
            the same steps, against MI355X's dense fp32 matrix peak;
  loss      cross-entropy of those logits against next-token targets, on
            the device (HBM-bound; GB/s of one read of the logits);
  load      the weights as a weight file streamed to the device;
  train     training steps on the device (zero_grad, forward with targets,
            backward, AdamW) at B=4 T=1024, tokens/s and the algorithmic
            FLOPs against the fp32 matrix peak;
  decode    greedy single-token steps with the KV cache (B=1: all steps in
            one persistent launch; otherwise one replayed HIP graph per
            step), tok/s and algorithmic HBM bytes / time;
  batched_decode  the decode halves of the GPT-2 medium (B=8 after a
            768-token prompt) and XL (B=32 after 32 tokens) workloads,
            each on a handle of its own, the same figures;
  cpu_baseline  the oracle (C restatement of the reference's fast path with
            OpenBLAS) timed on this host on a bounded sample.
--workload medium / xl measures GPT-2 medium (prefill B=8, decode B=8 after a
768-token prompt) and XL (prefill B=4, decode B=32 after a 32-token prompt).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import cngpt_amd  # noqa: E402

PEAK_FP32_MFMA = 157.3e12   # 256 CUs x 2.4 GHz x 256 FLOP/clk/CU
PEAK_HBM = 8.0e12
SEED = 1234

# name -> (config, prefill B, T, decode B, prompt, decode steps)
WORKLOADS = {
    "small": (cngpt_amd.GPT2_SMALL, 16, 1024, 1, 32, 512),
    "medium": (cngpt_amd.GPT2_MEDIUM, 8, 1024, 8, 768, 256),
    "xl": (cngpt_amd.GPT2_XL, 4, 1024, 32, 32, 128),
}
NAMES = {"small": "GPT-2 small", "medium": "GPT-2 medium", "xl": "GPT-2 XL"}


def lcg_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """Token ids from the LCG of the reference's bench (src/cngpt.c:338-342)."""
    out = np.empty(n, dtype=np.int64)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (s >> 8) % vocab
    return out.astype(np.int32)


def weights(name: str, cfg):
    """GPT-2 small: the reference's seeded init (srand(1234), the draw order of
    gpt_init_weights). Medium / XL: N(0, 0.02) from numpy's generator (the
    rand() stream would take minutes for 0.35-1.5 G values), 64 PCG64
    streams spawned from the seed, filled by a thread pool."""
    if name == "small":
        return cngpt_amd.init_weights(cfg, SEED), \
            "seeded N(0,0.02) weights (srand 1234, gpt_init_weights order)"
    n = cngpt_amd.num_params(cfg)
    p = np.empty(n, np.float32)
    streams = np.random.SeedSequence(SEED).spawn(64)
    cuts = np.linspace(0, n, len(streams) + 1).astype(np.int64)

    def fill(i):
        part = p[cuts[i]:cuts[i + 1]]
        np.random.Generator(np.random.PCG64(streams[i])).standard_normal(out=part,
                                                                         dtype=np.float32)
        part *= np.float32(0.02)

    with ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(fill, range(len(streams))))
    return p, "N(0,0.02) weights from 64 numpy PCG64 streams spawned from seed 1234"


def prefill(m: cngpt_amd.Model, cfg, B: int, T: int, steps: int, warmup: int,
            mode: int = cngpt_amd.ALL):
    tokens = lcg_tokens(B * T, cfg.vocab_size, 12345).reshape(B, T)
    m.reserve(B, T, mode)
    m.upload_tokens(tokens)
    for _ in range(warmup):
        m.forward_resident(B, T, mode)
    m.synchronize()
    m.profile_reset()
    m.profile(True)
    m.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.forward_resident(B, T, mode)
    m.synchronize()
    dt = time.perf_counter() - t0
    m.profile(False)
    prof = m.profile_read()
    m.profile_reset()
    return dt, prof


def train_flops(cfg, B: int, T: int) -> float:
    """Algorithmic FLOPs of one training step: the forward's products
    (linear layers, lm_head, causal attention) and twice that for the
    backward (dX and dW of each product; dV, dP, dQ, dK of attention),
    without the attention's recomputed scores."""
    C, L, V = cfg.n_embd, cfg.n_layer, cfg.vocab_size
    N = B * T
    linear = 2.0 * N * (12 * C * C * L + V * C)
    attn = 2.0 * C * T * (T + 1) * B * L
    return 3.0 * (linear + attn)


def train_leg(m: cngpt_amd.Model, cfg, B: int, T: int, steps: int, warmup: int) -> dict:
    """Training steps on the device (cngpt_amd.Trainer): zero_grad, forward
    with next-token targets, backward, AdamW (lr 3e-4, clip 1.0: `cngpt
    train`'s defaults, src/cngpt.c:94-162). The forward reads its loss and
    AdamW the gradient norm back, so each step ends synchronized, as the
    reference's loop does."""
    ids = lcg_tokens(B * T + 1, cfg.vocab_size, 4321)
    tok, tgt = ids[:-1].reshape(B, T), ids[1:].reshape(B, T)
    with cngpt_amd.Trainer(m, B, T) as tr:
        for _ in range(warmup):
            tr.zero_grad()
            tr.forward(tok, tgt)
            tr.backward()
            tr.adamw(3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
        m.synchronize()
        t0 = time.perf_counter()
        losses = []
        for _ in range(steps):
            tr.zero_grad()
            losses.append(tr.forward(tok, tgt))
            tr.backward()
            norm = tr.adamw(3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
        m.synchronize()
        dt = time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(steps):
            tr.forward(tok, tgt)
        m.synchronize()
        dt_f = time.perf_counter() - t0
    fl = train_flops(cfg, B, T)
    return {"train_B": B, "train_T": T, "tok_s": round(B * T * steps / dt, 1),
            "ms_per_step": round(dt * 1e3 / steps, 3),
            "forward_ms": round(dt_f * 1e3 / steps, 3),
            "tflops": round(fl * steps / dt / 1e12, 2),
            "mfma_frac": round(fl * steps / dt / PEAK_FP32_MFMA, 4),
            "first_loss": round(losses[0], 5), "last_loss": round(losses[-1], 5),
            "last_grad_norm": round(norm, 5)}


def loss_leg(m: cngpt_amd.Model, cfg, B: int, T: int, steps: int):
    """Cross-entropy (cross_entropy_fwd semantics) of the [B, T, V] logits the
    last forward left in HBM against next-token targets: `steps` launches,
    each timed with a HIP event pair on the library's stream. Algorithmic
    bytes per launch: every logit once, plus the target and row term of
    each row."""
    tokens = lcg_tokens(B * T, cfg.vocab_size, 12345)
    m.upload_targets(np.roll(tokens, -1).reshape(B, T))
    m.cross_entropy_resident(B, T)
    loss = m.read_loss()
    m.profile_reset()
    m.profile(True)
    for _ in range(steps):
        m.cross_entropy_resident(B, T)
    m.synchronize()
    m.profile(False)
    p = m.profile_read()["loss"]
    m.profile_reset()
    ms = p["ms"] / p["launches"]
    nbytes = 4.0 * B * T * cfg.vocab_size + 8.0 * B * T
    return {"loss": round(loss, 6), "ms_per_launch": round(ms, 4),
            "hbm": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                    "frac": round(nbytes / (ms * 1e-3) / PEAK_HBM, 4),
                    "bytes_per_launch": nbytes},
            "kernel": "k_ce_rows + k_ce_mean", "launches": p["launches"],
            "targets": "next token of the same LCG stream"}


def load_leg(m: cngpt_amd.Model, cfg, params) -> dict:
    """The weight file of these parameters streamed into the handle's
    parameter allocation (cngpt_hip_load_file), from a warm page cache:
    file written first, then timed loads."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "weights.bin")
        cngpt_amd.save_weights(path, cfg, params)
        m.load_file(path)
        t, th = [], []
        for _ in range(3):
            t0 = time.perf_counter()
            m.load_file(path)
            t.append(time.perf_counter() - t0)
        for _ in range(2):
            # the host-buffer route: whole file into host memory, then one upload
            t0 = time.perf_counter()
            _, p = cngpt_amd.load_weights(path)
            m.load_params(p)
            th.append(time.perf_counter() - t0)
            del p
    best = min(t)
    nbytes = 4.0 * params.size
    return {"bytes": nbytes, "s": round(best, 4), "gb_s": round(nbytes / best / 1e9, 2),
            "host_buffer_s": round(min(th), 4),
            "source": "page cache (file just written), pinned 16 MB chunks, 4 reader threads"}


def decode_bytes(cfg, params_n: int, B: int, first_pos: int, steps: int) -> float:
    """Algorithmic HBM bytes of `steps` decode steps whose tokens sit at
    positions first_pos.. : every weight once per step (wpe: one row per
    sequence), the K and V rows of keys 0..p, the new q/k/v row and the
    logits of each sequence."""
    C, L, V = cfg.n_embd, cfg.n_layer, cfg.vocab_size
    weights_b = 4.0 * (params_n - cfg.block_size * C + B * C)
    total = 0.0
    for p in range(first_pos, first_pos + steps):
        total += weights_b + 4.0 * L * B * (p + 1) * 2 * C + 4.0 * L * B * 3 * C + 4.0 * B * V
    return total


PATHS = {cngpt_amd.DECODE_KERNELS: "kernels", cngpt_amd.DECODE_PERSISTENT: "persistent"}


def decode(m: cngpt_amd.Model, cfg, B: int, prompt_len: int, steps: int, draws=None):
    """`steps` single-token decode steps for B sequences after a prompt_len
    prompt, as one cngpt_hip_generate call; greedy, or temp 0.8 / top-k 40
    sampling when draws are given."""
    prompt = lcg_tokens(B * prompt_len, cfg.vocab_size, 777).reshape(B, prompt_len)
    kw = {} if draws is None else {"temperature": 0.8, "top_k": 40,
                                   "draws": draws[:(steps + 1) * B]}
    nwarm = min(8, steps + 1)
    warm = {} if draws is None else {"temperature": 0.8, "top_k": 40, "draws": draws[:nwarm * B]}
    m.decode_begin(prompt, capacity=prompt_len + steps)
    m.generate(nwarm, **warm)                 # warm-up, captures the step graph
    m.decode_begin(prompt, capacity=prompt_len + steps)
    m.synchronize()
    t0 = time.perf_counter()
    m.generate(steps + 1, **kw)
    return time.perf_counter() - t0, PATHS.get(m.decode_path(), "none")


def batched_decode():
    """The decode halves of the GPT-2 medium and XL workloads, each on a
    handle of its own: greedy steps of B sequences after a prompt (medium
    B=8, 256 steps after 768 tokens; XL B=32, 128 steps after 32 tokens),
    one generate call timed after a warm-up one; HBM fraction of the
    algorithmic bytes per step (every weight, the cached keys and values)."""
    out = {}
    for wname in ("medium", "xl"):
        wcfg, _, _, dB, prompt, steps = WORKLOADS[wname]
        p, _ = weights(wname, wcfg)
        mm = cngpt_amd.Model(wcfg, p)
        dt, path = decode(mm, wcfg, dB, prompt, steps)
        nbytes = decode_bytes(wcfg, p.size, dB, prompt, steps)
        mm.close()
        del p
        out[f"{wname}_b{dB}"] = {"model": NAMES[wname], "B": dB, "prompt": prompt,
                                 "steps": steps, "ms_per_step": round(dt * 1e3 / steps, 4),
                                 "tok_s": round(steps * dB / dt, 1),
                                 "hbm_frac": round(nbytes / dt / PEAK_HBM, 4), "path": path}
    return out


def reference_shape(m: cngpt_amd.Model, iters: int = 100, warmup: int = 10):
    """The shape the reference publishes its fast-path numbers at (B=1,
    T=128, final-position logits, README.md:410-416), through the whole
    host API (tokens H2D, logits D2H, synchronise) as `cngpt bench --fast`
    does; `warmup` untimed forwards first (the first captures the forward's
    graph)."""
    tk = np.zeros((1, 128), np.int32)
    for _ in range(warmup):
        m.forward(tk, cngpt_amd.LAST)
    t0 = time.perf_counter()
    for _ in range(iters):
        m.forward(tk, cngpt_amd.LAST)
    dt = (time.perf_counter() - t0) / iters
    return {"B": 1, "T": 128, "tok_s": round(128 / dt, 1), "ms_per_forward": round(dt * 1e3, 3),
            "published_cpu_tok_s": 2261.6,
            "published_cpu": "Ryzen 5 7600, 6 threads, OpenBLAS 0.3.29 (reference README.md:415)"}


def dp_share(m: cngpt_amd.Model, cfg, steps: int = 10, warmup: int = 2):
    """One GPU's share of the B=16 T=1024 workload under 8-way sequence
    sharding: B=2, T=1024 (M = 2048 rows, where the products have too few
    128 x 128 tiles to fill the CUs without splitting K)."""
    dt, prof = prefill(m, cfg, 2, 1024, steps, warmup)
    g = prof["gemm"]
    return {"B": 2, "T": 1024, "tok_s": round(2 * 1024 * steps / dt, 1),
            "ms_per_forward": round(dt * 1e3 / steps, 3),
            "gemm_tflops": round(g["flops"] / (g["ms"] * 1e-3) / 1e12, 2),
            "gemm_frac": round(g["flops"] / (g["ms"] * 1e-3) / PEAK_FP32_MFMA, 4),
            "gemm_ms_per_forward": round(g["ms"] / steps, 3)}


def cpu_baseline(name: str, cfg, params, budget_s: float, B: int, T: int):
    """The oracle (C restatement of the reference's gpt_forward_fast with
    OpenBLAS, one pinned thread per physical core) on the workload itself:
    B x T tokens, all-position logits, one warm-up forward and then as many
    timed forwards as fit the budget (at least one)."""
    import oracle

    ocfg = oracle.Cfg(cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size)
    cores = oracle.set_threads(0)
    tk = lcg_tokens(B * T, cfg.vocab_size, 12345).reshape(B, T)
    oracle.forward(ocfg, params, tk, oracle.ALL)            # warm-up (first touch)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.forward(ocfg, params, tk, oracle.ALL)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n >= 20:
            break
    tok_s = n * B * T / dt
    # the reference's own semantics: final-position logits (gpt_forward_fast)
    t1 = time.perf_counter()
    oracle.forward(ocfg, params, tk, oracle.LAST)
    last_s = time.perf_counter() - t1
    return {"value": round(tok_s, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} timed forward(s) of the workload itself, B={B} x T={T} {NAMES[name]} "
                      f"fp32, all-position logits ({dt:.1f} s, after one warm-up forward); oracle "
                      f"C restatement of fast.c + {oracle.blas_info()}",
            "last_position_tok_s": round(B * T / last_s, 2)}


def copy_calibration(nbytes: int) -> int:
    """One plain device-to-device copy of nbytes (the HIP runtime's blit
    kernel). Under rocprofv3 --pmc its FETCH_SIZE and WRITE_SIZE give the
    counter's reading for a known number of bytes moved."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(nbytes)) == 0
    assert hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(nbytes)) == 0
    assert hip.hipMemset(src, 1, ctypes.c_size_t(nbytes)) == 0
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3) == 0   # device to device
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(src)
    hip.hipFree(dst)
    return nbytes


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="small")
    ap.add_argument("--decode-steps", type=int, default=None,
                    help="decode steps (default: the workload's)")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MiB",
                    help="also run one plain device copy of this size (counter calibration)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode legs (for kernel traces of the decode step)")
    ap.add_argument("--prefill", type=int, nargs=2, metavar=("B", "T"), default=None,
                    help="only time all-position forwards of B x T tokens of the workload's "
                         "model (for kernel traces of one prefill shape)")
    ap.add_argument("--last", action="store_true",
                    help="with --prefill: final-position logits (gpt_forward_fast's mode)")
    ap.add_argument("--loss", action="store_true",
                    help="with --prefill (all positions): also the cross-entropy leg over the "
                         "held logits (for counter runs of the loss kernels)")
    ap.add_argument("--train", type=int, nargs=2, metavar=("B", "T"), default=None,
                    help="only time training steps (zero_grad, forward with targets, backward, "
                         "AdamW) of B x T tokens of the workload's model")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    name = args.workload
    cfg, B, T, dB, prompt, dsteps = WORKLOADS[name]
    if args.decode_steps is not None:
        dsteps = args.decode_steps
    params, data = weights(name, cfg)
    m = cngpt_amd.Model(cfg, params)

    if args.prefill:
        pB, pT = args.prefill
        mode = cngpt_amd.LAST if args.last else cngpt_amd.ALL
        dt, prof = prefill(m, cfg, pB, pT, args.steps, args.warmup, mode)
        g = prof["gemm"]
        loss = loss_leg(m, cfg, pB, pT, max(args.steps, 1)) if args.loss and not args.last else None
        m.close()
        calib = copy_calibration(args.copy_calibration << 20) if args.copy_calibration else None
        print(json.dumps({"workload": name, "B": pB, "T": pT,
                          "logits": "final position" if args.last else "all positions",
                          "tok_s": round(pB * pT * args.steps / dt, 1),
                          "ms_per_forward": round(dt * 1e3 / args.steps, 3),
                          "gemm_tflops": round(g["flops"] / (g["ms"] * 1e-3) / 1e12, 2),
                          "gemm_frac": round(g["flops"] / (g["ms"] * 1e-3) / PEAK_FP32_MFMA, 4),
                          "kernel_ms_per_forward": {k: round(v["ms"] / args.steps, 3)
                                                    for k, v in prof.items() if v["launches"]},
                          "loss": loss,
                          "copy_calibration_bytes": calib}),
              flush=True)
        return

    if args.train:
        tB, tT = args.train
        res = train_leg(m, cfg, tB, tT, args.steps, args.warmup)
        m.close()
        print(json.dumps({"workload": name, **res}), flush=True)
        return

    if args.decode_only:
        dec_dt, dec_path = decode(m, cfg, dB, prompt, dsteps)
        dec_bytes = decode_bytes(cfg, params.size, dB, prompt, dsteps)
        m.set_decode_path(cngpt_amd.DECODE_KERNELS)
        kern_dt, _ = decode(m, cfg, dB, prompt, dsteps)
        m.set_decode_path(cngpt_amd.DECODE_AUTO)
        draws = np.random.default_rng(7).random((dsteps + 1) * dB).astype(np.float32)
        samp_dt, _ = decode(m, cfg, dB, prompt, dsteps, draws)
        # per-kernel-class split of the sampled steps (direct launches, HIP events)
        m.profile_reset()
        m.profile(True)
        prof_dt, _ = decode(m, cfg, dB, prompt, dsteps, draws)
        m.profile(False)
        prof = m.profile_read()
        m.close()
        calib = copy_calibration(args.copy_calibration << 20) if args.copy_calibration else None
        n = dsteps
        print(json.dumps({"workload": name, "B": dB, "decode_tok_s": round(n * dB / dec_dt, 1),
                          "ms_per_step": round(dec_dt * 1e3 / n, 4),
                          "hbm_frac": round(dec_bytes / dec_dt / PEAK_HBM, 4),
                          "path": dec_path,
                          "kernels_path_ms_per_step": round(kern_dt * 1e3 / n, 4),
                          "sampled_tok_s": round(n * dB / samp_dt, 1),
                          "graphs": os.environ.get("CNGPT_HIP_GRAPH", "1") != "0",
                          "evented_ms_per_step": round(prof_dt * 1e3 / n, 4),
                          "kernel_us_per_step": {k: round(v["ms"] * 1e3 / n, 2)
                                                 for k, v in prof.items() if v["launches"]},
                          "launches_per_step": {k: round(v["launches"] / n, 2)
                                                for k, v in prof.items() if v["launches"]},
                          "bytes_per_step": round(dec_bytes / n),
                          "copy_calibration_bytes": calib}),
              flush=True)
        return

    dt, prof = prefill(m, cfg, B, T, args.steps, args.warmup)
    tokens = B * T * args.steps
    g = prof["gemm"]
    gemm_ms_avg = g["ms"] / g["launches"]
    achieved = g["flops"] / (g["ms"] * 1e-3)
    gemm_share = g["ms"] / (dt * 1e3)
    loss = loss_leg(m, cfg, B, T, args.steps)

    dec_dt, dec_path = decode(m, cfg, dB, prompt, dsteps)
    dec_bytes = decode_bytes(cfg, params.size, dB, prompt, dsteps)
    kern_ms = None
    if dec_path != "kernels":
        m.set_decode_path(cngpt_amd.DECODE_KERNELS)
        kern_dt, _ = decode(m, cfg, dB, prompt, dsteps)
        kern_ms = round(kern_dt * 1e3 / dsteps, 4)
        m.set_decode_path(cngpt_amd.DECODE_AUTO)
    draws = np.random.default_rng(7).random((dsteps + 1) * dB).astype(np.float32)
    samp_dt, _ = decode(m, cfg, dB, prompt, dsteps, draws)
    ref_shape = reference_shape(m) if name == "small" else None
    share = dp_share(m, cfg) if name == "small" else None
    load = load_leg(m, cfg, params)
    # training steps on the device at `cngpt train`'s default batch (4 x 1024)
    train = train_leg(m, cfg, 4, 1024, 5, 2) if name == "small" else None
    m.close()
    bdec = batched_decode() if name == "small" else None

    # HBM-side bytes per GEMM launch from the committed rocprofv3 --pmc
    # summary of this workload (FETCH_SIZE + WRITE_SIZE, calibrated).
    # (not measured in this run: rocprofv3 counters need a profiler run of
    # their own; the file names the commit and date of the kernels it read)
    traffic, tsrc = None, None
    tpath = os.path.join(ROOT, "profiles", "gemm_traffic.json")
    if name == "small" and os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic = tj.get("measured_bytes_per_launch")
        tsrc = {k: tj.get(k) for k in ("source", "kernels_commit", "measured_on")}
    # the single-sequence decode's HBM-side reads per step, likewise from a
    # committed rocprofv3 --pmc FETCH_SIZE summary
    dtraffic, dsrc = None, None
    dpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if name == "small" and dB == 1 and dec_path == "persistent" and os.path.exists(dpath):
        with open(dpath) as f:
            dj = json.load(f)
        dtraffic = dj.get("measured_fetch_bytes_per_step")
        dsrc = {k: dj.get(k) for k in ("source", "kernel", "kernels_commit", "measured_on")}

    line = {
        "metric": f"forward tokens/sec + GEMM MFMA util %, {NAMES[name]} fp32 B={B} T={T}; "
                  f"decode tok/s",
        "value": round(tokens / dt, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic: {data}, LCG token ids uniform in [0,{cfg.vocab_size})",
        "config": {"workload": f"{NAMES[name]} fp32 batched prefill, full logits "
                               f"[{B},{T},{cfg.vocab_size}]",
                   "B": B, "T": T, "n_layer": cfg.n_layer, "n_embd": cfg.n_embd,
                   "vocab": cfg.vocab_size, "logits": "all positions, left in HBM"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2),
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": traffic,
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE+WRITE_SIZE)",
                     "traffic_source": tsrc,
                     "kernel": "k_gemm (all MFMA linear layers + lm_head)",
                     "avg_launch_ms": round(gemm_ms_avg, 4),
                     "launches": g["launches"], "share_of_step": round(gemm_share, 4)},
        "gemm_mfma_util_pct": round(100 * achieved / PEAK_FP32_MFMA, 2),
        "loss": loss,
        "load": load,
        "train": train,
        "decode": {"tok_s": round(dsteps * dB / dec_dt, 1),
                   "ms_per_step": round(dec_dt * 1e3 / dsteps, 4),
                   "prompt": prompt, "steps": dsteps, "B": dB, "sampling": "greedy", "path": dec_path,
                   "kernels_path_ms_per_step": kern_ms,
                   "hbm": {"bound": "hbm", "achieved": round(dec_bytes / dec_dt / 1e9, 1),
                           "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                           "frac": round(dec_bytes / dec_dt / PEAK_HBM, 4),
                           "bytes_per_step": round(dec_bytes / dsteps),
                           "traffic": dtraffic,
                           "traffic_unit": "HBM-side read bytes per step (rocprofv3 FETCH_SIZE)",
                           "traffic_source": dsrc},
                   "sampled_tok_s": round(dsteps * dB / samp_dt, 1),
                   "sampled": "temp 0.8, top-k 40, device sample_top_k"},
        "kernels": {k: {"ms_per_step": round(v["ms"] / args.steps, 3),
                        "launches_per_step": v["launches"] // max(args.steps, 1),
                        **({"tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2)}
                           if v["flops"] and v["ms"] else {}),
                        **({"gbps": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1)}
                           if v["bytes"] and v["ms"] else {})}
                    for k, v in prof.items() if v["launches"]},
    }
    if ref_shape:
        line["reference_shape"] = ref_shape
    if share:
        line["dp_share"] = share
    if bdec:
        line["batched_decode"] = bdec
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(name, cfg, params, args.cpu_budget, B, T)
    if args.copy_calibration:
        line["copy_calibration_bytes"] = copy_calibration(args.copy_calibration << 20)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
