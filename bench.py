"""Benchmark: GPT-2 small fp32 batched forward, B=16, T=1024, full logits.

Prints one JSON line. value = forward tokens/s over the timed steps (tokens
already in HBM, logits [16, 1024, 50257] left in HBM); roofline = the MFMA
GEMM kernels (all linear layers and the lm_head) timed with HIP events on
the library's stream during the same steps, against MI355X's dense fp32
matrix peak. Also reported: single-stream decode tok/s (32-token prompt,
512 greedy steps with the KV cache) and the CPU oracle timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import cngpt_amd  # noqa: E402

PEAK_FP32_MFMA = 157.3e12   # 256 CUs x 2.4 GHz x 256 FLOP/clk/CU
PEAK_HBM = 8.0e12
METRIC = "forward tokens/sec + GEMM MFMA util %, GPT-2 small fp32 B=16 T=1024; decode tok/s"
SEED = 1234


def lcg_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """Token ids from the LCG of the reference's bench (src/cngpt.c:338-342)."""
    out = np.empty(n, dtype=np.int64)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (s >> 8) % vocab
    return out.astype(np.int32)


def prefill(m: cngpt_amd.Model, cfg, B: int, T: int, steps: int, warmup: int):
    tokens = lcg_tokens(B * T, cfg.vocab_size, 12345).reshape(B, T)
    m.reserve(B, T, cngpt_amd.ALL)
    m.upload_tokens(tokens)
    for _ in range(warmup):
        m.forward_resident(B, T, cngpt_amd.ALL)
    m.synchronize()
    m.profile_reset()
    m.profile(True)
    m.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.forward_resident(B, T, cngpt_amd.ALL)
    m.synchronize()
    dt = time.perf_counter() - t0
    m.profile(False)
    prof = m.profile_read()
    m.profile_reset()
    return dt, prof, tokens


def decode_bytes(cfg, params_n: int, B: int, first_pos: int, steps: int) -> float:
    """Algorithmic HBM bytes of `steps` decode steps whose tokens sit at
    positions first_pos.. : every weight once per step (wpe: one row), the
    K and V rows of keys 0..p, the new q/k/v row and the logits."""
    C, L, V = cfg.n_embd, cfg.n_layer, cfg.vocab_size
    weights = 4.0 * (params_n - cfg.block_size * C + C)
    total = 0.0
    for p in range(first_pos, first_pos + steps):
        total += weights + 4.0 * L * B * (p + 1) * 2 * C + 4.0 * L * B * 3 * C + 4.0 * B * V
    return total


def decode(m: cngpt_amd.Model, cfg, prompt_len: int, steps: int, draws=None):
    """`steps` single-token decode steps after a prompt_len prompt, B=1, as
    one cngpt_hip_generate call (one replayed HIP graph per step); greedy, or
    temp 0.8 / top-k 40 sampling when draws are given."""
    prompt = lcg_tokens(prompt_len, cfg.vocab_size, 777).reshape(1, prompt_len)
    kw = {} if draws is None else {"temperature": 0.8, "top_k": 40,
                                   "draws": draws[:steps + 1]}
    m.decode_begin(prompt, capacity=prompt_len + steps)
    warm = {} if draws is None else {"temperature": 0.8, "top_k": 40, "draws": draws[:8]}
    m.generate(8, **warm)                     # warm-up, captures the step graph
    m.decode_begin(prompt, capacity=prompt_len + steps)
    m.synchronize()
    t0 = time.perf_counter()
    m.generate(steps + 1, **kw)
    return time.perf_counter() - t0


def cpu_baseline(cfg, params, budget_s: float):
    """The oracle (C restatement of the reference's gpt_forward_fast with
    OpenBLAS, one pinned thread per physical core) on a bounded sample of
    the same workload: B=1 sequences of T=1024 tokens, all-position logits."""
    import oracle

    ocfg = oracle.Cfg(cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size)
    cores = oracle.set_threads(0)
    tk = lcg_tokens(1024, cfg.vocab_size, 12345).reshape(1, 1024)
    oracle.forward(ocfg, params, tk, oracle.ALL)            # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.forward(ocfg, params, tk, oracle.ALL)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n >= 20:
            break
    tok_s = n * 1024 / dt
    # the reference's own semantics: final-position logits (gpt_forward_fast)
    t1 = time.perf_counter()
    oracle.forward(ocfg, params, tk, oracle.LAST)
    last_s = time.perf_counter() - t1
    return {"value": round(tok_s, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} forward(s) of B=1 x T=1024 GPT-2 small fp32, all-position logits "
                      f"({dt:.1f} s); oracle C restatement of fast.c + {oracle.blas_info()}",
            "last_position_tok_s": round(1024 / last_s, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--decode-steps", type=int, default=512)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MiB",
                    help="also run one plain device copy of this size (counter calibration)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode legs (for kernel traces of the decode step)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    cfg = cngpt_amd.GPT2_SMALL
    B, T = 16, 1024
    params = cngpt_amd.init_weights(cfg, SEED)
    m = cngpt_amd.Model(cfg, params)

    if args.decode_only:
        dec_dt = decode(m, cfg, 32, args.decode_steps)
        dec_bytes = decode_bytes(cfg, params.size, 1, 32, args.decode_steps)
        # per-kernel-class split of the same steps (direct launches, HIP events)
        m.profile_reset()
        m.profile(True)
        prof_dt = decode(m, cfg, 32, args.decode_steps)
        m.profile(False)
        prof = m.profile_read()
        m.close()
        n = args.decode_steps
        print(json.dumps({"decode_tok_s": round(n / dec_dt, 1),
                          "ms_per_token": round(dec_dt * 1e3 / n, 4),
                          "hbm_frac": round(dec_bytes / dec_dt / PEAK_HBM, 4),
                          "graphs": os.environ.get("CNGPT_HIP_GRAPH", "1") != "0",
                          "evented_ms_per_token": round(prof_dt * 1e3 / n, 4),
                          "kernel_us_per_token": {k: round(v["ms"] * 1e3 / n, 2)
                                                  for k, v in prof.items() if v["launches"]},
                          "launches_per_token": {k: round(v["launches"] / n, 2)
                                                 for k, v in prof.items() if v["launches"]}}),
              flush=True)
        return

    dt, prof, _ = prefill(m, cfg, B, T, args.steps, args.warmup)
    tokens = B * T * args.steps
    g = prof["gemm"]
    gemm_ms_avg = g["ms"] / g["launches"]
    achieved = g["flops"] / (g["ms"] * 1e-3)
    gemm_share = g["ms"] / (dt * 1e3)

    dec_dt = decode(m, cfg, 32, args.decode_steps)
    dec_bytes = decode_bytes(cfg, params.size, 1, 32, args.decode_steps)
    draws = np.random.default_rng(7).random(args.decode_steps + 1).astype(np.float32)
    samp_dt = decode(m, cfg, 32, args.decode_steps, draws)
    m.close()

    # HBM-side bytes per GEMM launch from the committed rocprofv3 --pmc
    # summary of this workload (FETCH_SIZE + WRITE_SIZE, calibrated).
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("measured_bytes_per_launch")

    line = {
        "metric": METRIC,
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
        "data": "synthetic: seeded N(0,0.02) weights (srand 1234, gpt_init_weights order), "
                "LCG token ids uniform in [0,50257)",
        "config": {"workload": "GPT-2 small fp32 batched prefill, full logits [16,1024,50257]",
                   "B": B, "T": T, "n_layer": 12, "n_embd": 768, "vocab": 50257,
                   "logits": "all positions, left in HBM"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2),
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": traffic,
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE+WRITE_SIZE)",
                     "kernel": "k_gemm (all MFMA linear layers + lm_head)",
                     "avg_launch_ms": round(gemm_ms_avg, 4),
                     "launches": g["launches"], "share_of_step": round(gemm_share, 4)},
        "gemm_mfma_util_pct": round(100 * achieved / PEAK_FP32_MFMA, 2),
        "decode": {"tok_s": round(args.decode_steps / dec_dt, 1),
                   "ms_per_token": round(dec_dt * 1e3 / args.decode_steps, 4),
                   "prompt": 32, "steps": args.decode_steps, "B": 1, "sampling": "greedy",
                   "hbm": {"bound": "hbm", "achieved": round(dec_bytes / dec_dt / 1e9, 1),
                           "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                           "frac": round(dec_bytes / dec_dt / PEAK_HBM, 4),
                           "bytes_per_step": round(dec_bytes / args.decode_steps)},
                   "sampled_tok_s": round(args.decode_steps / samp_dt, 1),
                   "sampled": "temp 0.8, top-k 40, device sample_top_k"},
        "kernels": {k: {"ms_per_step": round(v["ms"] / args.steps, 3),
                        "launches_per_step": v["launches"] // max(args.steps, 1),
                        **({"tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2)}
                           if v["flops"] and v["ms"] else {}),
                        **({"gbps": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1)}
                           if v["bytes"] and v["ms"] else {})}
                    for k, v in prof.items() if v["launches"]},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, params, args.cpu_budget)
    if args.copy_calibration:
        line["copy_calibration_bytes"] = copy_calibration(args.copy_calibration << 20)
    print(json.dumps(line), flush=True)


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


if __name__ == "__main__":
    main()
