"""Benchmark of the quantized matmul path on one MI355X.

Headline (BASELINE.json metric): Q4_K GEMV at M=1 over the Llama-3-8B projection set
(q, k, v, o, gate, up, down), reported as whole-step HBM GB/s.  One "step" is the seven
projections of one decoder layer, back to back on one stream.  The packed weights are
rotated over enough copies (> 512 MB) that every step reads them from HBM, not from the
256 MB Infinity Cache.  Also reported: per-projection kernel times from HIP events on the
launch stream, the bf16-MFMA prefill GEMM at M=2048 (TFLOP/s), and the reference's CPU
path (dequantize all of W to fp32, then the naive fp32 loop; oracle/ restatement) timed
on the host.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-prefill]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SEED_BASE = 0x4D4C5852

# Llama-3-8B projections: (name, N = out_features, K = in_features)
LLAMA3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the M=2048 MFMA measurement")
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--rotate-mb", type=int, default=640, help="weight bytes rotated per pass (MB)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import mlxr_amd as mx

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    qt = mx.QuantType.Q4_K

    # ---------------------------------------------------------------- inputs
    gguf = {}
    for i, (name, N, K) in enumerate(LLAMA3_8B):
        gguf[name] = mx.synth_gguf(qt, N, K, SEED_BASE + 1 + 16 * i)
    layer_bytes = sum(mx.packed_size(qt, N, K) for _, N, K in LLAMA3_8B)
    ncopies = max(2, -(-args.rotate_mb * 1000000 // layer_bytes))
    copies = []
    for c in range(ncopies):
        copies.append({name: mx.pack_weights(gguf[name], N, K, qt, device=dev) for name, N, K in LLAMA3_8B})
    torch.cuda.synchronize()

    def act(n, seed, M=1):
        bits = mx.synth_act(M * n, mx.BF16, seed)
        return torch.from_numpy(bits.view(np.int16).reshape(M, n)).to(dev).view(torch.bfloat16)

    x_h = act(4096, SEED_BASE + 1001)
    x_i = act(14336, SEED_BASE + 1002)
    ys = {name: torch.empty((1, N), dtype=torch.bfloat16, device=dev) for name, N, K in LLAMA3_8B}

    def xin(K):
        return x_h if K == 4096 else x_i

    # algorithmic bytes: GGUF weight bytes + activations read once + outputs written once
    alg = {name: mx.gguf_size(qt, N, K) + K * 2 + N * 2 for name, N, K in LLAMA3_8B}
    step_bytes = sum(alg.values())
    stream = torch.cuda.current_stream()

    def step(c):
        W = copies[c % ncopies]
        for name, N, K in LLAMA3_8B:
            mx.q_gemm_dequant(xin(K), W[name], 1, N, K, qt, out=ys[name], path=mx.PATH_GEMV, stream=stream)

    # ---------------------------------------------------------------- timed steps
    for c in range(args.warmup):
        step(c)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for c in range(args.steps):
        step(c)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---------------------------------------------------------------- per-kernel HIP events
    reps = max(args.steps, 10)
    evs = {name: [] for name, _, _ in LLAMA3_8B}
    for c in range(reps):
        W = copies[c % ncopies]
        for name, N, K in LLAMA3_8B:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            mx.q_gemm_dequant(xin(K), W[name], 1, N, K, qt, out=ys[name], path=mx.PATH_GEMV, stream=stream)
            b.record(stream)
            evs[name].append((a, b))
    torch.cuda.synchronize()
    kern_us = {name: float(np.mean([a.elapsed_time(b) for a, b in evs[name]]) * 1e3) for name in evs}
    shapes = {name: {"N": N, "K": K, "us": round(kern_us[name], 3),
                     "GBps": round(alg[name] / (kern_us[name] * 1e-6) / 1e9, 1),
                     "frac_hbm": round(alg[name] / (kern_us[name] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
              for name, N, K in LLAMA3_8B}
    kern_total_us = sum(kern_us.values())
    achieved = step_bytes / (kern_total_us * 1e-6) / 1e9

    # ---------------------------------------------------------------- prefill MFMA, M=2048
    prefill = None
    if not args.no_prefill:
        M = 2048
        xp = {4096: act(4096, SEED_BASE + 3001, M), 14336: act(14336, SEED_BASE + 3002, M)}
        yp = {name: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for name, N, K in LLAMA3_8B}
        W = copies[0]
        for name, N, K in LLAMA3_8B:  # warmup
            mx.q_gemm_dequant(xp[K], W[name], M, N, K, qt, out=yp[name], path=mx.PATH_MFMA, stream=stream)
        torch.cuda.synchronize()
        pev = {name: [] for name, _, _ in LLAMA3_8B}
        for r in range(args.prefill_reps):
            for name, N, K in LLAMA3_8B:
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                mx.q_gemm_dequant(xp[K], W[name], M, N, K, qt, out=yp[name], path=mx.PATH_MFMA, stream=stream)
                b.record(stream)
                pev[name].append((a, b))
        torch.cuda.synchronize()
        p_us = {name: float(np.mean([a.elapsed_time(b) for a, b in pev[name]]) * 1e3) for name in pev}
        flops = {name: 2.0 * M * N * K for name, N, K in LLAMA3_8B}
        tot_tf = sum(flops.values()) / (sum(p_us.values()) * 1e-6) / 1e12
        prefill = {"M": M, "TFLOPs": round(tot_tf, 1), "frac_bf16_peak": round(tot_tf / BF16_PEAK_TFLOPS, 4),
                   "shapes": {name: {"us": round(p_us[name], 1),
                                     "TFLOPs": round(flops[name] / (p_us[name] * 1e-6) / 1e12, 1)}
                              for name, _, _ in LLAMA3_8B}}

    # ---------------------------------------------------------------- CPU baseline (oracle)
    cpu = None
    if not args.no_cpu:
        from oracle import orc
        orc.set_threads(1)
        xh = orc.bf16_bits_to_f32(x_h.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(1, -1)
        xi = orc.bf16_bits_to_f32(x_i.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(1, -1)
        runs = []
        for _ in range(3):
            t = time.perf_counter()
            for name, N, K in LLAMA3_8B:
                orc.eval_cpu(int(qt), 1, N, K, gguf[name], xh if K == 4096 else xi)
            runs.append(time.perf_counter() - t)
        sec = float(np.median(runs))
        cpu = {"value": round(step_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": "full Llama-3-8B Q4_K projection set at M=1 (7 GEMVs), reference eval_cpu restated: "
                         "fp32 dequant of all of W then naive fp32 loop, 1 thread, median of 3 runs",
               "seconds_per_step": round(sec, 3)}

    out = {
        "metric": "Q4_K qGEMM: HBM GB/s at M=1 (Llama-3-8B projection set)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x bf16 -> fp32 acc -> bf16",
        "data": "synthetic (BASELINE generator: d,dmin=|N(0,1)|*1e-3, uniform scales/quants; x ~ N(0,1) bf16)",
        "config": {"workload": "Llama-3-8B q,k,v,o,gate,up,down Q4_K GEMV, M=1, one decoder layer per step",
                   "M": 1, "weight_copies_rotated": ncopies, "rotated_MB": round(ncopies * layer_bytes / 1e6, 1),
                   "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qgemv_kernel<Q4_K,bf16,M=1>", "kernel_us_per_step": round(kern_total_us, 3)},
        "shapes": shapes,
        "prefill_mfma": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
