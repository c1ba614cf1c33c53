"""Benchmark of the quantized matmul path on one MI355X.

Headline (BASELINE.json metric): Q4_K GEMV at M=1 over the Llama-3-8B projection set
(q, k, v, o, gate, up, down), as HBM GB/s.  One "step" is one token through the projections
of the model's 32 decoder layers, each layer its own packed weights (3.9 GB in all, so
everything streams from HBM, not the 256 MB Infinity Cache), captured as one hipGraph as a
decode engine captures its model.  A layer is four launches -- q/k/v and gate/up read the
same input and run as one grouped launch each (mlxr_qgemm_run_grouped), o and down alone.
A graph of one layer (a graph launch per four kernels) is reported beside it.  Per-launch durations come from HIP events on
the launch stream around graphs of back-to-back launches of one kind.  The seven-call
drop-in step (one q_gemm_dequant per projection) is reported beside it.

The other BASELINE configurations are reported under "configs":
  c1  Q8_0 GEMV, TinyLlama-1.1B q_proj (M=1, K=N=2048, fp16)
  c3  Q4_K skinny GEMM, gate/up/down, M in {8,16,32,64} (GEMV kernel and MFMA kernel)
(c1, c3 and c4 time each call inside a replayed hipGraph of back-to-back calls, so host
launch overhead is not in their figures.)
  c4  Q4_K prefill GEMM, Llama-3-8B set, M in {512, 2048} (bf16 MFMA)
  c5  Llama-3-70B layer, Q4_K + Q6_K (v, down), 7 GEMMs in a hipGraph at M=1 and M=256,
      grouped as a decoder layer issues them (5 launches, plus split-K reduces at M=256)
  mlp (extra) Llama-3-8B gate/up + SwiGLU gating at M = 1, 8, 512, 2048: fused launch vs
      grouped projections + gating kernel
  lmhead (extra) Llama-3-8B output head as Q6_K GEMV at M=1 (N = 128256)
The CPU baseline is the reference's CPU path (dequantize all of W to fp32, then the naive
fp32 loop; restated in oracle/orc.c) on the headline workload, one thread.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--only headline,c1,...]
                    [--no-cpu] [--calib-copy-mb MB]
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
SEED_BASE = 0x4D4C5852  # + configuration index
ROTATE_BYTES = 640e6

LLAMA3_8B_LAYERS = 32
LLAMA3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
Q4K, Q6K, Q80 = 3, 4, 2
LLAMA3_70B = [("q", 8192, 8192, Q4K), ("k", 1024, 8192, Q4K), ("v", 1024, 8192, Q6K), ("o", 8192, 8192, Q4K),
              ("gate", 28672, 8192, Q4K), ("up", 28672, 8192, Q4K), ("down", 8192, 28672, Q6K)]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_llama3_8b_m1_traffic.txt")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="headline,c1,c3,c4,c5,mlp,lmhead")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--skip-dropin", action="store_true",
                    help="do not time the seven-call drop-in step (profiler runs of the headline kernel)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="at the end, run one device copy of this many MB (profiler calibration)")
    return ap.parse_args()


class Ctx:
    def __init__(self, torch, mx):
        self.torch, self.mx = torch, mx
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()

    def act(self, M, K, dtype_code, seed):
        bits = self.mx.synth_act(M * K, dtype_code, seed)
        t = self.torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(self.dev)
        return t.view(self.torch.bfloat16 if dtype_code == self.mx.BF16 else self.torch.float16)

    def event_ms(self, fn, reps):
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(self.stream)
        for r in range(reps):
            fn(r)
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    def graph_ms(self, fn, n, replays=5):
        """Per-call time of fn(0..n-1) captured into one graph and replayed (no host launch
        overhead in the figure)."""
        torch = self.torch
        g = self.graph(lambda: [fn(r) for r in range(n)])
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(self.stream)
        for _ in range(replays):
            g.replay()
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (replays * n)

    def graph(self, fn):
        """Capture fn() (library launches on the capture stream) into a CUDA/HIP graph."""
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()  # warm-up outside capture (first-call attribute setup)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):  # the warm-up stream (per-stream split-K workspace)
            fn()
        torch.cuda.synchronize()
        return g


_BLIB = None


def blib():
    """libmlxr_bench.so: the benchmark's measurement probes (stream read, MFMA rate), built
    beside the matmul library but not part of it."""
    global _BLIB
    if _BLIB is None:
        import ctypes
        path = os.path.join(ROOT, "mlxr_amd", "lib", "libmlxr_bench.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build with `python -m mlxr_amd.build`")
        lb = ctypes.CDLL(path)
        lb.mlxr_bench_stream_read.restype = ctypes.c_int
        lb.mlxr_bench_stream_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_int, ctypes.c_void_p]
        lb.mlxr_bench_empty.restype = ctypes.c_int
        lb.mlxr_bench_empty.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lb.mlxr_bench_mfma_peak.restype = ctypes.c_int
        lb.mlxr_bench_mfma_peak.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        _BLIB = lb
    return _BLIB


def bcheck(rc):
    if rc != 0:
        raise RuntimeError(f"bench probe launch failed (status {rc})")


def pack_arena(cx, specs, seed0, ncopies):
    """Like pack_copies, but each copy of the layer is one allocation holding its weights in
    spec order (256-byte aligned), as a model loader lays a layer out: the weights of one
    launch are then one contiguous byte range.  Returns (gguf, copies, arenas, ranges) with
    ranges[name] = (offset, packed bytes)."""
    mx, torch = cx.mx, cx.torch
    gguf = {name: mx.synth_gguf(qt, N, K, seed0 + 16 * i) for i, (name, N, K, qt) in enumerate(specs)}
    ranges, off = {}, 0
    for name, N, K, qt in specs:
        sz = mx.packed_size(qt, N, K)
        ranges[name] = (off, sz)
        off = (off + sz + 255) // 256 * 256
    copies, arenas = [], []
    for _ in range(ncopies):
        arena = torch.empty(off, dtype=torch.uint8, device=cx.dev)
        copies.append({name: mx.pack_weights(gguf[name], N, K, qt, out=arena[ranges[name][0]:sum(ranges[name])])
                       for name, N, K, qt in specs})
        arenas.append(arena)
    torch.cuda.synchronize()
    return gguf, copies, arenas, ranges


def pack_copies(cx, specs, seed0, min_copies=2):
    """specs: [(name, N, K, qtype)] -> (gguf dict, list of {name: PackedWeight})."""
    mx = cx.mx
    gguf = {name: mx.synth_gguf(qt, N, K, seed0 + 16 * i) for i, (name, N, K, qt) in enumerate(specs)}
    layer = sum(mx.packed_size(qt, N, K) for _, N, K, qt in specs)
    ncopies = max(min_copies, int(-(-ROTATE_BYTES // layer)))
    copies = [{name: mx.pack_weights(gguf[name], N, K, qt, device=cx.dev) for name, N, K, qt in specs}
              for _ in range(ncopies)]
    cx.torch.cuda.synchronize()
    return gguf, copies, layer


def gemm_bytes(mx, qt, M, N, K, xsz=2, ysz=2):
    return mx.gguf_size(qt, N, K) + M * K * xsz + M * N * ysz


def rel_errs(cx, pw, x, y, bf16_w, cols=None, rows=None):
    """Normwise max|y - ref| / max|ref| and elementwise max |y - ref| / |ref| over
    |ref| >= 1e-2 max|ref|, with ref = fp64 x . W^T on the GPU from the library's fp32
    dequant of the packed weight (bit-exact to the GGUF formulas, checked in the tests),
    rounded to bf16 first for the MFMA paths, which multiply bf16 weights.  cols / rows:
    slices of N and M (default all)."""
    torch = cx.torch
    W = cx.mx.dequantize(pw, torch.float32)
    if cols is not None:
        W = W[cols]
    if bf16_w:
        W = W.to(torch.bfloat16).float()
    xs = x if rows is None else x[rows]
    ys = y if rows is None else y[rows]
    if cols is not None:
        ys = ys[:, cols]
    ref = xs.double() @ W.double().t()
    d = (ys.double() - ref).abs()
    a = ref.abs()
    amax = a.max()
    big = a >= 1e-2 * amax
    norm = float(d.max() / amax) if amax > 0 else float(d.max())
    elem = float((d[big] / a[big]).max()) if amax > 0 and bool(big.any()) else 0.0
    del W
    return {"normwise": float(f"{norm:.3e}"), "elementwise": float(f"{elem:.3e}")}


def worst(errs):
    """The largest normwise and elementwise errors over a list of rel_errs results."""
    return {"normwise": max(e["normwise"] for e in errs), "elementwise": max(e["elementwise"] for e in errs)}


# ------------------------------------------------------------------------------ headline

def stream_read_ms(cx, args, launches):
    """Graph-replayed time of a sequence of launches that only stream-read the given packed
    weights (launches = [[PackedWeight, ...] per launch], one mlxr_bench_stream_read each):
    milliseconds per replay of the whole sequence.  Grid: 2048 workgroups (fewer for a
    launch under 8 MB), the best of the grid sizes tried on MI355X for these buffers
    (256 .. 16384 workgroups, per launch kind and for the whole step)."""
    import ctypes
    mx, torch = cx.mx, cx.torch
    sink = torch.zeros(1024, dtype=torch.int32, device=cx.dev)
    calls = []
    for pws in launches:
        ptrs = (ctypes.c_void_p * len(pws))(*[pw.data_ptr() for pw in pws])
        sizes = (ctypes.c_size_t * len(pws))(*[pw.nbytes for pw in pws])
        grid = int(min(-(-sum(pw.nbytes for pw in pws) // 4096), 2048))
        calls.append((len(pws), ptrs, sizes, grid))
    lib = blib()

    def seq():
        st = mx.qgemm._stream_ptr(None)
        for n, ptrs, sizes, grid in calls:
            bcheck(lib.mlxr_bench_stream_read(n, ptrs, sizes, sink.data_ptr(), grid, st))

    g = cx.graph(seq)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = cx.event_ms(lambda r: g.replay(), args.steps)
    del g
    return ms


def empty_launch_ms(cx, args, nlaunch, grid=2048):
    """Graph-replayed time of nlaunch launches of an empty kernel (grid workgroups of 256
    threads): milliseconds per replay.  The per-launch cost the step's structure pays before
    any bytes move."""
    torch = cx.torch
    lib = blib()

    def seq():
        st = cx.mx.qgemm._stream_ptr(None)
        for _ in range(nlaunch):
            bcheck(lib.mlxr_bench_empty(grid, None, st))

    g = cx.graph(seq)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = cx.event_ms(lambda r: g.replay(), args.steps)
    del g
    return ms


def copy_ms(cx, args, ranges):
    """Graph-replayed time of a sequence of device-to-device copies (hipMemcpyAsync through
    torch's copy_), one per launch: ranges = [(arena, offset, bytes)], each copied into one
    scratch buffer.  Milliseconds per replay of the whole sequence.  An independent reader
    beside the stream-read probe: the runtime's own copy of the same bytes in the same
    launch structure (its bytes read are the weights, counted once)."""
    torch = cx.torch
    dst = torch.empty(max(n for _, _, n in ranges), dtype=torch.uint8, device=cx.dev)

    def seq():
        for a, o, n in ranges:
            dst[:n].copy_(a[o:o + n])

    g = cx.graph(seq)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = cx.event_ms(lambda r: g.replay(), args.steps)
    del g, dst
    return ms


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the CPU baselines."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def run_headline(cx, args, out):
    mx, torch = cx.mx, cx.torch
    specs = [(n, N, K, Q4K) for n, N, K in LLAMA3_8B]
    # one packed copy per layer of the model (one allocation per layer, the weights in
    # projection order): the timed step streams 32 distinct layers
    gguf, copies, arenas, wr = pack_arena(cx, specs, SEED_BASE + 1, LLAMA3_8B_LAYERS)
    x = {4096: cx.act(1, 4096, mx.BF16, SEED_BASE + 1001), 14336: cx.act(1, 14336, mx.BF16, SEED_BASE + 1002)}
    ys = {n: torch.empty((1, N), dtype=torch.bfloat16, device=cx.dev) for n, N, K in LLAMA3_8B}
    dims = {n: (N, K) for n, N, K in LLAMA3_8B}
    alg = {n: gemm_bytes(mx, Q4K, 1, N, K) for n, N, K in LLAMA3_8B}
    step_bytes = sum(alg.values())
    # one decoder layer = 4 launches: the projections of one input run as one grouped launch
    LAUNCHES = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",))]
    span = {ln: (wr[names[0]][0], sum(wr[names[-1]]) - wr[names[0]][0]) for ln, names in LAUNCHES}

    def launch(W, names):
        K = dims[names[0]][1]
        if len(names) == 1:
            n = names[0]
            mx.q_gemm_dequant(x[K], W[n], 1, dims[n][0], K, Q4K, out=ys[n], path=mx.PATH_GEMV)
        else:
            mx.q_gemm_dequant_grouped(x[K], [W[n] for n in names], outs=[ys[n] for n in names])

    def step(W):
        for _, names in LAUNCHES:
            launch(W, names)

    def step7(W):
        for n, N, K in LLAMA3_8B:
            mx.q_gemm_dequant(x[K], W[n], 1, N, K, Q4K, out=ys[n], path=mx.PATH_GEMV)

    R = 12  # launches per timing graph (rotating weight copies)
    lbytes = {lname: sum(alg[n] for n in names) for lname, names in LAUNCHES}
    # per-launch durations: graphs of R back-to-back launches of one kind (no host overhead)
    kern_us = {}
    for lname, names in LAUNCHES:
        g = cx.graph(lambda names=names: [launch(copies[r % len(copies)], names) for r in range(R)])
        g.replay()
        torch.cuda.synchronize()
        kern_us[lname] = 1e3 * cx.event_ms(lambda r: g.replay(), max(args.steps // 2, 5)) / R
        del g
    # warm: the same launches on one weight copy, resident in the 256 MB Infinity Cache
    warm_us = {}
    for lname, names in LAUNCHES:
        g = cx.graph(lambda names=names: [launch(copies[0], names) for r in range(R)])
        g.replay()
        torch.cuda.synchronize()
        warm_us[lname] = 1e3 * cx.event_ms(lambda r: g.replay(), max(args.steps // 2, 5)) / R
        del g

    # the timed step: one token through the 32 layers' projections (4 launches per layer,
    # 128 in all, each layer its own weights), captured as one hipGraph as a decode engine
    # captures its model; HIP events on the launch stream bracket the timed replays
    model = cx.graph(lambda: [step(W) for W in copies])
    for _ in range(args.warmup):
        model.replay()
    torch.cuda.synchronize()
    ms_model = cx.event_ms(lambda r: model.replay(), args.steps)
    del model
    # the same step's launch structure with a pure streaming read of the same packed weight
    # buffers in place of each GEMV launch (libmlxr_bench stream read): the HBM ceiling of
    # 4 launches per layer, 128 per step, in one graph
    ms_ceiling = stream_read_ms(cx, args, [[W[n] for n in names] for W in copies for _, names in LAUNCHES])
    # and per launch kind: R back-to-back reads of one kind's buffers (as kern_us above)
    read_us = {lname: 1e3 * stream_read_ms(cx, args, [[copies[r % len(copies)][n] for n in names] for r in range(R)]) / R
               for lname, names in LAUNCHES}
    # an independent reader: the runtime's device-to-device copy of each launch's packed
    # bytes (one contiguous range per launch), in the same 128-launch structure and per kind
    ms_copy = copy_ms(cx, args, [(A, span[ln][0], span[ln][1]) for A in arenas for ln, _ in LAUNCHES])
    copy_us = {ln: 1e3 * copy_ms(cx, args, [(arenas[r % len(arenas)], span[ln][0], span[ln][1]) for r in range(R)]) / R
               for ln, _ in LAUNCHES}
    # the structure's own cost: as many empty launches as the step has
    ms_empty = empty_launch_ms(cx, args, len(copies) * len(LAUNCHES))
    # one layer per graph (a graph launch per 4 kernels), for comparison
    graphs = [cx.graph(lambda W=W: step(W)) for W in copies[:8]]
    for c in range(args.warmup):
        graphs[c % len(graphs)].replay()
    torch.cuda.synchronize()
    ms_graph = cx.event_ms(lambda r: graphs[r % len(graphs)].replay(), args.steps)
    graphs7 = []
    ms_graph7 = ms_eager7 = grouped_ok = None
    if not args.skip_dropin:
        # drop-in path: seven separate q_gemm_dequant calls per layer, graph-replayed and eager
        graphs7 = [cx.graph(lambda W=W: step7(W)) for W in copies]
        ms_graph7 = cx.event_ms(lambda r: graphs7[r % len(graphs7)].replay(), args.steps)
        ms_eager7 = cx.event_ms(lambda r: step7(copies[r % len(copies)]), args.steps)
        # the grouped graph's outputs equal seven separate calls on the same weights, bit for bit
        graphs[-1].replay()
        torch.cuda.synchronize()
        y_g = {n: ys[n].clone() for n in ys}
        step7(copies[len(graphs) - 1])
        torch.cuda.synchronize()
        grouped_ok = all(torch.equal(y_g[n], ys[n]) for n in ys)

    # the decoder's MLP block as it runs in a layer: mlxr_qgemm_mlp_ex (gate/up and the
    # gating in one launch, then down over the real h), two launches; and its one-launch
    # mode.  Same weights and launch count per layer as the step above minus one.
    ws_mlp = mx.MlpWorkspace(cx.dev)
    y_mlp = torch.empty((1, 4096), dtype=torch.bfloat16, device=cx.dev)
    mlp_ms = {}
    for mname, mode in (("chain", mx.qgemm.MLP_CHAIN), ("one_launch", mx.qgemm.MLP_ONE_LAUNCH)):
        def dstep(W, mode=mode):
            launch(W, ("q", "k", "v"))
            launch(W, ("o",))
            mx.q_gemm_mlp(x[4096], W["gate"], W["up"], W["down"], ws_mlp, out=y_mlp, mode=mode)
        g = cx.graph(lambda: [dstep(W) for W in copies])
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        mlp_ms[mname] = cx.event_ms(lambda r: g.replay(), args.steps)
        del g
    ws_mlp.status()

    # accuracy of one layer of the step (as the graph ran it): every output
    step(copies[0])
    torch.cuda.synchronize()
    head_err = worst([rel_errs(cx, copies[0][n], x[dims[n][1]], ys[n], False) for n, _, _ in LLAMA3_8B])

    traffic = traffic_src = None
    if os.path.exists(TRAFFIC_FILE):
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = float(line.split(":")[1])
            if line.startswith("measured:"):
                traffic_src = line.split(":", 1)[1].strip()

    nlaunch = len(copies) * len(LAUNCHES)
    step_gbs = len(copies) * step_bytes / (ms_model * 1e-3) / 1e9
    out.update({
        "value": round(step_gbs, 1),
        "ms_per_step": round(ms_model, 5),
        "roofline": {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "qgemv_lds_kernel<Q4_K,bf16,M=1>: every launch of the step (128: qkv, o, gate_up, "
                               "down per layer)",
                     "achieved_from": "algorithmic bytes per step / ms_per_step (HIP events on the launch stream "
                                      "over the timed replays); per launch: alg_bytes_per_launch / us_per_launch",
                     "alg_bytes_per_launch": round(step_bytes / len(LAUNCHES)),
                     "us_per_launch_in_step": round(1e3 * ms_model / nlaunch, 3),
                     "traffic_from": "profiles/q4k_gemv_llama3_8b_m1_traffic.txt (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                     "mean bytes per launch; measured %s), not measured in this run" % traffic_src},
        "headline_detail": {
            "max_rel_err": head_err,
            "layers_per_step": len(copies), "layer_bytes": step_bytes,
            "us_per_layer": round(1e3 * ms_model / len(copies), 3),
            "stream_read_ceiling": {
                "what": "pure non-temporal streaming read of the same packed weight buffers in the same "
                        "launch structure (4 launches per layer, 128 per step, one graph), nothing computed; "
                        "2048 workgroups per launch, the best grid of a 256-16384 sweep",
                "ms_per_step": round(ms_ceiling, 5),
                "GBps": round(len(copies) * step_bytes / (ms_ceiling * 1e-3) / 1e9, 1),
                "frac_hbm": round(len(copies) * step_bytes / (ms_ceiling * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "gemv_step_vs_ceiling": round(ms_ceiling / ms_model, 4)},
            "launch_floor": {
                "what": "the same number of graph nodes (128) launching an empty kernel of 2048 workgroups: the "
                        "per-launch cost of this structure before any bytes move; max_frac_hbm = the step's bytes at "
                        "8 TB/s plus this floor",
                "ms_per_step": round(ms_empty, 5),
                "us_per_launch": round(1e3 * ms_empty / nlaunch, 3),
                "max_frac_hbm": round((len(copies) * step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3)
                                      / (len(copies) * step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3 + ms_empty), 4)},
            "copy_ceiling": {
                "what": "the runtime's device-to-device copy (hipMemcpyAsync via torch copy_) of each launch's "
                        "packed weight bytes (one contiguous range per launch) in the same 128-launch graph; "
                        "GBps counts the bytes read once (the copy also writes them)",
                "ms_per_step": round(ms_copy, 5),
                "GBps": round(len(copies) * step_bytes / (ms_copy * 1e-3) / 1e9, 1),
                "frac_hbm": round(len(copies) * step_bytes / (ms_copy * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "gemv_step_vs_copy": round(ms_copy / ms_model, 4)},
            "one_layer_graph_ms": round(ms_graph, 5),
            "one_layer_graph_GBps": round(step_bytes / (ms_graph * 1e-3) / 1e9, 1),
            "launches": {ln: {"us": round(kern_us[ln], 3), "bytes": lbytes[ln],
                              "GBps": round(lbytes[ln] / (kern_us[ln] * 1e-6) / 1e9, 1),
                              "frac_hbm": round(lbytes[ln] / (kern_us[ln] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                              "stream_read_us": round(read_us[ln], 3),
                              "vs_stream_read": round(read_us[ln] / kern_us[ln], 4),
                              "copy_us": round(copy_us[ln], 3),
                              "vs_copy": round(copy_us[ln] / kern_us[ln], 4)}
                         for ln, _ in LAUNCHES},
            "warm_launches_infinity_cache": {ln: {"us": round(warm_us[ln], 3),
                                                  "GBps": round(lbytes[ln] / (warm_us[ln] * 1e-6) / 1e9, 1)}
                                             for ln, _ in LAUNCHES},
            "decoder_mlp_step": {
                "what": "the same 32 layers with the MLP block as a decoder runs it (mlxr_qgemm_mlp_ex: down over "
                        "the real h); GBps over the same layer bytes",
                **{k: {"ms_per_step": round(v, 5), "GBps": round(len(copies) * step_bytes / (v * 1e-3) / 1e9, 1),
                       "launches_per_layer": 4 if k == "chain" else 3} for k, v in mlp_ms.items()}},
            "dropin_7_calls_graph_ms": ms_graph7 and round(ms_graph7, 5),
            "dropin_7_calls_graph_GBps": ms_graph7 and round(step_bytes / (ms_graph7 * 1e-3) / 1e9, 1),
            "dropin_7_calls_eager_ms": ms_eager7 and round(ms_eager7, 5),
            "grouped_equals_separate_calls": grouped_ok,
            "weight_copies_rotated": len(copies), "rotated_MB": round(sum(a.numel() for a in arenas) / 1e6, 1)},
    })

    if not args.no_cpu:
        from oracle import orc
        orc.set_threads(1)
        xf = {k: orc.bf16_bits_to_f32(v.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(1, -1)
              for k, v in x.items()}
        runs = []
        for _ in range(5):
            t = time.perf_counter()
            for n, N, K in LLAMA3_8B:
                orc.eval_cpu(Q4K, 1, N, K, gguf[n], xf[K])
            runs.append(time.perf_counter() - t)
        sec = float(np.median(runs))
        out["cpu_baseline"] = {
            "value": round(step_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "one layer of the headline step (Llama-3-8B Q4_K q,k,v,o,gate,up,down at M=1) through the "
                      "reference eval_cpu restated in oracle/orc.c: fp32 dequant of all of W, then the naive "
                      "fp32 loop; 1 thread; median of 5 runs",
            "seconds_per_step": round(sec, 4), "cpu_model": cpu_model()}
        # "MLX-CPU-class" baseline: the same fp32 dequant on every core of this process's
        # CPU share (OpenMP over rows), then a BLAS fp32 GEMV (torch on the host)
        cores = min(len(os.sched_getaffinity(0)), 16)
        orc.set_threads(cores)
        nthr = torch.get_num_threads()
        torch.set_num_threads(cores)
        xt = {k: torch.from_numpy(v) for k, v in xf.items()}
        dq_runs, mm_runs = [], []
        for _ in range(5):
            tdq = tmm = 0.0
            for n, N, K in LLAMA3_8B:
                t = time.perf_counter()
                w = orc.dequant(Q4K, N, K, gguf[n])
                tdq += time.perf_counter() - t
                t = time.perf_counter()
                torch.matmul(xt[K], torch.from_numpy(w).t())
                tmm += time.perf_counter() - t
                del w
            dq_runs.append(tdq)
            mm_runs.append(tmm)
        orc.set_threads(1)
        torch.set_num_threads(nthr)
        dq, mm = float(np.median(dq_runs)), float(np.median(mm_runs))
        out["cpu_baseline_all_cores"] = {
            "value": round(step_bytes / (dq + mm) / 1e9, 3), "unit": "GB/s", "cores": cores,
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "kind": "port", "dequant_s": round(dq, 4), "matmul_s": round(mm, 4),
            "sample": "one layer of the headline step: oracle fp32 dequant (OpenMP) + host BLAS fp32 GEMV "
                      "(torch.matmul), all cores of the process's CPU share; median of 5 runs"}
    del graphs, graphs7, copies, arenas
    torch.cuda.empty_cache()


# ------------------------------------------------------------------------------ other configs

def run_c1(cx, args):
    mx, torch = cx.mx, cx.torch
    N = K = 2048
    _, copies, _ = pack_copies(cx, [("q", N, K, Q80)], SEED_BASE + 0, min_copies=8)
    x = cx.act(1, K, mx.F16, SEED_BASE + 2001)
    y = torch.empty((1, N), dtype=torch.float16, device=cx.dev)
    fn = lambda r: mx.q_gemm_dequant(x, copies[r % len(copies)]["q"], 1, N, K, Q80, out=y, path=mx.PATH_GEMV)
    for r in range(args.warmup):
        fn(r)
    us = 1e3 * cx.graph_ms(fn, len(copies))
    b = gemm_bytes(mx, Q80, 1, N, K)
    fn(0)
    err = rel_errs(cx, copies[0]["q"], x, y, False)
    # ceiling: a pure streaming read of the same packed weights, one launch per call
    read_us = 1e3 * stream_read_ms(cx, args, [[c["q"]] for c in copies]) / len(copies)
    return {"shape": "M=1 K=2048 N=2048 Q8_0, x/y fp16", "us": round(us, 3), "GBps": round(b / us / 1e3, 1),
            "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "alg_bytes": b, "max_rel_err": err,
            "stream_read_us": round(read_us, 3), "vs_stream_read": round(read_us / us, 4)}


def run_c3(cx, args):
    mx, torch = cx.mx, cx.torch
    specs = [(n, N, K, Q4K) for n, N, K in LLAMA3_8B if n in ("gate", "up", "down")]
    _, copies, _ = pack_copies(cx, specs, SEED_BASE + 2)
    res = {}
    for M in (8, 16, 32, 64):
        x = {4096: cx.act(M, 4096, mx.BF16, SEED_BASE + 3000 + M), 14336: cx.act(M, 14336, mx.BF16, SEED_BASE + 3100 + M)}
        row = {}
        for n, N, K, _ in specs:
            y = torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev)
            b = gemm_bytes(mx, Q4K, M, N, K)
            for path, pname in ((mx.PATH_GEMV, "gemv"), (mx.PATH_MFMA, "mfma")):
                fn = lambda r: mx.q_gemm_dequant(x[K], copies[r % len(copies)][n], M, N, K, Q4K, out=y, path=path)
                fn(0)
                us = 1e3 * cx.graph_ms(fn, 2 * len(copies))
                fn(0)
                err = rel_errs(cx, copies[0][n], x[K], y, path == mx.PATH_MFMA)
                row[f"{n}_{pname}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1),
                                       "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "max_rel_err": err}
        res[f"M={M}"] = row
    # ceiling per weight: a pure streaming read of the same packed bytes, one launch per call
    res["stream_read_us"] = {n: round(1e3 * stream_read_ms(cx, args, [[c[n]] for c in copies]) / len(copies), 3)
                             for n, _, _, _ in specs}
    return res


def run_c4(cx, args):
    mx, torch = cx.mx, cx.torch
    specs = [(n, N, K, Q4K) for n, N, K in LLAMA3_8B]
    _, copies, _ = pack_copies(cx, specs, SEED_BASE + 3, min_copies=1)
    W = copies[0]
    res = {}
    for M in (512, 2048):
        x = {4096: cx.act(M, 4096, mx.BF16, SEED_BASE + 4000 + M), 14336: cx.act(M, 14336, mx.BF16, SEED_BASE + 4100 + M)}
        tot_f = tot_us = 0.0
        shapes = {}
        for n, N, K in LLAMA3_8B:
            y = torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev)
            fn = lambda r: mx.q_gemm_dequant(x[K], W[n], M, N, K, Q4K, out=y, path=mx.PATH_MFMA)
            fn(0)
            us = 1e3 * cx.graph_ms(fn, 5 if M == 2048 else 10)
            f = 2.0 * M * N * K
            fn(0)
            # every column, rows in three 64-row slices (first, middle, last)
            errs = [rel_errs(cx, W[n], x[K], y, True, rows=slice(m0, m0 + 64)) for m0 in (0, M // 2, M - 64)]
            shapes[n] = {"us": round(us, 1), "TFLOPs": round(f / us / 1e6, 1), "max_rel_err": worst(errs)}
            tot_f += f
            tot_us += us
        # the same seven GEMMs as a decoder layer issues them: q/k/v and gate/up as grouped
        # calls (one tiled launch each), o and down alone -- 4 calls
        ys = {n: torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev) for n, N, K in LLAMA3_8B}
        dims = {n: (N, K) for n, N, K in LLAMA3_8B}

        def layer(r):
            for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
                K = dims[names[0]][1]
                if len(names) == 1:
                    n = names[0]
                    mx.q_gemm_dequant(x[K], W[n], M, dims[n][0], K, Q4K, out=ys[n])
                else:
                    mx.q_gemm_dequant_grouped(x[K], [W[n] for n in names], outs=[ys[n] for n in names])
        layer(0)
        lus = 1e3 * cx.graph_ms(layer, 2 if M == 2048 else 4)
        res[f"M={M}"] = {"TFLOPs": round(tot_f / tot_us / 1e6, 1),
                         "frac_bf16_peak": round(tot_f / tot_us / 1e6 / BF16_PEAK_TFLOPS, 4), "shapes": shapes,
                         "layer_grouped_4_calls": {"us": round(lus, 1), "TFLOPs": round(tot_f / lus / 1e6, 1),
                                                   "frac_bf16_peak": round(tot_f / lus / 1e6 / BF16_PEAK_TFLOPS, 4)}}
    # context only: a plain (unquantized) bf16 GEMM of the same gate shape through torch's
    # library path (hipBLASLt), i.e. what the MFMA units give without any dequant work
    M, N, K = 2048, 14336, 4096
    a = cx.act(M, K, mx.BF16, SEED_BASE + 4200)
    b = torch.randn((N, K), dtype=torch.bfloat16, device=cx.dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev)
    fn = lambda r: torch.matmul(a, b.t(), out=y)
    fn(0)
    us = 1e3 * cx.graph_ms(fn, 5)
    res["plain_bf16_gemm_library_M2048_gate"] = {"us": round(us, 1), "TFLOPs": round(2.0 * M * N * K / us / 1e6, 1)}
    # ceiling: back-to-back bf16 MFMAs from registers on every SIMD, no memory traffic
    # (mlxr_bench_mfma_peak) -- the rate the matrix cores sustain here, clock throttling
    # under full load included
    cus = torch.cuda.get_device_properties(cx.dev).multi_processor_count
    iters = 1024
    out = torch.empty(cus * 256, dtype=torch.float32, device=cx.dev)
    lib = blib()
    fn = lambda r: bcheck(lib.mlxr_bench_mfma_peak(cus, iters, out.data_ptr(), torch.cuda.current_stream().cuda_stream))
    fn(0)
    us = 1e3 * cx.graph_ms(fn, 4)
    tf = cus * 4 * iters * 16 * 32768 / us / 1e6
    res["mfma_ceiling"] = {"TFLOPs": round(tf, 1), "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4),
                           "c4_M2048_vs_ceiling": round(res["M=2048"]["TFLOPs"] / tf, 4),
                           "c4_M2048_layer_vs_ceiling": round(res["M=2048"]["layer_grouped_4_calls"]["TFLOPs"] / tf, 4)}
    return res


def run_mlp(cx, args):
    """Llama-3-8B MLP gate/up half (K = 4096, N = 14336) at M = 1, 8, 512 and 2048: the fused
    gate + up + gating launch (mlxr_qgemm_swiglu; GEMV, narrow skinny and tiled kernels)
    against the grouped gate/up projections followed by the gating kernel.  Not a BASELINE
    config (the reference plans the fusion in swiglu_mlp_fused.metal:131-345)."""
    mx, torch = cx.mx, cx.torch
    specs = [(n, N, K, Q4K) for n, N, K in LLAMA3_8B if n in ("gate", "up")]
    _, copies, _ = pack_copies(cx, specs, SEED_BASE + 6)
    N, K = 14336, 4096
    res = {}
    for M in (1, 8, 512, 2048):
        x = cx.act(M, K, mx.BF16, SEED_BASE + 6001 + M)
        h = torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev)
        g = torch.empty_like(h)
        u = torch.empty_like(h)
        fused = lambda r: mx.q_gemm_swiglu(x, copies[r % len(copies)]["gate"], copies[r % len(copies)]["up"], out=h)

        def unfused(r):
            W = copies[r % len(copies)]
            mx.q_gemm_dequant_grouped(x, [W["gate"], W["up"]], outs=[g, u])
            mx.swiglu(g, u, out=h)

        b = 2 * mx.gguf_size(Q4K, N, K) + M * K * 2 + M * N * 2
        f = 2.0 * 2 * M * N * K
        row = {}
        for name, fn in (("fused", fused), ("grouped_plus_gating", unfused)):
            fn(0)
            us = 1e3 * cx.graph_ms(fn, 2 * len(copies) if M <= 8 else 4)
            row[name] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1), "TFLOPs": round(f / us / 1e6, 1)}
        # accuracy of the fused launch: fp64 gating of fp64 gate/up (bf16 weights where the
        # MFMA kernels run), 256 columns at both ends
        fused(0)
        torch.cuda.synchronize()
        errs = []
        for cols in (slice(0, 256), slice(N - 256, N)):
            rows = None if M <= 64 else slice(0, 64)
            ref = []
            for nm in ("gate", "up"):
                W = mx.dequantize(copies[0][nm], torch.float32)[cols]
                if M > 4:
                    W = W.to(torch.bfloat16).float()
                xs = x if rows is None else x[rows]
                ref.append(xs.double() @ W.double().t())
            r = ref[0] / (1.0 + torch.exp(-ref[0])) * ref[1]
            hs = (h if rows is None else h[rows])[:, cols].double()
            d, a = (hs - r).abs(), r.abs()
            big = a >= 1e-2 * a.max()
            errs.append({"normwise": float(f"{float(d.max() / a.max()):.3e}"),
                         "elementwise": float(f"{float((d[big] / a[big]).max()):.3e}")})
        row["fused_max_rel_err"] = worst(errs)
        row["fused_speedup"] = round(row["grouped_plus_gating"]["us"] / row["fused"]["us"], 3)
        res[f"M={M}"] = row
    return res


def run_lmhead(cx, args):
    """Llama-3-8B lm_head as Q6_K (the Q4_K_M layout keeps the output head in Q6_K): GEMV at
    M=1, N = 128256 (vocabulary), K = 4096; 431 MB of weights, over two packed copies so
    consecutive calls stream from HBM.  Not a BASELINE config."""
    mx, torch = cx.mx, cx.torch
    N, K = 128256, 4096
    _, copies, _ = pack_copies(cx, [("head", N, K, Q6K)], SEED_BASE + 7, min_copies=2)
    x = cx.act(1, K, mx.BF16, SEED_BASE + 7001)
    y = torch.empty((1, N), dtype=torch.bfloat16, device=cx.dev)
    fn = lambda r: mx.q_gemm_dequant(x, copies[r % len(copies)]["head"], 1, N, K, Q6K, out=y, path=mx.PATH_GEMV)
    fn(0)
    us = 1e3 * cx.graph_ms(fn, 2 * len(copies))
    b = gemm_bytes(mx, Q6K, 1, N, K)
    # ceiling: a pure streaming read of the same packed weights, one launch per call
    read_us = 1e3 * stream_read_ms(cx, args, [[c["head"]] for c in copies]) / len(copies)
    return {"shape": "M=1 N=128256 K=4096 Q6_K, x/y bf16", "us": round(us, 2), "GBps": round(b / us / 1e3, 1),
            "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "stream_read_us": round(read_us, 2),
            "vs_stream_read": round(read_us / us, 4)}


def run_c5(cx, args):
    mx, torch = cx.mx, cx.torch
    _, copies, layer = pack_copies(cx, LLAMA3_70B, SEED_BASE + 4, min_copies=2)
    res = {"weight_bytes_per_layer": sum(mx.gguf_size(qt, N, K) for _, N, K, qt in LLAMA3_70B)}
    for M in (1, 256):
        x = {8192: cx.act(M, 8192, mx.BF16, SEED_BASE + 5000 + M), 28672: cx.act(M, 28672, mx.BF16, SEED_BASE + 5100 + M)}
        ys = {n: torch.empty((M, N), dtype=torch.bfloat16, device=cx.dev) for n, N, K, qt in LLAMA3_70B}

        def layer_fn(W):
            # projections of one input as grouped calls, as a decoder layer issues them:
            # q,k (Q4_K) in one launch + v (Q6_K), o, gate/up in one launch, down (GEMV at
            # M = 1, tiled MFMA GEMM at M = 256)
            for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
                K = dict((n, k) for n, _, k, _ in LLAMA3_70B)[names[0]]
                mx.q_gemm_dequant_grouped(x[K], [W[n] for n in names], outs=[ys[n] for n in names])
        graphs = [cx.graph(lambda W=W: layer_fn(W)) for W in copies]
        for r in range(2):
            graphs[r % len(graphs)].replay()
        torch.cuda.synchronize()
        ms = cx.event_ms(lambda r: graphs[r % len(graphs)].replay(), 10 if M == 1 else 4)
        graphs[0].replay()
        torch.cuda.synchronize()
        rows = None if M == 1 else slice(0, 64)
        err = worst([rel_errs(cx, copies[0][n], x[K], ys[n], M > 4, rows=rows) for n, _, K, _ in LLAMA3_70B])
        byts = sum(gemm_bytes(mx, qt, M, N, K) for _, N, K, qt in LLAMA3_70B)
        flops = sum(2.0 * M * N * K for _, N, K, qt in LLAMA3_70B)
        res[f"M={M}"] = {"ms_per_layer": round(ms, 4), "launches_per_layer": 5,
                         "GBps": round(byts / (ms * 1e-3) / 1e9, 1),
                         "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
                         "frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "max_rel_err": err}
        del graphs
        if M == 1:
            # ceiling: the same five launches as pure streaming reads of the same packed weights
            groups = (("q", "k"), ("v",), ("o",), ("gate", "up"), ("down",))
            rms = stream_read_ms(cx, args, [[W[n] for n in g] for W in copies for g in groups]) / len(copies)
            res["M=1"]["stream_read_ms_per_layer"] = round(rms, 4)
            res["M=1"]["vs_stream_read"] = round(rms / ms, 4)
        if M > 4:
            # beside it: the seven projections as seven separate calls
            def sep_fn(W):
                for n, N, K, qt in LLAMA3_70B:
                    mx.q_gemm_dequant(x[K], W[n], M, N, K, qt, out=ys[n])
            graphs = [cx.graph(lambda W=W: sep_fn(W)) for W in copies]
            graphs[0].replay()
            torch.cuda.synchronize()
            ms7 = cx.event_ms(lambda r: graphs[r % len(graphs)].replay(), 4)
            res[f"M={M}"]["separate_7_calls"] = {"ms_per_layer": round(ms7, 4),
                                                 "TFLOPs": round(flops / (ms7 * 1e-3) / 1e12, 1)}
            del graphs
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import mlxr_amd as mx

    torch.cuda.set_device(0)
    cx = Ctx(torch, mx)
    only = set(args.only.split(","))
    out = {
        "metric": "Q4_K qGEMM: HBM GB/s at M=1 (Llama-3-8B projection set)",
        "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k weights x bf16 activations, fp32 accumulate, bf16 out",
        "data": "synthetic (BASELINE generators: Q4_K d,dmin=|N(0,1)|*1e-3, uniform scales/quants; x ~ N(0,1))",
        "config": {"workload": "Llama-3-8B q,k,v,o,gate,up,down Q4_K GEMV at M=1; one step = one token through "
                               "the 32 layers (distinct weights, 3.9 GB), 4 launches per layer (grouped qkv, o, "
                               "grouped gate_up, down), one hipGraph", "M": 1},
        "roofline": None, "cpu_baseline": None,
    }
    if "headline" in only:
        run_headline(cx, args, out)
    configs = {}
    for key, fn in (("c1_q8_0_gemv_tinyllama", run_c1), ("c3_q4k_skinny", run_c3), ("c4_q4k_prefill", run_c4),
                    ("c5_llama3_70b_layer_graph", run_c5), ("mlp_swiglu", run_mlp),
                    ("lmhead_q6k_llama3_8b_m1", run_lmhead)):
        if key.split("_")[0] in only:
            configs[key] = fn(cx, args)
            torch.cuda.empty_cache()
    if configs:
        out["configs"] = configs
    c4 = configs.get("c4_q4k_prefill")
    if c4:
        # the metric's other half: the prefill GEMM at M = 2048 on the matrix cores
        r = c4["M=2048"]
        out["roofline_prefill"] = {
            "bound": "mfma", "achieved": r["TFLOPs"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": r["frac_bf16_peak"], "traffic": None,
            "kernel": "qgemm_tile_kernel<Q4_K> (tiled bf16 MFMA GEMM; the seven Llama-3-8B projections at M=2048 "
                      "as seven graph-replayed calls)",
            "layer_as_4_grouped_calls": r["layer_grouped_4_calls"],
            "mfma_ceiling_TFLOPs": c4["mfma_ceiling"]["TFLOPs"]}
    if args.calib_copy_mb:
        # one device copy of a known size, for scaling the profiler's traffic counters
        nb = args.calib_copy_mb * 1000000
        src = torch.empty(nb, dtype=torch.uint8, device=cx.dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
