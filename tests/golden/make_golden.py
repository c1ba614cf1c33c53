"""Writes the golden fixtures in this directory (small GGUF blocks, their fp32
dequantization, and a tiny GEMM per type with fp64-accumulated outputs).

Inputs come from the library's deterministic synthetic generator (mlxr_synth_*), outputs
from the CPU oracle (oracle/orc.c); the reference ships no vectors for this path.
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import mlxr_amd as mx  # noqa: E402
from oracle import orc  # noqa: E402

# (name, qtype, N, K for the dequant blocks, x dtype of the GEMM)
CASES = [("q8_0", 2, 2, 256, mx.F16), ("q4_k", 3, 4, 1024, mx.BF16), ("q6_k", 4, 4, 1024, mx.BF16),
         ("q4_0", 0, 4, 256, mx.BF16), ("q4_1", 1, 4, 256, mx.F16), ("q5_k", 10, 4, 1024, mx.BF16)]
GEMM_M, GEMM_N, GEMM_K = 3, 256, 512


def make():
    for i, (name, qt, N, K, xdt) in enumerate(CASES):
        blocks = mx.synth_gguf(qt, N, K, 0x60 + i)
        deq = orc.dequant(qt, N, K, blocks)
        w = mx.synth_gguf(qt, GEMM_N, GEMM_K, 0x70 + i)
        xbits = mx.synth_act(GEMM_M * GEMM_K, xdt, 0x80 + i)
        xf = (orc.bf16_bits_to_f32(xbits) if xdt == mx.BF16 else orc.f16_bits_to_f32(xbits)).reshape(GEMM_M, GEMM_K)
        y64 = orc.gemm_f64(qt, GEMM_M, GEMM_N, GEMM_K, w, xf)
        y64b = orc.gemm_f64(qt, GEMM_M, GEMM_N, GEMM_K, w, xf, w_to_bf16=True)
        ycpu = orc.eval_cpu(qt, GEMM_M, GEMM_N, GEMM_K, w, xf)
        np.savez(os.path.join(HERE, f"{name}.npz"), qtype=np.int32(qt), N=np.int32(N), K=np.int32(K),
                 blocks=blocks, dequant=deq, gemm_w=w, gemm_x_bits=xbits, gemm_x_dtype=np.int32(xdt),
                 gemm_shape=np.array([GEMM_M, GEMM_N, GEMM_K], np.int32), gemm_y_f64=y64,
                 gemm_y_f64_wbf16=y64b, gemm_y_eval_cpu=ycpu)


if __name__ == "__main__":
    make()
