"""ctypes wrapper of the CPU oracle (oracle/orc.c).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build
            build.build()
        l = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        l.orc_f16_to_f32.restype = ctypes.c_float
        l.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.orc_ref_fp16_to_fp32.restype = ctypes.c_float
        l.orc_ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        l.orc_f32_to_f16.restype = ctypes.c_uint16
        l.orc_f32_to_f16.argtypes = [ctypes.c_float]
        l.orc_bf16_to_f32.restype = ctypes.c_float
        l.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        l.orc_f32_to_bf16.restype = ctypes.c_uint16
        l.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        l.orc_weight_bytes.restype = ctypes.c_uint64
        l.orc_weight_bytes.argtypes = [I, I, I]
        l.orc_block_bytes.argtypes = [I]
        l.orc_block_elems.argtypes = [I]
        l.orc_dequant.argtypes = [I, I, I, P, P]
        l.orc_eval_cpu.argtypes = [I, I, I, I, P, P, P, P]
        l.orc_eval_cpu_cols.argtypes = [I, I, I, I, I, I, P, P, P, P]
        l.orc_gemm_f64.argtypes = [I, I, I, I, P, P, P, I, I, I, P]
        l.orc_dequant_refcpu_q4.argtypes = [I, P, P]
        _lib = l
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def f16_to_f32(codes):
    l = lib()
    return np.array([l.orc_f16_to_f32(int(c)) for c in codes], dtype=np.float32)


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def dequant(qtype, N, K, w):
    out = np.empty((N, K), dtype=np.float32)
    rc = lib().orc_dequant(int(qtype), N, K, _p(np.ascontiguousarray(w)), _p(out))
    if rc:
        raise ValueError(f"orc_dequant rc={rc}")
    return out


def dequant_refcpu_q4(qtype, block):
    """The reference CPU routine's element order for one Q4_0/Q4_1 block (32 floats)."""
    b = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.empty(32, np.float32)
    assert lib().orc_dequant_refcpu_q4(int(qtype), _p(b), _p(out)) == 0
    return out


def eval_cpu(qtype, M, N, K, w, x_f32, bias=None):
    """Restatement of the reference eval_cpu: fp32 dequant of all of W, naive fp32 loop."""
    y = np.empty((M, N), dtype=np.float32)
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_eval_cpu(int(qtype), M, N, K, _p(np.ascontiguousarray(w)), _p(x), _p(b), _p(y))
    if rc:
        raise ValueError(f"orc_eval_cpu rc={rc}")
    return y


def eval_cpu_cols(qtype, M, N, K, n0, n1, w, x_f32, bias=None):
    y = np.zeros((M, N), dtype=np.float32)
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().orc_eval_cpu_cols(int(qtype), M, N, K, n0, n1, _p(np.ascontiguousarray(w)), _p(x), _p(b), _p(y))
    if rc:
        raise ValueError(f"orc_eval_cpu_cols rc={rc}")
    return y


def gemm_f64(qtype, M, N, K, w, x_f32, bias=None, w_to_bf16=False, m0=0, m1=None, w_to_f16=False):
    """fp64-accumulated tolerance oracle over the exact dequantized weights, rows [m0, m1).

    w_to_bf16 / w_to_f16 first round the weights to bf16 / fp16 (RNE): the operands the MFMA
    paths multiply for bf16 / fp16 activations."""
    m1 = M if m1 is None else m1
    y = np.empty((m1 - m0, N), dtype=np.float32)
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    wr = 2 if w_to_f16 else (1 if w_to_bf16 else 0)
    rc = lib().orc_gemm_f64(int(qtype), M, N, K, _p(np.ascontiguousarray(w)), _p(x), _p(b), wr, m0, m1, _p(y))
    if rc:
        raise ValueError(f"orc_gemm_f64 rc={rc}")
    return y


def set_threads(n):
    """OpenMP thread count of the oracle (1 for the faithful single-core baseline)."""
    import ctypes.util
    name = ctypes.util.find_library("gomp")
    if name:
        ctypes.CDLL(name).omp_set_num_threads(int(n))


def normwise_rel_err(y, ref):
    """max_i |y_i - ref_i| / max_i |ref_i|."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / den) if den > 0 else float(np.max(np.abs(y - ref)))


def elementwise_rel_err(y, ref, floor=1e-2):
    """max_i |y_i - ref_i| / |ref_i| over the outputs with |ref_i| >= floor * max_j |ref_j|.

    The floor keeps the metric away from the zeros of a random dot product, where a
    relative error is ill-posed; 0.0 when no output qualifies (all-zero ref)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    a = np.abs(ref)
    big = a >= floor * np.max(a) if a.size else a.astype(bool)
    if not np.any(big) or np.max(a) == 0:
        return 0.0
    return float(np.max(np.abs(y[big] - ref[big]) / a[big]))


def rel_err(y, ref):
    """The larger of the normwise and the elementwise relative errors (both must meet a
    tolerance)."""
    return max(normwise_rel_err(y, ref), elementwise_rel_err(y, ref))
