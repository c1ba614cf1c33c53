"""Python host side of the quantized matmul: ctypes over libmlxr_qgemm.so.

Mirrors the reference operator (core/kernels/primitives/q_gemm_dequant_primitive.h):
``QuantType`` keeps the enum values (:18-35), ``q_gemm_dequant(input, weights, M, N, K,
quant_type, group_size, bias)`` keeps the argument order and meaning (:211-215), and
errors raise ``RuntimeError`` subclasses with the messages of the reference where it has
one (.mm:490-496).  torch tensors are used only as device memory and streams; every
computation runs in the HIP library, and the module raises if that library is missing.
"""
import ctypes
import enum
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libmlxr_qgemm.so")

F32, F16, BF16 = 0, 1, 2
MLP_AUTO, MLP_CHAIN, MLP_ONE_LAUNCH = 0, 1, 2
MLP_H_OFFSET = 163840  # MLXR_MLP_H_OFFSET: byte offset of h in an MLP workspace
PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2


class QuantType(enum.IntEnum):
    Q4_0 = 0
    Q4_1 = 1
    Q8_0 = 2
    Q4_K = 3
    Q6_K = 4
    Q5_0 = 5
    Q5_1 = 6
    Q8_1 = 7
    Q2_K = 8
    Q3_K = 9
    Q5_K = 10
    Q8_K = 11
    IQ2_XXS = 12
    IQ2_XS = 13
    IQ3_XXS = 14
    IQ3_S = 15


class Item(ctypes.Structure):
    """mlxr_qgemm_item."""
    _fields_ = [("qtype", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int), ("group_size", ctypes.c_int),
                ("packed_dev", ctypes.c_void_p), ("bias_dev", ctypes.c_void_p), ("bias_dtype", ctypes.c_int),
                ("y_dev", ctypes.c_void_p), ("y_dtype", ctypes.c_int)]


class QGemmError(RuntimeError):
    """A nonzero status from the C ABI; ``code`` holds the MLXR_E_* value."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


_lib = None

_SIGS = {
    "mlxr_qgemm_version": (ctypes.c_int, []),
    "mlxr_qgemm_last_error": (ctypes.c_char_p, []),
    "mlxr_qgemm_gguf_size": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_group_size": (ctypes.c_int, [ctypes.c_int]),
    "mlxr_qgemm_type_name": (ctypes.c_char_p, [ctypes.c_int]),
    "mlxr_qgemm_packed_size": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_pack": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "mlxr_qgemm_pack_device": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "mlxr_qgemm_dequant": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_run": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_run_ex": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_workspace_size": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_run_ws": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_qgemm_run_noalloc": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p] * 2 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_swiglu_workspace_size": (ctypes.c_int, [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_swiglu": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_swiglu": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_run_grouped": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "mlxr_qgemm_run_grouped_ws": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_qgemm_grouped_workspace_size": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_mlp_workspace_size": (ctypes.c_int, [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_size_t)]),
    "mlxr_qgemm_mlp_workspace_init": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_qgemm_mlp": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_qgemm_mlp_ex": (ctypes.c_int, [ctypes.c_int] * 4 + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mlxr_qgemm_mlp_status": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "mlxr_qgemm_test_set_operand_limit": (ctypes.c_int, [ctypes.c_size_t]),
    "mlxr_qgemm_test_set_mlp_spin_limit": (ctypes.c_int, [ctypes.c_uint]),
    "mlxr_qgemm_test_force_skinny": (ctypes.c_int, [ctypes.c_int]),
    "mlxr_qgemm_test_skinny_stage": (ctypes.c_int, [ctypes.c_int]),
    "mlxr_qgemm_auto_path": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(ctypes.c_int)]),
    "mlxr_synth_gguf": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p]),
    "mlxr_synth_act": (ctypes.c_int, [ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p]),
}


def lib():
    """The loaded HIP library.  Raises if it has not been built (no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mlxr_amd.build` "
                               "(there is no non-HIP implementation)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _check(rc):
    if rc != 0:
        raise QGemmError(rc, lib().mlxr_qgemm_last_error().decode())


# ----------------------------------------------------------------- metadata helpers

def gguf_size(qtype, N, K):
    """N * ceil(K/group) * sizeof(block) (reference compute_quantized_weight_size)."""
    v = ctypes.c_size_t()
    _check(lib().mlxr_qgemm_gguf_size(int(qtype), N, K, ctypes.byref(v)))
    return v.value


compute_quantized_weight_size = gguf_size


def packed_size(qtype, N, K):
    v = ctypes.c_size_t()
    _check(lib().mlxr_qgemm_packed_size(int(qtype), N, K, ctypes.byref(v)))
    return v.value


def get_default_group_size(qtype):
    return lib().mlxr_qgemm_group_size(int(qtype))


def quant_type_name(qtype):
    return lib().mlxr_qgemm_type_name(int(qtype)).decode()


_BPW = {QuantType.Q4_0: 18 / 32, QuantType.Q4_1: 20 / 32, QuantType.Q8_0: 34 / 32,
        QuantType.Q4_K: 144 / 256, QuantType.Q5_K: 176 / 256, QuantType.Q6_K: 210 / 256}


def get_bytes_per_weight(qtype):
    """Bytes per weight (reference QGemmDequantPrimitive::get_bytes_per_weight, .mm:63-78)."""
    try:
        return _BPW[QuantType(qtype)]
    except (KeyError, ValueError):
        raise QGemmError(-2, "Unsupported quantization type") from None


# ------------------------------------------------------------------ synthetic inputs

def synth_gguf(qtype, N, K, seed):
    """Deterministic GGUF blocks (numpy uint8) with the benchmark distributions."""
    out = np.empty(gguf_size(qtype, N, K), dtype=np.uint8)
    _check(lib().mlxr_synth_gguf(int(qtype), N, K, seed, out.ctypes.data))
    return out


def synth_act(count, dtype, seed):
    """count N(0,1) values rounded to dtype (BF16/F16 -> uint16 bits, F32 -> float32)."""
    out = np.empty(count, dtype=np.float32 if dtype == F32 else np.uint16)
    _check(lib().mlxr_synth_act(count, dtype, seed, out.ctypes.data))
    return out


# ------------------------------------------------------------------ device operations

def _torch():
    import torch
    return torch


def _stream_ptr(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dt_code(dtype):
    torch = _torch()
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[dtype]


class PackedWeight:
    """A weight repacked into the library's HBM layout (device uint8 tensor)."""

    def __init__(self, buf, qtype, N, K):
        self.buf, self.qtype, self.N, self.K = buf, QuantType(qtype), N, K

    def data_ptr(self):
        return self.buf.data_ptr()

    @property
    def nbytes(self):
        return self.buf.numel()


def pack_weights(gguf, N, K, qtype, device="cuda", stream=None, out=None):
    """One-time upload of GGUF blocks (numpy/CPU tensor/device tensor) to the packed layout.

    The packed buffer and any device staging copy are allocated on the stream the pack runs
    on (torch's stream-ordered allocator), so a staging copy freed on return is reused only
    after the pack.  ``out``: a contiguous uint8 device tensor of packed_size bytes to pack
    into instead (e.g. a slice of one allocation that holds a whole layer)."""
    torch = _torch()
    need = gguf_size(qtype, N, K)
    if isinstance(gguf, np.ndarray):
        gguf = torch.from_numpy(np.ascontiguousarray(gguf).view(np.uint8).reshape(-1))
    if gguf.numel() * gguf.element_size() < need:
        raise QGemmError(-1, "weights buffer is smaller than N * K/group * sizeof(block)")
    if out is not None:
        if out.dtype != torch.uint8 or out.dim() != 1 or not out.is_contiguous() or \
                out.numel() != packed_size(qtype, N, K) or out.device.type != "cuda":
            raise QGemmError(-1, "out must be a contiguous uint8 device tensor of packed_size bytes")
        device = out.device
    with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
        buf = out if out is not None else torch.empty(packed_size(qtype, N, K), dtype=torch.uint8, device=device)
        if gguf.device.type == "cpu":
            gguf = gguf.to(device, non_blocking=False)
        elif not gguf.is_contiguous():
            gguf = gguf.contiguous()
        _check(lib().mlxr_qgemm_pack_device(int(qtype), N, K, gguf.data_ptr(), buf.data_ptr(), _stream_ptr(stream)))
    if stream is None:
        torch.cuda.current_stream().synchronize()  # one-time upload: done when it returns
    return PackedWeight(buf, qtype, N, K)


def _check_out(t, M, N, device, what="out"):
    """A caller's output tensor: contiguous [M, N] fp32/fp16/bf16 on the input's device."""
    torch = _torch()
    if tuple(t.shape) != (M, N) or not t.is_contiguous() or t.device != device or \
            t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise QGemmError(-1, f"{what} must be a contiguous [{M}, {N}] float32/float16/bfloat16 tensor on {device}")


def _check_bias(b, N, device):
    if b is None:
        return None
    if b.dim() != 1 or b.shape[0] != N:
        raise QGemmError(-3, "Bias shape must be [N]")
    if b.device != device:
        raise QGemmError(-1, f"bias must be on {device}")
    return b.contiguous()


def dequantize(pw, dtype=None, stream=None):
    """[N, K] fp32 (bit-exact GGUF formulas) or bf16 (RNE of those) from a packed weight."""
    torch = _torch()
    dtype = dtype or torch.float32
    out = torch.empty((pw.N, pw.K), dtype=dtype, device=pw.buf.device)
    _check(lib().mlxr_qgemm_dequant(int(pw.qtype), pw.N, pw.K, pw.data_ptr(), out.data_ptr(),
                                    _dt_code(dtype), _stream_ptr(stream)))
    return out


def q_gemm_dequant(input, weights, M, N, K, quant_type, group_size=0, bias=None, out=None,
                   out_dtype=None, path=PATH_AUTO, stream=None):
    """Y[M,N] = input[M,K] . W[N,K]^T (+ bias), fp32 accumulation.

    Same arguments as the reference's q_gemm_dequant (q_gemm_dequant_primitive.h:211-215).
    ``weights`` is a PackedWeight, or raw GGUF bytes (uint8 tensor on the device) which are
    packed for this call.  Output dtype defaults to the input dtype.
    """
    torch = _torch()
    if input.dim() != 2 or input.shape[0] != M or input.shape[1] != K:
        raise QGemmError(-3, "Input shape must be [M, K]")
    bias = _check_bias(bias, N, input.device)
    if not isinstance(weights, PackedWeight):
        weights = pack_weights(weights, N, K, quant_type, device=input.device, stream=stream)
    elif (weights.qtype, weights.N, weights.K) != (QuantType(quant_type), N, K):
        raise QGemmError(-3, "packed weights do not match (quant_type, N, K)")
    if not input.is_contiguous():
        input = input.contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or input.dtype, device=input.device)
    _check_out(out, M, N, input.device)
    # split-K workspace from torch's stream-ordered caching allocator (graph-capture safe)
    ws_bytes = workspace_size(quant_type, N, K, M) if path != PATH_GEMV else 0
    ws = None
    if ws_bytes:
        with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=input.device)
    _check(lib().mlxr_qgemm_run_ws(int(quant_type), N, K, group_size, weights.data_ptr(), input.data_ptr(),
                                   _dt_code(input.dtype), bias.data_ptr() if bias is not None else None,
                                   _dt_code(bias.dtype) if bias is not None else F32, out.data_ptr(),
                                   _dt_code(out.dtype), M, path, ws.data_ptr() if ws is not None else None,
                                   ws_bytes, _stream_ptr(stream)))
    return out


def auto_path(qtype, N, K, M):
    """The kernel family PATH_AUTO runs an [M, N, K] call on: PATH_GEMV or PATH_MFMA."""
    v = ctypes.c_int(0)
    _check(lib().mlxr_qgemm_auto_path(int(qtype), N, K, M, ctypes.byref(v)))
    return v.value


def workspace_size(qtype, N, K, M):
    """Device workspace bytes q_gemm_dequant uses for split-K at this shape (0 = none)."""
    out = ctypes.c_size_t(0)
    _check(lib().mlxr_qgemm_workspace_size(int(qtype), int(N), int(K), int(M), ctypes.byref(out)))
    return out.value


def q_gemm_dequant_grouped(input, weights, outs=None, biases=None, out_dtype=None, stream=None, workspace=True):
    """y_i = input . W_i^T (+ bias_i) for packed weights that read the same input (e.g. the
    q/k/v or gate/up projections), in as few launches as the library can (one per four
    same-type weights at M <= 4 and in the tiled GEMM).  With `workspace` (default) the
    library's split-K workspace comes from torch's allocator (mlxr_qgemm_run_grouped_ws);
    without it the call is mlxr_qgemm_run_grouped.  Returns the list of outputs."""
    torch = _torch()
    M, K = input.shape
    if not input.is_contiguous():
        input = input.contiguous()
    n = len(weights)
    biases = biases or [None] * n
    if outs is None:
        outs = [torch.empty((M, w.N), dtype=out_dtype or input.dtype, device=input.device) for w in weights]
    if len(outs) != n or len(biases) != n:
        raise QGemmError(-1, "one output and one bias (or None) per weight")
    biases = [_check_bias(b, w.N, input.device) for w, b in zip(weights, biases)]
    arr = (Item * n)()
    for i, (w, y, b) in enumerate(zip(weights, outs, biases)):
        if w.K != K:
            raise QGemmError(-3, "Input shape must be [M, K]")
        _check_out(y, M, w.N, input.device, f"outs[{i}]")
        arr[i] = Item(int(w.qtype), w.N, w.K, 0, w.data_ptr(), b.data_ptr() if b is not None else None,
                      _dt_code(b.dtype) if b is not None else F32, y.data_ptr(), _dt_code(y.dtype))
    if not workspace:
        _check(lib().mlxr_qgemm_run_grouped(n, arr, input.data_ptr(), _dt_code(input.dtype), M, _stream_ptr(stream)))
        return outs
    nb = ctypes.c_size_t(0)
    _check(lib().mlxr_qgemm_grouped_workspace_size(n, arr, M, ctypes.byref(nb)))
    ws = None
    if nb.value:
        with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
            ws = torch.empty(nb.value, dtype=torch.uint8, device=input.device)
    _check(lib().mlxr_qgemm_run_grouped_ws(n, arr, input.data_ptr(), _dt_code(input.dtype), M,
                                           ws.data_ptr() if ws is not None else None, nb.value, _stream_ptr(stream)))
    return outs


def q_gemm_swiglu(input, gate, up, out=None, out_dtype=None, stream=None, workspace=True):
    """h = swish(input . gate^T) * (input . up^T) for packed gate/up weights of one shape
    (mlxr_qgemm_swiglu: one launch computes both projections and the gating; with
    workspace, launches whose tiles cannot fill the device split K into a workspace and
    add one reduce launch)."""
    torch = _torch()
    M, K = input.shape
    if (gate.qtype, gate.N, gate.K) != (up.qtype, up.N, up.K) or gate.K != K:
        raise QGemmError(-3, "gate and up must be packed weights of the same type and [N, K]")
    if not input.is_contiguous():
        input = input.contiguous()
    if out is None:
        out = torch.empty((M, gate.N), dtype=out_dtype or input.dtype, device=input.device)
    _check_out(out, M, gate.N, input.device)
    n = ctypes.c_size_t(0)
    _check(lib().mlxr_qgemm_swiglu_workspace_size(int(gate.qtype), gate.N, K, M, _dt_code(out.dtype), ctypes.byref(n)))
    ws = None
    if n.value and workspace:
        with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
            ws = torch.empty(n.value, dtype=torch.uint8, device=input.device)
    _check(lib().mlxr_qgemm_swiglu(int(gate.qtype), gate.N, K, gate.data_ptr(), up.data_ptr(), input.data_ptr(),
                                   _dt_code(input.dtype), out.data_ptr(), _dt_code(out.dtype), M,
                                   ws.data_ptr() if ws is not None else None, n.value if ws is not None else 0,
                                   _stream_ptr(stream)))
    return out



class MlpWorkspace:
    """Device workspace of the fused MLP (mlxr_qgemm_mlp): sync words (zeroed once here, left
    zero by every launch), the gated intermediate h, split-K partials.  Grows on demand;
    calls that share one must not overlap."""

    def __init__(self, device):
        self.device, self.buf = device, None

    def get(self, nbytes, stream=None):
        torch = _torch()
        if self.buf is None or self.buf.numel() < nbytes:
            with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
                self.buf = torch.empty(max(nbytes, MLP_H_OFFSET), dtype=torch.uint8, device=self.device)
            _check(lib().mlxr_qgemm_mlp_workspace_init(self.buf.data_ptr(), self.buf.numel(), _stream_ptr(stream)))
        return self.buf

    def status(self, stream=None):
        """Raises QGemmError (MLXR_E_TIMEOUT) if a launch on this workspace gave up its wait."""
        if self.buf is not None:
            _check(lib().mlxr_qgemm_mlp_status(self.buf.data_ptr(), _stream_ptr(stream)))


def mlp_workspace_size(qtype_gu, qtype_down, hidden, inter, M):
    n = ctypes.c_size_t(0)
    _check(lib().mlxr_qgemm_mlp_workspace_size(int(qtype_gu), int(qtype_down), int(hidden), int(inter), int(M),
                                               ctypes.byref(n)))
    return n.value


def q_gemm_mlp(input, gate, up, down, workspace, out=None, out_dtype=None, stream=None, mode=MLP_AUTO):
    """y = down . (swish(input . gate^T) * (input . up^T)) (mlxr_qgemm_mlp_ex): the fused
    gate/up/gating launch and the down projection, or with mode=MLP_ONE_LAUNCH (M = 1) one
    launch for the whole MLP.  ``workspace`` is an MlpWorkspace."""
    torch = _torch()
    M, H = input.shape
    if (gate.qtype, gate.N, gate.K) != (up.qtype, up.N, up.K) or gate.K != H:
        raise QGemmError(-3, "gate and up must be packed weights of the same type and [inter, hidden]")
    if (down.N, down.K) != (H, gate.N):
        raise QGemmError(-3, "down must be a packed [hidden, inter] weight")
    if not input.is_contiguous():
        input = input.contiguous()
    if out is None:
        out = torch.empty((M, H), dtype=out_dtype or input.dtype, device=input.device)
    _check_out(out, M, H, input.device)
    need = mlp_workspace_size(gate.qtype, down.qtype, H, gate.N, M)
    ws = workspace.get(need, stream)
    _check(lib().mlxr_qgemm_mlp_ex(int(gate.qtype), int(down.qtype), H, gate.N, gate.data_ptr(), up.data_ptr(),
                                   down.data_ptr(), input.data_ptr(), _dt_code(input.dtype), out.data_ptr(),
                                   _dt_code(out.dtype), M, int(mode), ws.data_ptr(), ws.numel(), _stream_ptr(stream)))
    return out


def test_set_operand_limit(nbytes):
    """Test hook: lower the 2 GiB single-launch operand limit (0 restores it)."""
    _check(lib().mlxr_qgemm_test_set_operand_limit(int(nbytes)))


def test_set_mlp_spin_limit(ticks):
    """Test hook: the fused MLP's wait bound in 100 MHz ticks (0 restores 0.2 s)."""
    _check(lib().mlxr_qgemm_test_set_mlp_spin_limit(int(ticks)))


def test_force_skinny(on):
    """Test hook: send every MFMA-family call to the skinny kernel (any M, in 64-row blocks
    of M above 32) while on."""
    _check(lib().mlxr_qgemm_test_force_skinny(1 if on else 0))


def test_skinny_stage(mode):
    """Test hook: whether the narrow skinny kernel stages its activations in LDS where they
    fit (True / 1, the default); False / 0: it reads them from global memory at every step;
    2: two slabs per workgroup share their stages wherever that fits."""
    _check(lib().mlxr_qgemm_test_skinny_stage(int(mode)))
