"""C-ABI library checks that need no GPU: it loads, exports every symbol the headers
declare, reports sizes/names like the reference helpers, and rejects bad arguments with
the documented status codes before touching a device."""
import ctypes
import os
import re
import subprocess
import threading

import numpy as np
import pytest

import mlxr_amd as mx
from mlxr_amd import qgemm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "mlxr_qgemm.h")
C_HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
             if h.startswith("mlxr_") and h.endswith(".h")]


def test_exports_every_declared_symbol():
    names = set()
    for h in C_HEADERS:
        names |= set(re.findall(r"\b(mlxr_\w+)\s*\(", open(h).read()))
    assert len(names) >= 30
    lib = ctypes.CDLL(qgemm.LIB_PATH)
    for n in sorted(names):
        assert hasattr(lib, n), n
    # the C++ operator interface is exported too
    out = subprocess.run(["nm", "-D", "--defined-only", qgemm.LIB_PATH], capture_output=True, text=True).stdout
    for sym in ("q_gemm_dequant", "pack_weights", "compute_quantized_weight_size", "quant_type_name",
                "QGemmDequantPrimitive"):
        assert sym in out


def test_metadata_matches_reference_helpers():
    assert mx.lib().mlxr_qgemm_version() >= 10000
    assert [mx.quant_type_name(t) for t in range(16)] == [
        "Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q6_K", "Q5_0", "Q5_1", "Q8_1", "Q2_K", "Q3_K", "Q5_K", "Q8_K",
        "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S"]
    assert mx.quant_type_name(99) == "Unknown"
    assert mx.get_default_group_size(mx.QuantType.Q8_0) == 32
    assert mx.get_default_group_size(mx.QuantType.Q4_K) == 256
    assert mx.get_default_group_size(mx.QuantType.Q6_K) == 256
    assert mx.gguf_size(mx.QuantType.Q4_K, 14336, 4096) == 33030144
    assert mx.gguf_size(mx.QuantType.Q6_K, 8192, 28672) == 192675840
    assert mx.gguf_size(mx.QuantType.Q8_0, 2048, 2048) == 4456448
    assert mx.gguf_size(mx.QuantType.Q4_0, 1, 32) == 18  # reference parser test: Q4_0 = 18 B / 32
    assert mx.get_bytes_per_weight(mx.QuantType.Q4_K) < 1.0
    for qt, N, K in ((3, 14336, 4096), (4, 1024, 8192), (2, 2048, 2048), (3, 3, 256), (0, 5, 96), (1, 7, 4096), (10, 9, 512)):
        ps, gs = mx.packed_size(qt, N, K), mx.gguf_size(qt, N, K)
        assert gs <= ps < gs + 4 * 256  # same bytes, planes 256-byte aligned


def _err(fn):
    with pytest.raises(mx.QGemmError) as e:
        fn()
    return e.value


def test_error_paths():
    L = mx.lib()
    e = _err(lambda: mx.packed_size(mx.QuantType.Q2_K, 16, 256))
    assert e.code == -2 and "Unsupported quantization type Q2_K" in str(e)
    e = _err(lambda: mx.packed_size(mx.QuantType.Q4_K, 16, 300))
    assert e.code == -3 and "multiple" in str(e)
    e = _err(lambda: mx.packed_size(mx.QuantType.Q6_K, 0, 256))
    assert e.code == -1
    run = L.mlxr_qgemm_run_ex
    p = ctypes.c_void_p(8)
    assert run(3, 16, 256, 128, p, p, 2, None, 0, p, 2, 1, 0, None) == -3  # group size mismatch
    assert run(3, 16, 256, 0, p, p, 0, None, 0, p, 2, 1, 0, None) == -1    # fp32 activations
    assert run(3, 16, 256, 0, p, p, 2, None, 0, p, 7, 1, 0, None) == -1    # bad output dtype
    assert run(3, 16, 256, 0, p, p, 2, p, 9, p, 2, 1, 0, None) == -1       # bad bias dtype
    assert run(3, 16, 256, 0, p, p, 2, None, 0, p, 2, 65, 1, None) == -1   # GEMV path, M > 64
    assert run(3, 16, 256, 0, p, p, 2, None, 0, p, 2, 1, 5, None) == -1    # bad path
    assert run(3, 16, 256, 0, None, p, 2, None, 0, p, 2, 1, 0, None) == -1  # null weights
    assert run(3, 16, 256, 0, p, p, 2, None, 0, p, 2, -1, 0, None) == -1   # negative M
    assert run(3, 16, 256, 0, p, p, 2, None, 0, p, 2, 0, 0, None) == 0     # M = 0: nothing to do
    assert L.mlxr_qgemm_dequant(3, 16, 256, p, p, 1, None) == -1          # fp16 dequant output
    assert L.mlxr_qgemm_pack_device(3, 16, 256, None, p, None) == -1


def test_last_error_is_thread_local():
    L = mx.lib()
    assert L.mlxr_qgemm_packed_size(8, 1, 256, ctypes.byref(ctypes.c_size_t())) == -2
    seen = []
    t = threading.Thread(target=lambda: seen.append(L.mlxr_qgemm_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert b"Q2_K" in L.mlxr_qgemm_last_error()


def test_python_operator_shape_checks():
    torch = pytest.importorskip("torch")
    x = torch.zeros((2, 256), dtype=torch.bfloat16)
    w = torch.zeros(mx.gguf_size(3, 8, 256), dtype=torch.uint8)
    with pytest.raises(mx.QGemmError, match=r"Input shape must be \[M, K\]"):
        mx.q_gemm_dequant(x, w, 1, 8, 256, mx.QuantType.Q4_K, 256)
    with pytest.raises(mx.QGemmError, match=r"Bias shape must be \[N\]"):
        mx.q_gemm_dequant(x, w, 2, 8, 256, mx.QuantType.Q4_K, 256, bias=torch.zeros(9))


def test_synthetic_generators():
    a = mx.synth_gguf(mx.QuantType.Q6_K, 64, 512, 5)
    assert np.array_equal(a, mx.synth_gguf(mx.QuantType.Q6_K, 64, 512, 5))
    assert not np.array_equal(a, mx.synth_gguf(mx.QuantType.Q6_K, 64, 512, 6))
    b6 = a.reshape(-1, 210)
    sc = b6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d6 = b6[:, 208:210].copy().view(np.float16).astype(np.float64)
    assert (d6 >= 0).all() and 0.6e-3 < d6.mean() < 1.0e-3  # E|N(0,1)| * 1e-3 = 0.798e-3
    q8 = mx.synth_gguf(mx.QuantType.Q8_0, 256, 1024, 7).reshape(-1, 34)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() == -127 and qs.max() == 127
    d8 = q8[:, 0:2].copy().view(np.float16).astype(np.float64)
    assert 0.6 * 0.02 / 127 < d8.mean() < 1.0 * 0.02 / 127
    x = mx.synth_act(100000, mx.F32, 9)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02


def test_cpp_operator_interface(tmp_path):
    exe = tmp_path / "test_q_gemm_api"
    cmd = ["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "cpp", "test_q_gemm_api.cpp"), "-o", str(exe),
           "-L", os.path.dirname(qgemm.LIB_PATH), "-lmlxr_qgemm", "-Wl,-rpath," + os.path.dirname(qgemm.LIB_PATH)]
    subprocess.run(cmd, check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout + r.stderr


def test_workspace_queries():
    """Workspace sizes need no device: zero where nothing splits (GEMV sizes, M = 0), whole
    planes of M x N fp32 partials otherwise, and for a grouped call the largest need of its
    launches (same-type items share one launch in the tiled GEMM)."""
    L = mx.lib()
    Q4K, Q6K = int(mx.QuantType.Q4_K), int(mx.QuantType.Q6_K)
    assert mx.workspace_size(Q4K, 1024, 4096, 1) == 0
    assert mx.workspace_size(Q4K, 1024, 4096, 0) == 0
    w = mx.workspace_size(Q4K, 1024, 4096, 512)
    assert w > 0 and w % (4 * 512 * 1024) == 0

    def grouped(specs, K, M):
        arr = (qgemm.Item * len(specs))()
        for i, (qt, N) in enumerate(specs):
            arr[i] = qgemm.Item(qt, N, K, 0, None, None, 0, None, 2)
        n = ctypes.c_size_t(7)
        rc = L.mlxr_qgemm_grouped_workspace_size(len(specs), arr, M, ctypes.byref(n))
        return rc, n.value

    assert grouped([(Q4K, 4096), (Q4K, 1024), (Q4K, 1024)], 4096, 1) == (0, 0)
    rc, b = grouped([(Q4K, 4096), (Q4K, 1024), (Q4K, 1024)], 4096, 512)
    assert rc == 0 and b > 0 and b % (4 * 512 * 6144) == 0  # one launch over N = 6144
    # a Q6_K item runs on its own: the need is the larger of the two launches
    rc, b2 = grouped([(Q4K, 4096), (Q4K, 1024), (Q6K, 1024)], 4096, 512)
    single = mx.workspace_size(Q6K, 1024, 4096, 512)
    assert rc == 0 and b2 >= single
    assert grouped([(Q4K, 4096), (Q4K, 1024)], 2048, 512)[0] == 0
    rc, _ = grouped([(Q4K, 4096), (Q4K, 1000)], 4096, 512)
    assert rc == 0
    arr = (qgemm.Item * 2)(qgemm.Item(Q4K, 4096, 4096, 0, None, None, 0, None, 2),
                           qgemm.Item(Q4K, 4096, 2048, 0, None, None, 0, None, 2))
    n = ctypes.c_size_t(0)
    assert L.mlxr_qgemm_grouped_workspace_size(2, arr, 512, ctypes.byref(n)) == -3  # K differs


def test_workspace_sizes_hold_whole_partial_planes():
    """Across types, shapes and M (GEMV sizes, the skinny kernel's, the mid-M range where
    the skinny and tiled kernels compete, prefill): the size is 0 or a whole number of
    M x N fp32 partial planes, with at least two planes (a split); the same query twice
    gives the same answer."""
    qts = [int(q) for q in (mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q8_0, mx.QuantType.Q4_0,
                            mx.QuantType.Q4_1, mx.QuantType.Q5_K)]
    for qt in qts:
        for N, K in [(1024, 4096), (4096, 4096), (14336, 4096), (4096, 14336), (100, 768), (1000, 2048)]:
            for M in [1, 4, 5, 8, 16, 32, 33, 64, 65, 100, 128, 200, 256, 257, 512, 2048]:
                w = mx.workspace_size(qt, N, K, M)
                assert w == mx.workspace_size(qt, N, K, M)
                if M <= 4 and mx.auto_path(qt, N, K, M) == mx.PATH_GEMV:
                    assert w == 0, (qt, N, K, M, w)
                assert w % (4 * M * N) == 0, (qt, N, K, M, w)
                assert w == 0 or w // (4 * M * N) >= 2, (qt, N, K, M, w)


def test_auto_path_rule():
    """The automatic path's kernel family: the GEMV at M = 1 and for short rows at M <= 4;
    the skinny MFMA kernel for long rows at M = 3, 4 (K >= 8192) and M = 2 (K >= 16384) and
    for large weights at M = 4 (not Q6_K); MFMA above M = 4.  A call the MFMA kernels take
    at M <= 4 gets a workspace size when its slabs are few (down shapes)."""
    Q4K, Q6K = int(mx.QuantType.Q4_K), int(mx.QuantType.Q6_K)
    G, F = mx.PATH_GEMV, mx.PATH_MFMA
    cases = [(Q4K, 14336, 4096, 1, G), (Q4K, 4096, 14336, 1, G), (Q4K, 8192, 28672, 1, G),
             (Q4K, 4096, 14336, 2, G), (Q4K, 8192, 28672, 2, F), (Q4K, 4096, 4096, 3, G),
             (Q4K, 4096, 14336, 3, F), (Q4K, 14336, 4096, 3, G), (Q4K, 14336, 4096, 4, F),
             (Q4K, 4096, 4096, 4, G), (Q6K, 128256, 4096, 4, G), (Q6K, 4096, 14336, 4, F),
             (Q4K, 100, 256, 5, F), (Q4K, 100, 256, 0, G)]
    for qt, N, K, M, want in cases:
        assert mx.auto_path(qt, N, K, M) == want, (qt, N, K, M)
    assert mx.workspace_size(Q4K, 4096, 14336, 3) > 0
    assert mx.workspace_size(Q4K, 4096, 14336, 2) == 0

