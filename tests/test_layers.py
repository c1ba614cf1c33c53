"""Linear / MLP layers (mlxr_amd/layers.py, include/mlxr_linear.h): the caller side of
q_gemm_dequant, checked stage by stage against the oracle."""
import os
import subprocess

import numpy as np
import pytest

import mlxr_amd as mx
from mlxr_amd import qgemm
from oracle import orc
from tests import gguf_writer as gw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL = 5e-3
Q4K, Q6K = mx.QuantType.Q4_K, mx.QuantType.Q6_K


def test_linear_argument_checks():
    with pytest.raises(mx.QGemmError):
        mx.Linear(0, 4)
    lin = mx.Linear(256, 8)
    with pytest.raises(mx.QGemmError, match="not loaded"):
        lin.forward(np.zeros((1, 256)))
    with pytest.raises(mx.QGemmError, match="without bias"):
        lin.set_bias(None)


def _act(torch, shape, seed, cuda):
    n = int(np.prod(shape))
    bits = mx.synth_act(n, mx.BF16, seed)
    t = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16).reshape(shape)
    return t, orc.bf16_bits_to_f32(bits).reshape(-1, shape[-1])


@pytest.mark.gpu
@pytest.mark.parametrize("qt,shape", [(Q4K, (1, 1, 1024)), (Q4K, (2, 3, 1024)), (Q6K, (4, 75, 512)),
                                      (Q4K, (300, 512))])
def test_linear_forward_matches_oracle(cuda, qt, shape):
    import torch
    K, N = shape[-1], 384
    w = mx.synth_gguf(qt, N, K, 7)
    lin = mx.Linear(K, N, bias=True).load_weight(w, qt, device=cuda)
    lin.set_bias(torch.linspace(-1, 1, N, device=cuda, dtype=torch.float32))
    x, xf = _act(torch, shape, 11, cuda)
    y = lin(x)
    assert tuple(y.shape) == tuple(shape[:-1]) + (N,) and y.dtype == torch.bfloat16
    M = xf.shape[0]
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=np.linspace(-1, 1, N).astype(np.float32), w_to_bf16=M > 4)
    assert orc.rel_err(y.float().reshape(M, N).cpu().numpy(), ref) <= TOL


def _swiglu64(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_swiglu_kernel(cuda, dt):
    import torch
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]
    rng = np.random.default_rng(3)
    n = 4099  # a tail that is not a multiple of four
    g = rng.standard_normal(n) * 4
    g[:6] = [-100.0, -30.0, 0.0, -0.0, 30.0, 88.0]
    u = rng.standard_normal(n)
    gt = torch.tensor(g, dtype=tdt, device=cuda)
    ut = torch.tensor(u, dtype=tdt, device=cuda)
    out = mx.swiglu(gt, ut)
    ref = _swiglu64(gt.float().cpu().numpy(), ut.float().cpu().numpy())
    got = out.float().cpu().numpy().astype(np.float64)
    # fp32 math with a fast exp, then one rounding to the output type
    # (plus half the smallest subnormal step of the output type, for results that underflow)
    rel = {"f32": 2e-6, "f16": 2 ** -10, "bf16": 2 ** -7}[dt]
    atol = {"f32": 2.0 ** -126, "f16": 2.0 ** -25, "bf16": 2.0 ** -126}[dt]  # fp32 subnormals may flush
    assert np.all(np.abs(got - ref) <= rel * np.abs(ref) + atol), np.max(np.abs(got - ref) / (np.abs(ref) + 1e-30))
    assert np.all(np.isfinite(got))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 40, 300])
def test_mlp_forward_stagewise(cuda, M):
    import torch
    H, I = 512, 1024
    ws = {n: mx.synth_gguf(Q4K, N, K, s) for n, N, K, s in (("g", I, H, 21), ("u", I, H, 22), ("d", H, I, 23))}
    mlp = mx.MLP(H, I)
    mlp.gate_proj.load_weight(ws["g"], Q4K, device=cuda)
    mlp.up_proj.load_weight(ws["u"], Q4K, device=cuda)
    mlp.down_proj.load_weight(ws["d"], Q4K, device=cuda)
    x, xf = _act(torch, (M, H), 31, cuda)
    y = mlp(x)
    # stage by stage: gate/up against the oracle; the fused gate/up/gating launch the layer
    # runs against fp64 gating of the oracle's gate/up; down against the oracle on the GPU's
    # own h; the layer is exactly that chain
    wb = M > 4
    gu = {}
    for name in ("g", "u"):
        t = (mlp.gate_proj if name == "g" else mlp.up_proj)(x)
        gu[name] = orc.gemm_f64(int(Q4K), M, I, H, ws[name], xf, w_to_bf16=wb)
        assert orc.rel_err(t.float().cpu().numpy(), gu[name]) <= TOL
    h = mx.q_gemm_swiglu(x, mlp.gate_proj.weight, mlp.up_proj.weight)
    assert orc.rel_err(h.float().cpu().numpy(), _swiglu64(gu["g"], gu["u"])) <= TOL
    hf = h.float().cpu().numpy()
    ref = orc.gemm_f64(int(Q4K), M, H, I, ws["d"], hf, w_to_bf16=wb)
    assert orc.rel_err(y.float().cpu().numpy(), ref) <= TOL
    assert torch.equal(y, mlp.down_proj(h))


@pytest.mark.gpu
def test_cpp_layers(cuda, tmp_path):
    """The C++ Linear/MLP classes, compiled against include/ and the library."""
    K, N = 512, 384
    w = gw.Writer(3)
    w.add_tensor("w", [K, N], 12, mx.synth_gguf(Q4K, N, K, 77).tobytes())
    p = tmp_path / "w.gguf"
    p.write_bytes(w.to_bytes()[0])
    exe = tmp_path / "test_linear_gpu"
    libdir = os.path.dirname(qgemm.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "cpp", "test_linear_gpu.cpp"), "-o", str(exe), "-L", libdir,
           "-lmlxr_qgemm", "-Wl,-rpath," + libdir]
    subprocess.run(cmd, check=True, capture_output=True)
    r = subprocess.run([str(exe), str(p), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout + r.stderr
    # the C++ layers' outputs against the oracle (generators as in the program)
    y = orc.bf16_bits_to_f32(np.fromfile(tmp_path / "linear_m3.bin", dtype=np.uint16)).reshape(3, N)
    xb = mx.synth_act(3 * K, mx.BF16, 103)
    bias = orc.bf16_bits_to_f32(mx.synth_act(N, mx.BF16, 5))
    ref = orc.gemm_f64(int(Q4K), 3, N, K, mx.synth_gguf(Q4K, N, K, 77), orc.bf16_bits_to_f32(xb).reshape(3, K),
                       bias=bias)
    assert orc.rel_err(y, ref) <= TOL
    H, I, M = 256, 512, 24
    y = orc.bf16_bits_to_f32(np.fromfile(tmp_path / "mlp_m24.bin", dtype=np.uint16)).reshape(M, H)
    xf = orc.bf16_bits_to_f32(mx.synth_act(M * H, mx.BF16, 50 + M)).reshape(M, H)
    g = orc.gemm_f64(int(Q4K), M, I, H, mx.synth_gguf(Q4K, I, H, 1), xf, w_to_bf16=True)
    u = orc.gemm_f64(int(Q4K), M, I, H, mx.synth_gguf(Q4K, I, H, 2), xf, w_to_bf16=True)
    import torch
    # the layer stores h in bf16 (RNE), which down then reads
    h = torch.from_numpy(_swiglu64(g, u).astype(np.float32)).to(torch.bfloat16).float().numpy()
    ref = orc.gemm_f64(int(Q4K), M, H, I, mx.synth_gguf(Q4K, H, I, 3), h, w_to_bf16=True)
    assert orc.rel_err(y, ref) <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("qt", [mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q8_0, mx.QuantType.Q4_0,
                                mx.QuantType.Q4_1, mx.QuantType.Q5_K])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 16, 30, 48, 130])
def test_q_gemm_swiglu_matches_oracle(cuda, qt, M):
    """h = swish(x Wg^T) * (x Wu^T) against fp64 on the oracle's gate and up: one launch
    computes both projections and the gating at every M (GEMV at M <= 4, the narrow skinny
    kernel to M = 32, the tiled kernel above), with and without a split-K workspace."""
    import torch
    N, K = 768, 1024
    wg, wu = mx.synth_gguf(qt, N, K, 61), mx.synth_gguf(qt, N, K, 62)
    pg = mx.pack_weights(wg, N, K, qt, device=cuda)
    pu = mx.pack_weights(wu, N, K, qt, device=cuda)
    x, xf = _act(torch, (M, K), 63 + M, cuda)
    wb = M > 4  # the MFMA kernels multiply bf16-rounded weights
    g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=wb).astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=wb).astype(np.float64)
    ref = _swiglu64(g, u)
    for odt in (torch.bfloat16, torch.float32):
        for ws in (True, False):
            h = mx.q_gemm_swiglu(x, pg, pu, out_dtype=odt, workspace=ws)
            assert orc.rel_err(h.float().cpu().numpy(), ref) <= TOL, (odt, ws)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N", [(130, 300), (257, 258), (300, 130), (8, 250), (30, 77), (5, 16), (17, 33)])
def test_q_gemm_swiglu_ragged_tiles(cuda, M, N):
    """The fused kernels where the tile edges cut rows and columns: N not a multiple of the
    128-column SwiGLU tile (tiled kernel, M > 32) or of the 16-row slab (narrow skinny
    kernel, M <= 32), N % 4 != 0 (scalar stores), M not a multiple of 32, split and unsplit,
    bf16 and fp32 outputs."""
    import torch
    qt, K = mx.QuantType.Q4_K, 1024
    wg, wu = mx.synth_gguf(qt, N, K, 81), mx.synth_gguf(qt, N, K, 82)
    pg = mx.pack_weights(wg, N, K, qt, device=cuda)
    pu = mx.pack_weights(wu, N, K, qt, device=cuda)
    x, xf = _act(torch, (M, K), 83 + M, cuda)
    g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=True).astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=True).astype(np.float64)
    ref = _swiglu64(g, u)
    for odt in (torch.bfloat16, torch.float32):
        for ws in (True, False):
            h = mx.q_gemm_swiglu(x, pg, pu, out_dtype=odt, workspace=ws)
            assert h.shape == (M, N)
            assert orc.rel_err(h.float().cpu().numpy(), ref) <= TOL, (odt, ws)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [512, 2048])
def test_q_gemm_swiglu_prefill_sizes(cuda, M):
    """The fused tiled kernel at prefill sizes (Llama-3-8B gate/up, K = 4096, N = 14336 cut
    to row slices for the oracle): split and unsplit launches against the oracle on the
    first, middle and last 256 columns of three row ranges."""
    import torch
    N, K = 14336, 4096
    wg, wu = mx.synth_gguf(Q4K, N, K, 71), mx.synth_gguf(Q4K, N, K, 72)
    pg = mx.pack_weights(wg, N, K, Q4K, device=cuda)
    pu = mx.pack_weights(wu, N, K, Q4K, device=cuda)
    x, xf = _act(torch, (M, K), 73 + M, cuda)
    rb = mx.gguf_size(Q4K, 1, K)
    hs = [mx.q_gemm_swiglu(x, pg, pu, workspace=ws).float().cpu().numpy() for ws in (True, False)]
    for n0 in (0, N // 2 - 128, N - 256):
        sl = slice(n0 * rb, (n0 + 256) * rb)
        for m0 in (0, M // 2, M - 32):
            g = orc.gemm_f64(int(Q4K), M, 256, K, wg[sl], xf, w_to_bf16=True, m0=m0, m1=m0 + 32)
            u = orc.gemm_f64(int(Q4K), M, 256, K, wu[sl], xf, w_to_bf16=True, m0=m0, m1=m0 + 32)
            ref = _swiglu64(g, u)
            for h in hs:
                assert orc.rel_err(h[m0:m0 + 32, n0:n0 + 256], ref) <= TOL, (n0, m0)
