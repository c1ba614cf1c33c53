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
    assert orc.normwise_rel_err(y.float().reshape(M, N).cpu().numpy(), ref) <= TOL


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
    # stage by stage: gate/up against the oracle, the gating against fp64 on the GPU's own
    # gate/up, down against the oracle on the GPU's own h
    g = mlp.gate_proj(x)
    u = mlp.up_proj(x)
    wb = M > 4
    for t, name in ((g, "g"), (u, "u")):
        ref = orc.gemm_f64(int(Q4K), M, I, H, ws[name], xf, w_to_bf16=wb)
        assert orc.normwise_rel_err(t.float().cpu().numpy(), ref) <= TOL
    h = mx.swiglu(g, u)
    href = _swiglu64(g.float().cpu().numpy(), u.float().cpu().numpy())
    assert np.max(np.abs(h.float().cpu().numpy() - href)) <= 2 ** -7 * np.max(np.abs(href))
    hf = h.float().cpu().numpy()
    ref = orc.gemm_f64(int(Q4K), M, H, I, ws["d"], hf, w_to_bf16=wb)
    assert orc.normwise_rel_err(y.float().cpu().numpy(), ref) <= TOL
    if M > 4:
        # the layer is exactly that chain
        assert torch.equal(y, mlp.down_proj(h))
    else:
        # one fused launch: the gating sees fp32 gate/up (no bf16 round trip in between)
        hf = mx.q_gemm_swiglu(x, mlp.gate_proj.weight, mlp.up_proj.weight)
        assert torch.equal(y, mlp.down_proj(hf))


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
    r = subprocess.run([str(exe), str(p)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("qt", [mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q8_0, mx.QuantType.Q4_0,
                                mx.QuantType.Q4_1, mx.QuantType.Q5_K])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 130])
def test_q_gemm_swiglu_matches_oracle(cuda, qt, M):
    """h = swish(x Wg^T) * (x Wu^T) against fp64 on the oracle's gate and up; one launch for
    M <= 4, projections + gating (workspace) above."""
    import torch
    N, K = 768, 1024
    wg, wu = mx.synth_gguf(qt, N, K, 61), mx.synth_gguf(qt, N, K, 62)
    pg = mx.pack_weights(wg, N, K, qt, device=cuda)
    pu = mx.pack_weights(wu, N, K, qt, device=cuda)
    x, xf = _act(torch, (M, K), 63 + M, cuda)
    for odt in (torch.bfloat16, torch.float32):
        h = mx.q_gemm_swiglu(x, pg, pu, out_dtype=odt)
        wb = M > 4
        g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=wb).astype(np.float64)
        u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=wb).astype(np.float64)
        if M > 4:  # the unfused path rounds gate and up to the output type first
            rnd = (lambda a: torch.tensor(a).to(odt).double().numpy())
            g, u = rnd(g), rnd(u)
        ref = _swiglu64(g, u)
        assert orc.normwise_rel_err(h.float().cpu().numpy(), ref) <= TOL
