"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the CPU
oracle must reproduce them exactly; the HIP path must match them (GPU tests)."""
import glob
import os

import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc

FILES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _load(f):
    return dict(np.load(f, allow_pickle=False))


def _x(g):
    bits = g["gemm_x_bits"]
    M, N, K = (int(v) for v in g["gemm_shape"])
    xf = orc.bf16_bits_to_f32(bits) if int(g["gemm_x_dtype"]) == mx.BF16 else orc.f16_bits_to_f32(bits)
    return bits, xf.reshape(M, K), M, N, K


def test_fixtures_present():
    assert {os.path.basename(f) for f in FILES} == {"q8_0.npz", "q4_k.npz", "q6_k.npz", "q4_0.npz", "q4_1.npz",
                                                        "q5_k.npz"}


@pytest.mark.parametrize("f", FILES, ids=os.path.basename)
def test_oracle_reproduces_golden(f):
    g = _load(f)
    qt, N, K = int(g["qtype"]), int(g["N"]), int(g["K"])
    np.testing.assert_array_equal(orc.dequant(qt, N, K, g["blocks"]).view(np.uint32), g["dequant"].view(np.uint32))
    _, xf, M, N2, K2 = _x(g)
    np.testing.assert_array_equal(orc.gemm_f64(qt, M, N2, K2, g["gemm_w"], xf), g["gemm_y_f64"])
    np.testing.assert_array_equal(orc.gemm_f64(qt, M, N2, K2, g["gemm_w"], xf, w_to_bf16=True), g["gemm_y_f64_wbf16"])
    np.testing.assert_array_equal(orc.eval_cpu(qt, M, N2, K2, g["gemm_w"], xf), g["gemm_y_eval_cpu"])


@pytest.mark.gpu
@pytest.mark.parametrize("f", FILES, ids=os.path.basename)
def test_hip_matches_golden(f, cuda):
    import torch
    g = _load(f)
    qt, N, K = int(g["qtype"]), int(g["N"]), int(g["K"])
    pw = mx.pack_weights(g["blocks"], N, K, qt, device=cuda)
    got = mx.dequantize(pw, torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), g["dequant"].view(np.uint32))
    bits, _, M, N2, K2 = _x(g)
    xt = torch.from_numpy(bits.view(np.int16).reshape(M, K2)).to(cuda)
    xt = xt.view(torch.bfloat16 if int(g["gemm_x_dtype"]) == mx.BF16 else torch.float16)
    pw2 = mx.pack_weights(g["gemm_w"], N2, K2, qt, device=cuda)
    for path, ref in ((mx.PATH_GEMV, g["gemm_y_f64"]), (mx.PATH_MFMA, g["gemm_y_f64_wbf16"])):
        y = mx.q_gemm_dequant(xt, pw2, M, N2, K2, qt, out_dtype=torch.float32, path=path)
        f16_mfma = path == mx.PATH_MFMA and int(g["gemm_x_dtype"]) == mx.F16
        if f16_mfma:
            # fp16 activations: the MFMA multiplies fp16-rounded weights, not the bf16 ones
            # of the fixture's second output; elementwise against the oracle of those
            xf = (orc.f16_bits_to_f32(bits)).reshape(M, K2)
            wr = orc.gemm_f64(qt, M, N2, K2, g["gemm_w"], xf, w_to_f16=True)
            assert orc.rel_err(y.cpu().numpy(), wr) <= 5e-3
            assert orc.normwise_rel_err(y.cpu().numpy(), ref) <= 5e-3
        else:
            assert orc.rel_err(y.cpu().numpy(), ref) <= 5e-3
