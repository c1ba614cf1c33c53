"""The BASELINE configurations at their full sizes on the GPU, against the fp64 oracle: every
output at decode sizes where the oracle is quick, row slices of the weights (and, at prefill
sizes, the first and last rows of X) elsewhere.  The generators are the bench's."""
import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc

pytestmark = pytest.mark.gpu

TOL = 5e-3
Q4K, Q6K, Q80 = mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q8_0
LLAMA3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
LLAMA3_70B = [("q", 8192, 8192, Q4K), ("k", 1024, 8192, Q4K), ("v", 1024, 8192, Q6K), ("o", 8192, 8192, Q4K),
              ("gate", 28672, 8192, Q4K), ("up", 28672, 8192, Q4K), ("down", 8192, 28672, Q6K)]


def _act(torch, M, K, dt, seed, device):
    bits = mx.synth_act(M * K, dt, seed)
    t = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(device)
    t = t.view(torch.bfloat16 if dt == mx.BF16 else torch.float16)
    xf = (orc.bf16_bits_to_f32(bits) if dt == mx.BF16 else orc.f16_bits_to_f32(bits)).reshape(M, K)
    return t, xf


def _rows(qt, w, K, n0, n1):
    """GGUF bytes of weight rows [n0, n1) (blocks are row-major)."""
    rb = mx.gguf_size(qt, 1, K)
    return w[n0 * rb:n1 * rb]


def _check(qt, y, w, xf, N, K, slices, mrows=None, bf16_weights=False, tol=TOL):
    """y [M, N] (torch, device) against the oracle on weight row slices and X row ranges: the
    normwise error within tol, the elementwise one within the 5e-3 contract.  With
    bf16_weights (the MFMA paths, which multiply RNE-bf16 weights) the reference rounds the
    weights as the kernel does, and the output must also stay within the 5e-3 contract
    normwise of the reference over the exact GGUF weights."""
    yh = y.float().cpu().numpy()
    M = yh.shape[0]
    for n0, n1 in slices:
        for m0, m1 in (mrows or [(0, M)]):
            ref = orc.gemm_f64(int(qt), M, n1 - n0, K, _rows(qt, w, K, n0, n1), xf, w_to_bf16=bf16_weights,
                               m0=m0, m1=m1)
            err = orc.normwise_rel_err(yh[m0:m1, n0:n1], ref)
            assert err <= tol, (n0, n1, m0, m1, err)
            # elementwise over the outputs with |ref| >= 1e-2 * max |ref|
            err = orc.elementwise_rel_err(yh[m0:m1, n0:n1], ref)
            assert err <= TOL, (n0, n1, m0, m1, "elementwise", err)
            if bf16_weights:
                exact = orc.gemm_f64(int(qt), M, n1 - n0, K, _rows(qt, w, K, n0, n1), xf, m0=m0, m1=m1)
                err = orc.normwise_rel_err(yh[m0:m1, n0:n1], exact)
                assert err <= TOL, (n0, n1, m0, m1, "exact weights", err)


def test_c1_q8_0_tinyllama_m1(cuda):
    import torch
    N = K = 2048
    w = mx.synth_gguf(Q80, N, K, 0x4D4C5852)
    pw = mx.pack_weights(w, N, K, Q80, device=cuda)
    x, xf = _act(torch, 1, K, mx.F16, 0x4D4C5852 + 2001, cuda)
    y = mx.q_gemm_dequant(x, pw, 1, N, K, Q80, out_dtype=torch.float32)
    _check(Q80, y, w, xf, N, K, [(0, N)], tol=3e-5)
    y16 = mx.q_gemm_dequant(x, pw, 1, N, K, Q80)  # fp16 out, as the config
    assert y16.dtype == torch.float16
    assert torch.equal(y16, y.to(torch.float16))


def test_c2_llama3_8b_layer_m1(cuda):
    """The headline step's launches (grouped q/k/v, o, grouped gate/up, down): every output."""
    import torch
    gg = {n: mx.synth_gguf(Q4K, N, K, 0x4D4C5853 + 16 * i) for i, (n, N, K) in enumerate(LLAMA3_8B)}
    pw = {n: mx.pack_weights(gg[n], N, K, Q4K, device=cuda) for n, N, K in LLAMA3_8B}
    dims = {n: (N, K) for n, N, K in LLAMA3_8B}
    xs = {K: _act(torch, 1, K, mx.BF16, 1001 + K, cuda) for K in (4096, 14336)}
    for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
        K = dims[names[0]][1]
        ys = mx.q_gemm_dequant_grouped(xs[K][0], [pw[n] for n in names], out_dtype=torch.float32)
        for n, y in zip(names, ys):
            _check(Q4K, y, gg[n], xs[K][1], dims[n][0], K, [(0, dims[n][0])], tol=3e-5)


@pytest.mark.parametrize("M", [8, 16, 32, 64])
def test_c3_batched_decode(cuda, M):
    import torch
    for i, (n, N, K) in enumerate([("gate", 14336, 4096), ("down", 4096, 14336)]):
        w = mx.synth_gguf(Q4K, N, K, 0x4D4C5854 + i)
        pw = mx.pack_weights(w, N, K, Q4K, device=cuda)
        x, xf = _act(torch, M, K, mx.BF16, 3000 + M + i, cuda)
        y = mx.q_gemm_dequant(x, pw, M, N, K, Q4K, out_dtype=torch.float32)
        _check(Q4K, y, w, xf, N, K, [(0, 512), (N // 2 - 256, N // 2 + 256), (N - 512, N)], bf16_weights=True)


@pytest.mark.parametrize("M", [512, 2048])
def test_c4_prefill(cuda, M):
    import torch
    mrows = [(0, 32), (M // 2, M // 2 + 32), (M - 32, M)]
    xs = {K: _act(torch, M, K, mx.BF16, 4000 + M + K, cuda) for K in (4096, 14336)}
    for i, (n, N, K) in enumerate(LLAMA3_8B):
        w = mx.synth_gguf(Q4K, N, K, 0x4D4C5855 + 16 * i)
        pw = mx.pack_weights(w, N, K, Q4K, device=cuda)
        y = mx.q_gemm_dequant(xs[K][0], pw, M, N, K, Q4K, out_dtype=torch.float32)
        _check(Q4K, y, w, xs[K][1], N, K, [(0, 256), (N - 256, N)], mrows=mrows, bf16_weights=True)


@pytest.mark.parametrize("M", [1, 256])
def test_c5_llama3_70b_layer(cuda, M):
    """q,k,v,o,gate,up,down of a 70B layer (v and down Q6_K) issued as a decoder issues them."""
    import torch
    gg = {n: mx.synth_gguf(qt, N, K, 0x4D4C5856 + 16 * i) for i, (n, N, K, qt) in enumerate(LLAMA3_70B)}
    pw = {n: mx.pack_weights(gg[n], N, K, qt, device=cuda) for n, N, K, qt in LLAMA3_70B}
    spec = {n: (N, K, qt) for n, N, K, qt in LLAMA3_70B}
    xs = {K: _act(torch, M, K, mx.BF16, 5000 + M + K, cuda) for K in (8192, 28672)}
    mrows = None if M == 1 else [(0, 16), (M - 16, M)]
    for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
        K = spec[names[0]][1]
        ys = mx.q_gemm_dequant_grouped(xs[K][0], [pw[n] for n in names], out_dtype=torch.float32)
        for n, y in zip(names, ys):
            N, _, qt = spec[n]
            _check(qt, y, gg[n], xs[K][1], N, K, [(0, 1024), (N - 1024, N)], mrows=mrows, bf16_weights=M > 4,
                   tol=3e-5 if M == 1 else TOL)
