"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bars: packed bytes and fp32 dequant bit-exact; bf16 dequant bit-exact to RNE_bf16 of the
oracle; matmul outputs within max|y-ref|/max|ref| <= 5e-3 of the fp64-accumulated oracle
(GEMV over the exact weights, MFMA over the bf16-rounded weights it consumes).
"""
import ctypes

import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc
from tests import packref

pytestmark = pytest.mark.gpu

TOL = 5e-3
Q4K, Q6K, Q80 = mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q8_0
Q40, Q41, Q5K = mx.QuantType.Q4_0, mx.QuantType.Q4_1, mx.QuantType.Q5_K


def _dev_bytes(torch, arr, device):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def _act(torch, M, K, dtype_code, seed, device):
    bits = mx.synth_act(M * K, dtype_code, seed)
    t = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(device)
    t = t.view(torch.bfloat16 if dtype_code == mx.BF16 else torch.float16)
    xf = (orc.bf16_bits_to_f32(bits) if dtype_code == mx.BF16 else orc.f16_bits_to_f32(bits)).reshape(M, K)
    return t, xf


def _packed(torch, qt, N, K, seed, device):
    w = mx.synth_gguf(qt, N, K, seed)
    return w, mx.pack_weights(w, N, K, qt, device=device)


@pytest.mark.parametrize("qt,N,K", [(Q4K, 64, 1024), (Q6K, 48, 768), (Q80, 40, 2048), (Q4K, 3, 256), (Q40, 33, 96),
                                    (Q41, 40, 1024), (Q5K, 24, 1280)])
def test_pack_bytes_match_layout(cuda, qt, N, K):
    import torch
    w = mx.synth_gguf(qt, N, K, 11)
    pw = mx.pack_weights(w, N, K, qt, device=cuda)
    got = pw.buf.cpu().numpy()
    ref_planes = packref.planes(int(qt), N, K, w)
    off = 0
    for p in ref_planes:
        np.testing.assert_array_equal(got[off:off + p.size], p)
        off = (off + p.size + 255) & ~255
    assert off == pw.nbytes


@pytest.mark.parametrize("qt,N,K", [(Q4K, 256, 4096), (Q6K, 128, 8192), (Q80, 256, 2048), (Q4K, 1, 256),
                                    (Q40, 128, 2048), (Q41, 96, 4128), (Q5K, 64, 4096)])
def test_dequant_f32_bit_exact(cuda, qt, N, K):
    import torch
    w, pw = _packed(torch, qt, N, K, 21, cuda)
    got = mx.dequantize(pw, torch.float32).cpu().numpy()
    ref = orc.dequant(int(qt), N, K, w)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qt,N,K", [(Q4K, 256, 4096), (Q6K, 128, 8192), (Q80, 64, 2048), (Q40, 64, 1024),
                                    (Q41, 64, 1056), (Q5K, 32, 2048)])
def test_dequant_bf16_rne_bit_exact(cuda, qt, N, K):
    import torch
    w, pw = _packed(torch, qt, N, K, 22, cuda)
    got = mx.dequantize(pw, torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
    ref = orc.dequant(int(qt), N, K, w)
    refb = torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, refb)


GEMV_CASES = [
    (Q4K, 1, 512, 1024), (Q4K, 1, 1000, 2304), (Q4K, 3, 257, 4096), (Q4K, 8, 128, 512),
    (Q4K, 16, 96, 768), (Q4K, 33, 64, 1024), (Q4K, 64, 80, 512),
    (Q6K, 1, 300, 2048), (Q6K, 5, 128, 1280), (Q6K, 64, 64, 512),
    (Q80, 1, 256, 2048), (Q80, 2, 100, 96), (Q80, 40, 64, 1024),
    (Q40, 1, 300, 2048), (Q40, 3, 64, 96), (Q40, 12, 128, 1024), (Q41, 1, 256, 4096), (Q41, 4, 200, 160),
    (Q41, 64, 64, 512), (Q5K, 1, 300, 4096), (Q5K, 3, 64, 768), (Q5K, 20, 128, 512),
]


@pytest.mark.parametrize("xdt", [mx.BF16, mx.F16])
@pytest.mark.parametrize("qt,M,N,K", GEMV_CASES)
def test_gemv_matches_oracle(cuda, qt, M, N, K, xdt):
    import torch
    w, pw = _packed(torch, qt, N, K, 31 + M, cuda)
    x, xf = _act(torch, M, K, xdt, 41 + N, cuda)
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_GEMV)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf)
    err = orc.rel_err(y.cpu().numpy(), ref)
    assert err <= TOL, err
    # the GEMV accumulates in fp32 (magic-offset dot products, one cancellation per
    # sub-block): far tighter than the contract
    assert orc.normwise_rel_err(y.cpu().numpy(), ref) <= 3e-5


MFMA_CASES = [
    (Q4K, 128, 256, 1024), (Q4K, 130, 200, 512), (Q4K, 1, 128, 256), (Q4K, 256, 384, 2048),
    (Q6K, 128, 128, 1024), (Q6K, 200, 96, 512), (Q80, 128, 160, 1024), (Q80, 77, 64, 96),
    (Q40, 128, 256, 1024), (Q40, 33, 96, 96), (Q40, 8, 512, 2048), (Q41, 160, 128, 1056), (Q41, 64, 300, 4096),
    (Q41, 5, 64, 160),
    # tile edges with N % 4 != 0 (the epilogue's scalar stores) and ragged M
    (Q4K, 130, 250, 512), (Q6K, 300, 77, 256), (Q80, 200, 130, 1024),
    # one wavefront per workgroup (short K) with two M-blocks: every row must be stored
    (Q4K, 40, 64, 256), (Q6K, 64, 32, 512), (Q80, 33, 64, 64),
    (Q5K, 128, 256, 1024), (Q5K, 9, 96, 768), (Q5K, 300, 200, 2048),
    # the skinny kernel's narrow variant with one and two 16-row activation blocks
    (Q6K, 12, 200, 512), (Q6K, 24, 96, 768), (Q80, 30, 64, 1056), (Q40, 17, 130, 96), (Q5K, 32, 64, 256),
]


def test_gemv_lm_head_q6k_full_size(cuda):
    """The Llama-3-8B output head as Q6_K (N = 128256 rows, K = 4096) at M = 1: every row
    against the fp64 oracle."""
    import torch
    N, K = 128256, 4096
    w, pw = _packed(torch, Q6K, N, K, 91, cuda)
    x, xf = _act(torch, 1, K, mx.BF16, 92, cuda)
    y = mx.q_gemm_dequant(x, pw, 1, N, K, Q6K, out_dtype=torch.float32)
    ref = orc.gemm_f64(int(Q6K), 1, N, K, w, xf)
    assert orc.normwise_rel_err(y.cpu().numpy(), ref) <= 3e-5
    assert orc.elementwise_rel_err(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("qt,M,N,K", MFMA_CASES)
def test_mfma_matches_oracle(cuda, qt, M, N, K):
    import torch
    w, pw = _packed(torch, qt, N, K, 51 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 61 + N, cuda)
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    err = orc.rel_err(y.cpu().numpy(), ref)
    assert err <= TOL, err
    # against the exact (unrounded) weights the bf16 rounding still stays in contract
    ref_exact = orc.gemm_f64(int(qt), M, N, K, w, xf)
    assert orc.normwise_rel_err(y.cpu().numpy(), ref_exact) <= TOL  # normwise only: see rel_err


def test_mfma_f16_activations(cuda):
    import torch
    qt, M, N, K = Q4K, 160, 192, 1024
    w, pw = _packed(torch, qt, N, K, 71, cuda)
    x, xf = _act(torch, M, K, mx.F16, 72, cuda)
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    assert orc.rel_err(y.cpu().numpy(), orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_f16=True)) <= TOL
    assert orc.normwise_rel_err(y.cpu().numpy(), orc.gemm_f64(int(qt), M, N, K, w, xf)) <= TOL  # normwise: fp16-rounded weights


@pytest.mark.parametrize("path", [mx.PATH_GEMV, mx.PATH_MFMA])
@pytest.mark.parametrize("ydt", ["bf16", "f16", "f32"])
def test_bias_and_output_dtypes(cuda, path, ydt):
    import torch
    qt, M, N, K = Q4K, 4 if path == mx.PATH_GEMV else 136, 200, 512
    w, pw = _packed(torch, qt, N, K, 81, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 82, cuda)
    bias_f = np.linspace(-1, 1, N).astype(np.float32)
    bias = torch.from_numpy(bias_f).to(cuda).to(torch.bfloat16)
    bias_ref = bias.float().cpu().numpy()
    odt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[ydt]
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=odt, path=path)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bias_ref, w_to_bf16=(path == mx.PATH_MFMA))
    assert y.dtype == odt
    assert orc.rel_err(y.float().cpu().numpy(), ref) <= TOL


def test_raw_gguf_weights_are_packed_per_call(cuda):
    import torch
    qt, M, N, K = Q6K, 2, 64, 512
    w = mx.synth_gguf(qt, N, K, 91)
    x, xf = _act(torch, M, K, mx.BF16, 92, cuda)
    y = mx.q_gemm_dequant(x, torch.from_numpy(w).to(cuda), M, N, K, qt, out_dtype=torch.float32)
    assert orc.normwise_rel_err(y.cpu().numpy(), orc.gemm_f64(int(qt), M, N, K, w, xf)) <= TOL


def test_gemv_rows_independent_of_batch(cuda):
    """M-tiling invariance.  Within one kernel variant (M <= 4 share the LDS-staged kernel)
    row m of a batched call equals the M=1 call on row m bit for bit; the M=64 call runs the
    register-staged variant, whose reduction order differs, so it must agree to fp32
    rounding."""
    import torch
    qt, N, K = Q4K, 512, 4096
    w, pw = _packed(torch, qt, N, K, 101, cuda)
    x, _ = _act(torch, 64, K, mx.BF16, 102, cuda)
    y3 = mx.q_gemm_dequant(x[:3].contiguous(), pw, 3, N, K, qt, out_dtype=torch.float32, path=mx.PATH_GEMV)
    y64 = mx.q_gemm_dequant(x, pw, 64, N, K, qt, out_dtype=torch.float32, path=mx.PATH_GEMV)
    for m in (0, 1, 2, 17, 63):
        y1 = mx.q_gemm_dequant(x[m:m + 1], pw, 1, N, K, qt, out_dtype=torch.float32, path=mx.PATH_GEMV)
        if m < 3:
            assert torch.equal(y1[0], y3[m])
        assert orc.normwise_rel_err(y1[0].cpu().numpy(), y64[m].cpu().numpy()) <= 1e-6


@pytest.mark.parametrize("qt,M,N,K", [(Q4K, 512, 2048, 1024), (Q4K, 300, 1000, 512), (Q6K, 512, 1536, 768),
                                      (Q80, 512, 1536, 256)])
def test_mfma_large_tile_matches_oracle(cuda, qt, M, N, K):
    """Shapes with enough 256x256 tiles to take the large-tile kernel (ragged M and N too)."""
    import torch
    w, pw = _packed(torch, qt, N, K, 111 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 112 + N, cuda)
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    assert orc.rel_err(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M", [1, 3, 8])
def test_grouped_equals_separate_calls(cuda, M):
    """q/k/v-style projections of one input: the grouped call (one launch per four
    same-type weights at M <= 4, separate launches otherwise) equals separate calls bit for
    bit, including a mixed-type group and a bias."""
    import torch
    K = 1024
    specs = [(Q4K, 512), (Q4K, 128), (Q6K, 128), (Q4K, 640), (Q4K, 256)]
    ws = [mx.pack_weights(mx.synth_gguf(qt, N, K, 200 + i), N, K, qt, device=cuda) for i, (qt, N) in enumerate(specs)]
    x, xf = _act(torch, M, K, mx.BF16, 210, cuda)
    bias = torch.linspace(-1, 1, 128, device=cuda).to(torch.bfloat16)
    biases = [None, bias, None, None, None]
    ys = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=torch.float32)
    for i, (w, y) in enumerate(zip(ws, ys)):
        y1 = mx.q_gemm_dequant(x, w, M, w.N, K, w.qtype, bias=biases[i], out_dtype=torch.float32)
        assert torch.equal(y, y1), i
        ref = orc.gemm_f64(int(w.qtype), M, w.N, K, mx.synth_gguf(w.qtype, w.N, K, 200 + i), xf, w_to_bf16=M > 4,
                           bias=None if biases[i] is None else biases[i].float().cpu().numpy())
        assert orc.rel_err(y.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M,K", [(65, 1024), (130, 4096), (300, 2048), (48, 4096)])
def test_grouped_tiled_launches(cuda, M, K):
    """Grouped calls on the tiled MFMA GEMM: same-type weights share one launch (tile columns
    side by side).  Without a workspace the launch is unsplit and equals separate calls bit
    for bit (M > 64); with the workspace the library asks for, the concatenated N may split
    K (also for 32 < M <= 64) and stays within tolerance of the oracle, deterministically,
    with a bias, a ragged N and a mixed-type group."""
    import torch
    specs = [(Q4K, 512), (Q4K, 130), (Q6K, 128), (Q4K, 640), (Q4K, 256)]
    gg = [mx.synth_gguf(qt, N, K, 300 + i) for i, (qt, N) in enumerate(specs)]
    ws = [mx.pack_weights(g, N, K, qt, device=cuda) for g, (qt, N) in zip(gg, specs)]
    x, xf = _act(torch, M, K, mx.BF16, 310, cuda)
    bias = torch.linspace(-1, 1, 130, device=cuda).to(torch.bfloat16)
    biases = [None, bias, None, None, None]
    if M > 64:
        ys = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=torch.float32, workspace=False)
        for i, (w, y) in enumerate(zip(ws, ys)):
            y1 = torch.empty_like(y)
            L = mx.lib()
            rc = L.mlxr_qgemm_run_ex(int(w.qtype), w.N, K, 0, w.data_ptr(), x.data_ptr(), mx.BF16,
                                     biases[i].data_ptr() if biases[i] is not None else None, mx.BF16,
                                     y1.data_ptr(), mx.F32, M, mx.PATH_AUTO,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == 0, L.mlxr_qgemm_last_error()
            assert torch.equal(y, y1), i
    yw = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=torch.float32)
    yw2 = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=torch.float32)
    for i, (w, y, y2) in enumerate(zip(ws, yw, yw2)):
        assert torch.equal(y, y2), i
        ref = orc.gemm_f64(int(w.qtype), M, w.N, K, gg[i], xf, w_to_bf16=True,
                           bias=None if biases[i] is None else biases[i].float().cpu().numpy())
        assert orc.rel_err(y.cpu().numpy(), ref) <= TOL, i


@pytest.mark.parametrize("ydt", ["bf16", "f32"])
def test_grouped_split_reduce_vectorized(cuda, ydt):
    """Grouped tiled launch split over K whose weights all have N % 4 == 0 (the reduce then
    handles four columns per thread): within tolerance of the oracle with a bias on a middle
    weight, deterministic, for bf16 and f32 outputs."""
    import torch
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[ydt]
    M, K = 130, 4096
    Ns = [512, 132, 1024]
    gg = [mx.synth_gguf(Q4K, N, K, 500 + i) for i, N in enumerate(Ns)]
    ws = [mx.pack_weights(g, N, K, Q4K, device=cuda) for g, N in zip(gg, Ns)]
    x, xf = _act(torch, M, K, mx.BF16, 510, cuda)
    bias = torch.linspace(-1, 1, 132, device=cuda).to(torch.bfloat16)
    biases = [None, bias, None]
    ys = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=tdt)
    ys2 = mx.q_gemm_dequant_grouped(x, ws, biases=biases, out_dtype=tdt)
    for i, (y, y2) in enumerate(zip(ys, ys2)):
        assert torch.equal(y, y2), i
        ref = orc.gemm_f64(int(Q4K), M, Ns[i], K, gg[i], xf, w_to_bf16=True,
                           bias=None if biases[i] is None else biases[i].float().cpu().numpy())
        assert orc.rel_err(y.float().cpu().numpy(), ref) <= TOL, i


def test_grouped_tiled_many_items_f16(cuda):
    """Five same-type weights (more than one launch holds: four, then one), fp16 activations
    and outputs, a K that ends on a half step (Q8_0, K % 64 == 32), with and without the
    workspace."""
    import torch
    M, K = 100, 1056
    Ns = [256, 100, 384, 64, 520]
    gg = [mx.synth_gguf(Q80, N, K, 400 + i) for i, N in enumerate(Ns)]
    ws = [mx.pack_weights(g, N, K, Q80, device=cuda) for g, N in zip(gg, Ns)]
    x, xf = _act(torch, M, K, mx.F16, 410, cuda)
    for use_ws in (False, True):
        ys = mx.q_gemm_dequant_grouped(x, ws, out_dtype=torch.float16, workspace=use_ws)
        for i, (w, y) in enumerate(zip(ws, ys)):
            ref = orc.gemm_f64(int(Q80), M, w.N, K, gg[i], xf, w_to_f16=True)
            assert orc.rel_err(y.float().cpu().numpy(), ref) <= TOL, (use_ws, i)
            if not use_ws:
                y1 = mx.q_gemm_dequant(x, w, M, w.N, K, Q80, out_dtype=torch.float16)
                if mx.workspace_size(Q80, w.N, K, M) == 0:  # the separate call is unsplit too
                    assert torch.equal(y, y1), i


@pytest.mark.parametrize("qt,M,N,K", [(Q4K, 300, 512, 4096), (Q6K, 256, 256, 2048), (Q80, 130, 384, 1056),
                                      (Q4K, 64, 1024, 14336)])
def test_mfma_few_tiles_long_k(cuda, qt, M, N, K):
    """Few output tiles (the 128-row tile variant) and long K, with bias; two calls in a
    row agree bit for bit."""
    import torch
    w, pw = _packed(torch, qt, N, K, 131 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 132 + N, cuda)
    bias = torch.linspace(-2, 2, N, device=cuda).to(torch.float32)
    y1 = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=torch.float32, path=mx.PATH_MFMA)
    y2 = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=torch.float32, path=mx.PATH_MFMA)
    assert torch.equal(y1, y2)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bias.cpu().numpy(), w_to_bf16=True)
    assert orc.rel_err(y1.cpu().numpy(), ref) <= TOL


def test_mfma_chunked_launches(cuda):
    """Operands past the 32-bit offset range run as several launches over M and N chunks;
    a lowered chunk limit makes small shapes take that path (three M chunks, three N
    chunks), which must stay within tolerance like the single launch."""
    import torch
    qt, M, N, K = Q4K, 600, 700, 1024
    w, pw = _packed(torch, qt, N, K, 141, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 142, cuda)
    y1 = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    mx.qgemm.test_set_operand_limit(1 << 17)  # 256-row and 256-column chunks
    try:
        y2 = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    finally:
        mx.qgemm.test_set_operand_limit(0)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    assert orc.rel_err(y2.cpu().numpy(), ref) <= TOL
    assert orc.rel_err(y1.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M", [8, 40])
def test_skinny_operand_limit_falls_back_to_chunked_tiles(cuda, M):
    """The skinny kernels address every operand with 32-bit offsets: when a weight plane
    reaches the limit (lowered here so that a small shape does) the call runs on the tiled
    kernel's chunked launches instead, and stays within tolerance; grouped calls and the
    fused SwiGLU fall back the same way."""
    import torch
    qt, N, K = Q4K, 700, 1024
    w, pw = _packed(torch, qt, N, K, 151 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 152 + M, cuda)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    y1 = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    mx.qgemm.test_set_operand_limit(1 << 17)  # below the 358 KB qs plane
    try:
        y2 = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
        ys = mx.q_gemm_dequant_grouped(x, [pw, pw], out_dtype=torch.float32)
        wu = mx.synth_gguf(qt, N, K, 161 + M)
        pu = mx.pack_weights(wu, N, K, qt, device=cuda)
        h = mx.q_gemm_swiglu(x, pw, pu, out_dtype=torch.float32)
    finally:
        mx.qgemm.test_set_operand_limit(0)
    for y in (y1, y2, ys[0], ys[1]):
        assert orc.rel_err(y.cpu().numpy(), ref) <= TOL
    g = ref.astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=True).astype(np.float64)
    assert orc.rel_err(h.cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= TOL


# The skinny kernel's narrow (16x16x32) variant on Q4_K: ragged N, K shorter than or not a
# multiple of its ring (steps of 128), both activation dtypes, M from 1 to 16.
@pytest.mark.parametrize("M,N,K,xdt", [(5, 100, 768, mx.BF16), (8, 1000, 2304, mx.F16), (9, 257, 4096, mx.BF16),
                                       (16, 64, 256, mx.F16), (12, 30, 1280, mx.BF16), (1, 33, 512, mx.BF16),
                                       (16, 512, 14336, mx.BF16), (7, 4096, 1024, mx.F16)])
def test_skinny_q4k_matches_oracle(cuda, M, N, K, xdt):
    import torch
    w, pw = _packed(torch, Q4K, N, K, 71 + M, cuda)
    x, xf = _act(torch, M, K, xdt, 81 + N, cuda)
    y = mx.q_gemm_dequant(x, pw, M, N, K, Q4K, out_dtype=torch.float32, path=mx.PATH_MFMA)
    ref = orc.gemm_f64(int(Q4K), M, N, K, w, xf, w_to_bf16=xdt == mx.BF16, w_to_f16=xdt == mx.F16)
    err = orc.rel_err(y.cpu().numpy(), ref)
    assert err <= TOL, err
    if xdt == mx.BF16:  # same bf16 weights as the oracle: only accumulation order differs
        assert err <= 1e-5, err
    y2 = mx.q_gemm_dequant(x, pw, M, N, K, Q4K, out_dtype=torch.float32, path=mx.PATH_MFMA)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("qt,M,N,K,ydt", [(Q4K, 512, 1024, 4096, "bf16"), (Q6K, 256, 1000, 2048, "f32"),
                                          (Q41, 300, 512, 4096, "bf16"), (Q4K, 40, 1024, 4096, "bf16"),
                                          (Q6K, 64, 512, 2048, "f32"), (Q5K, 17, 768, 1024, "f16"),
                                          (Q4K, 8, 1024, 8192, "bf16"), (Q6K, 12, 2048, 4096, "f32"),
                                          (Q80, 5, 512, 2048, "f16"), (Q41, 16, 992, 4096, "bf16"),
                                          (Q80, 130, 384, 1056, "f16"), (Q4K, 2048, 1024, 4096, "f32")])
def test_mfma_split_k(cuda, qt, M, N, K, ydt):
    """Split-K through the C ABI: mlxr_qgemm_run_ws with the workspace size the library
    asks for splits K over workgroups (partials + reduce kernel: the skinny kernel for
    M <= 32 with few 32-row slabs, the tiled kernel otherwise, with 64-row tiles
    for 32 < M <= 64) and stays within tolerance of the oracle,
    with bias, for every output dtype and N % 4 != 0; repeated calls are bit-identical, and
    a workspace one byte too small gives exactly the unsplit mlxr_qgemm_run_ex result."""
    import ctypes
    import torch
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[ydt]
    w, pw = _packed(torch, qt, N, K, 151 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 152 + N, cuda)
    bias = torch.linspace(-1, 1, N, device=cuda).to(torch.bfloat16)
    wsb = mx.workspace_size(qt, N, K, M)
    assert wsb > 0 and wsb % (4 * M * N) == 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=cuda)
    L = mx.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(y, wsp, nbytes):
        rc = L.mlxr_qgemm_run_ws(int(qt), N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, bias.data_ptr(), mx.BF16,
                                 y.data_ptr(), {"bf16": mx.BF16, "f16": mx.F16, "f32": mx.F32}[ydt], M,
                                 mx.PATH_MFMA, wsp, nbytes, s)
        assert rc == 0, L.mlxr_qgemm_last_error()

    ys = [torch.empty((M, N), dtype=tdt, device=cuda) for _ in range(4)]
    run(ys[0], ws.data_ptr(), wsb)
    run(ys[1], ws.data_ptr(), wsb)
    run(ys[2], ws.data_ptr(), wsb - 1)
    rc = L.mlxr_qgemm_run_ex(int(qt), N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, bias.data_ptr(), mx.BF16,
                             ys[3].data_ptr(), {"bf16": mx.BF16, "f16": mx.F16, "f32": mx.F32}[ydt], M,
                             mx.PATH_MFMA, s)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1])
    assert torch.equal(ys[2], ys[3])
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bias.float().cpu().numpy(), w_to_bf16=True)
    for y in (ys[0], ys[3]):
        assert orc.rel_err(y.float().cpu().numpy(), ref) <= TOL


def test_python_binding_checks_outputs_and_bias(cuda):
    """Caller-supplied outputs must be contiguous [M, N] tensors on the input's device (the
    kernels write M*N elements); biases must be [N] on that device."""
    import torch
    qt, M, N, K = Q4K, 3, 64, 256
    w, pw = _packed(torch, qt, N, K, 171, cuda)
    x, _ = _act(torch, M, K, mx.BF16, 172, cuda)
    for bad in (torch.empty((M, N - 1), device=cuda), torch.empty((N, M), device=cuda).t(),
                torch.empty((M, N)), torch.empty((M, N), dtype=torch.int32, device=cuda)):
        with pytest.raises(mx.QGemmError):
            mx.q_gemm_dequant(x, pw, M, N, K, qt, out=bad)
        with pytest.raises(mx.QGemmError):
            mx.q_gemm_dequant_grouped(x, [pw], outs=[bad])
    with pytest.raises(mx.QGemmError):
        mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=torch.zeros(N))  # host bias
    strided = torch.zeros(2 * N, device=cuda)[::2]
    y = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=strided, out_dtype=torch.float32)
    assert torch.equal(y, mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32))


# The 32x32x16 skinny kernel in 64-row blocks of M (second grid dimension), forced at
# shapes the automatic choice may give the tiled kernel: ragged last M block, ragged N,
# every type, K not a multiple of 64 (Q8_0, Q4_0), split K through the workspace.
@pytest.mark.parametrize("qt,M,N,K", [(Q4K, 65, 100, 768), (Q6K, 130, 257, 1024), (Q80, 200, 64, 1056),
                                      (Q40, 96, 33, 96), (Q41, 256, 128, 2048), (Q5K, 129, 96, 512),
                                      (Q4K, 300, 1024, 4096)])
def test_skinny_m_blocks_match_oracle(cuda, qt, M, N, K):
    import torch
    w, pw = _packed(torch, qt, N, K, 171 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 181 + N, cuda)
    bias = torch.linspace(-1, 1, N, device=cuda).to(torch.bfloat16)
    mx.qgemm.test_force_skinny(True)
    try:
        y = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=torch.float32, path=mx.PATH_MFMA)
        y2 = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=torch.float32, path=mx.PATH_MFMA)
    finally:
        mx.qgemm.test_force_skinny(False)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bias.float().cpu().numpy(), w_to_bf16=True)
    err = orc.rel_err(y.cpu().numpy(), ref)
    # same bf16 weights as the oracle: only the fp32 accumulation order differs (K up to
    # 4096 in up to eight split partials)
    assert err <= 3e-5, err


# Shapes whose narrow-kernel plan stages the activations in LDS (M <= 8, eight or more steps
# per wavefront): Llama-3-8B gate, ragged N with a bias and half-precision outputs, K not a
# multiple of the 128-wide step (Q4_0, Q8_0), M <= 4 through the MFMA path, down shapes (K
# split over two workgroups, seven wavefronts of 112 KiB of stages), long stages at M = 1
# and 2 (32 and 16 steps per wavefront), M = 9 to 16 (two slabs per workgroup sharing their
# stages; 14300 rows: an odd slab count, the last workgroup's second slab past N).
@pytest.mark.parametrize("qt,M,N,K,path,ydt", [(Q4K, 8, 14336, 4096, mx.PATH_AUTO, "f32"),
                                               (Q6K, 6, 14000, 4096, mx.PATH_AUTO, "bf16"),
                                               (Q80, 5, 11008, 4000, mx.PATH_AUTO, "f16"),
                                               (Q40, 7, 13000, 4064, mx.PATH_AUTO, "f32"),
                                               (Q5K, 1, 14336, 4096, mx.PATH_MFMA, "f32"),
                                               (Q41, 3, 11000, 4096, mx.PATH_MFMA, "bf16"),
                                               (Q80, 8, 4096, 14336, mx.PATH_AUTO, "f32"),
                                               (Q6K, 7, 4000, 14336, mx.PATH_AUTO, "bf16"),
                                               (Q4K, 1, 9000, 32768, mx.PATH_MFMA, "f32"),
                                               (Q40, 2, 9000, 16384, mx.PATH_MFMA, "f32"),
                                               (Q4K, 16, 14336, 4096, mx.PATH_AUTO, "bf16"),
                                               (Q80, 12, 14000, 4000, mx.PATH_AUTO, "f32"),
                                               (Q6K, 9, 4096, 14336, mx.PATH_AUTO, "f16"),
                                               (Q41, 13, 11001, 4096, mx.PATH_AUTO, "f32"),
                                               (Q4K, 12, 14300, 4096, mx.PATH_AUTO, "bf16")])
def test_skinny_staged_activations_match_oracle(cuda, qt, M, N, K, path, ydt):
    """The narrow skinny kernel with its activations staged in LDS (one slab per workgroup
    where that fits, two slabs sharing their stages otherwise or when preferred through the
    test hook) gives the same bits as the kernel reading them from global memory (same
    products in the same order), and all agree with the oracle over the bf16-rounded
    weights."""
    import torch
    w, pw = _packed(torch, qt, N, K, 211 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 221 + M, cuda)
    bias = torch.linspace(-1, 1, N, device=cuda).to(torch.bfloat16)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[ydt]
    ys = {}
    try:
        for mode in (1, 2, 0):
            mx.qgemm.test_skinny_stage(mode)
            ys[mode] = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=tdt, path=path)
    finally:
        mx.qgemm.test_skinny_stage(1)
    torch.cuda.synchronize()
    assert torch.equal(ys[1], ys[0])
    assert torch.equal(ys[2], ys[0])
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bias.float().cpu().numpy(), w_to_bf16=True)
    # half-precision outputs add their own rounding (2^-9 / 2^-12 relative)
    assert orc.rel_err(ys[1].float().cpu().numpy(), ref) <= (5e-3 if ydt != "f32" else 3e-5)


@pytest.mark.parametrize("qt,M", [(Q4K, 8), (Q80, 5), (Q6K, 3)])
def test_skinny_staged_f16_activations_match_oracle(cuda, qt, M):
    """fp16 activations (the fp16 MFMA, fp16-rounded weights) through the staged narrow
    kernel on the Llama-3-8B gate shape: same bits as the global-read mode, within 3e-5 of
    the oracle over the fp16-rounded weights."""
    import torch
    N, K = 14336, 4096
    w, pw = _packed(torch, qt, N, K, 281 + M, cuda)
    x, xf = _act(torch, M, K, mx.F16, 291 + M, cuda)
    ys = {}
    try:
        for on in (True, False):
            mx.qgemm.test_skinny_stage(on)
            ys[on] = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    finally:
        mx.qgemm.test_skinny_stage(True)
    torch.cuda.synchronize()
    assert torch.equal(ys[True], ys[False])
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_f16=True)
    assert orc.rel_err(ys[True].cpu().numpy(), ref) <= 3e-5


@pytest.mark.parametrize("M", [6, 8, 16])
def test_skinny_staged_swiglu_matches_oracle(cuda, M):
    """Fused SwiGLU through the staged narrow kernel (16-row slabs of gate and up, 512 of
    them: N = 8192 at K = 4096): same bits as the global-read mode, and the oracle's
    swish(g) * u within 5e-3."""
    import torch
    qt, N, K = Q4K, 8192, 4096
    wg, pg = _packed(torch, qt, N, K, 231, cuda)
    wu, pu = _packed(torch, qt, N, K, 232, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 233 + M, cuda)
    hs = {}
    try:
        for mode in (1, 2, 0):
            mx.qgemm.test_skinny_stage(mode)
            hs[mode] = mx.q_gemm_swiglu(x, pg, pu, out_dtype=torch.float32)
    finally:
        mx.qgemm.test_skinny_stage(1)
    torch.cuda.synchronize()
    assert torch.equal(hs[1], hs[0])
    assert torch.equal(hs[2], hs[0])
    g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=True).astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=True).astype(np.float64)
    assert orc.rel_err(hs[1].cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= 5e-3


@pytest.mark.parametrize("qt,M,N,K", [(Q4K, 3, 4096, 14336), (Q6K, 4, 2000, 8192), (Q4K, 2, 1500, 16384),
                                      (Q80, 4, 14336, 4096)])
def test_auto_path_takes_mfma_for_long_rows_at_small_m(cuda, qt, M, N, K):
    """At M <= 4 the automatic path runs long rows (and, at M = 4, large weights) on the skinny
    MFMA kernel: the same bits as the forced MFMA path with the workspace the library asks
    for, within the contract of the oracle over the bf16-rounded weights."""
    import torch
    assert mx.auto_path(qt, N, K, M) == mx.PATH_MFMA
    w, pw = _packed(torch, qt, N, K, 301 + M, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 311 + M, cuda)
    y_auto = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32)
    y_mfma = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32, path=mx.PATH_MFMA)
    torch.cuda.synchronize()
    assert torch.equal(y_auto, y_mfma)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    assert orc.rel_err(y_auto.cpu().numpy(), ref) <= 3e-5


@pytest.mark.parametrize("qt,M,N,K", [(Q4K, 3, 600, 8192), (Q80, 4, 14336, 4096), (Q4K, 2, 300, 16384)])
def test_swiglu_at_small_m_follows_auto_path(cuda, qt, M, N, K):
    """The fused SwiGLU at M <= 4 takes the kernel family the automatic path gives its gate
    shape: here the narrow skinny kernel (long rows, or a large weight at M = 4), so h is
    swish(g) * u over the bf16-rounded weights of the oracle, within 5e-3."""
    import torch
    assert mx.auto_path(qt, N, K, M) == mx.PATH_MFMA
    wg, pg = _packed(torch, qt, N, K, 321, cuda)
    wu, pu = _packed(torch, qt, N, K, 322, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 323 + M, cuda)
    h = mx.q_gemm_swiglu(x, pg, pu, out_dtype=torch.float32)
    torch.cuda.synchronize()
    g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=True).astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=True).astype(np.float64)
    assert orc.rel_err(h.cpu().numpy(), g / (1.0 + np.exp(-g)) * u) <= TOL


@pytest.mark.parametrize("M", [3, 4])
def test_grouped_call_at_small_m_with_large_weights(cuda, M):
    """A grouped call at M <= 4 keeps small weights in one GEMV launch (even with rows the
    automatic path of a single call would give the skinny kernel) and gives very large ones
    with long rows (here 8192 x 16384) the skinny kernel: the large output equals its single
    automatic call, the small one its single GEMV call, bit for bit, and both are within 3e-5
    of the oracle over the operands they multiply."""
    import torch
    K = 16384
    specs = [(Q4K, 8192, 16384), (Q4K, 512, 16384)]
    gg = [mx.synth_gguf(qt, N, K, 331 + i) for i, (qt, N, _) in enumerate(specs)]
    pws = [mx.pack_weights(g, N, K, qt, device=cuda) for g, (qt, N, _) in zip(gg, specs)]
    assert mx.auto_path(Q4K, 8192, K, M) == mx.PATH_MFMA
    x, xf = _act(torch, M, K, mx.BF16, 341 + M, cuda)
    ys = mx.q_gemm_dequant_grouped(x, pws, out_dtype=torch.float32)
    singles = [mx.q_gemm_dequant(x, pws[0], M, 8192, K, Q4K, out_dtype=torch.float32),
               mx.q_gemm_dequant(x, pws[1], M, 512, K, Q4K, out_dtype=torch.float32, path=mx.PATH_GEMV)]
    torch.cuda.synchronize()
    for i, (y, y1) in enumerate(zip(ys, singles)):
        assert torch.equal(y, y1), i
    big = orc.gemm_f64(int(Q4K), M, 8192, K, gg[0], xf, w_to_bf16=True)
    small = orc.gemm_f64(int(Q4K), M, 512, K, gg[1], xf)
    assert orc.rel_err(ys[0].cpu().numpy(), big) <= 3e-5
    assert orc.rel_err(ys[1].cpu().numpy(), small) <= 3e-5


@pytest.mark.parametrize("qt,N,K", [(Q4K, 1024, 4096), (Q6K, 4096, 4096)])
def test_narrow_weights_at_mid_m_take_skinny_kernel(cuda, qt, N, K):
    """Shapes at M = 128 whose estimated times favour the skinny kernel: Llama-3-8B k (the
    skinny kernel splits K, so it asks for a workspace) and a Q6_K 4096x4096 weight (256
    blocks fill the device: workspace size 0).  With the workspace the library asks for the
    call is bit-equal to the forced skinny call; mlxr_qgemm_run_ex without a workspace makes
    the same choice when the size is 0 and otherwise runs the tiled kernel unsplit; all
    within tolerance of the oracle."""
    import torch
    M = 128
    w, pw = _packed(torch, qt, N, K, 191, cuda)
    x, xf = _act(torch, M, K, mx.BF16, 192, cuda)
    need = mx.workspace_size(qt, N, K, M)
    y_auto = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32)
    mx.qgemm.test_force_skinny(True)
    try:
        y_sk = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32)
    finally:
        mx.qgemm.test_force_skinny(False)
    y_ex = torch.empty((M, N), dtype=torch.float32, device=cuda)
    rc = mx.lib().mlxr_qgemm_run_ex(int(qt), N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, None, mx.F32,
                                    y_ex.data_ptr(), mx.F32, M, mx.PATH_AUTO, None)
    assert rc == 0, mx.lib().mlxr_qgemm_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y_auto, y_sk)
    if need == 0:
        assert torch.equal(y_ex, y_sk)
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, w_to_bf16=True)
    for y in (y_auto, y_ex):
        assert orc.rel_err(y.cpu().numpy(), ref) <= 3e-5


def test_concurrent_calls_from_host_threads(cuda):
    """Four host threads, each with its own stream and workspace, issue calls of every kernel
    family (GEMV, staged and unstaged skinny, tiled split-K) at once; every output equals the
    same call made alone, bit for bit (the library's per-device caches and per-thread error
    strings are shared state)."""
    import threading
    import torch
    shapes = [(Q4K, 1, 4096, 4096), (Q4K, 8, 14336, 4096), (Q80, 16, 4096, 4096), (Q6K, 64, 1024, 4096),
              (Q4K, 300, 2048, 2048)]
    pws = {}
    for i, (qt, M, N, K) in enumerate(shapes):
        pws[i] = mx.pack_weights(mx.synth_gguf(qt, N, K, 351 + i), N, K, qt, device=cuda)
    xs = {i: _act(torch, M, K, mx.BF16, 361 + i, cuda)[0] for i, (qt, M, N, K) in enumerate(shapes)}
    L = mx.lib()

    def call(i, stream, ws, y):
        qt, M, N, K = shapes[i]
        need = mx.workspace_size(qt, N, K, M)
        rc = L.mlxr_qgemm_run_ws(int(qt), N, K, 0, pws[i].data_ptr(), xs[i].data_ptr(), mx.BF16, None, mx.BF16,
                                 y.data_ptr(), mx.F32, M, mx.PATH_AUTO, ws.data_ptr() if need else None, need,
                                 ctypes.c_void_p(stream.cuda_stream))
        return rc

    cap = max(mx.workspace_size(qt, N, K, M) for qt, M, N, K in shapes) + 1
    ref = {}
    s0 = torch.cuda.Stream()
    w0 = torch.empty(cap, dtype=torch.uint8, device=cuda)
    for i, (qt, M, N, K) in enumerate(shapes):
        ref[i] = torch.empty((M, N), dtype=torch.float32, device=cuda)
        assert call(i, s0, w0, ref[i]) == 0
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        torch.cuda.set_device(cuda)
        st = torch.cuda.Stream()
        ws = torch.empty(cap, dtype=torch.uint8, device=cuda)
        outs = []
        for rep in range(20):
            i = (t + rep) % len(shapes)
            qt, M, N, K = shapes[i]
            y = torch.empty((M, N), dtype=torch.float32, device=cuda)
            if call(i, st, ws, y) != 0:
                errors.append((t, rep, L.mlxr_qgemm_last_error()))
            outs.append((i, y))
            st.synchronize()  # the workspace is reused by the next call on this thread
        for i, y in outs:
            if not torch.equal(y, ref[i]):
                errors.append((t, i, "mismatch"))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
