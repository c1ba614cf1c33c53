"""Seeded random calls through the C ABI against the oracle: every quant type, M from 1 to
300 (the GEMV, the skinny kernels with and without 64-row M blocks, the tiled GEMM), ragged
N, K from one block to many, a workspace of the size asked for or none, a bias or none,
bf16 / fp16 / fp32 outputs, and the automatic, GEMV and MFMA paths.  Each call is checked
against the fp64 oracle over the operands its kernel multiplies (exact weights for the GEMV,
RNE-rounded weights for the MFMA kernels) within the 5e-3 contract, and normwise against
the exact weights in every case; a repeated call must give the same bits."""
import ctypes

import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc

pytestmark = pytest.mark.gpu

TOL = 5e-3
TYPES = [mx.QuantType.Q4_K, mx.QuantType.Q6_K, mx.QuantType.Q5_K, mx.QuantType.Q8_0, mx.QuantType.Q4_0,
         mx.QuantType.Q4_1]


def _case(seed):
    rng = np.random.default_rng(seed)
    qt = TYPES[int(rng.integers(len(TYPES)))]
    blk = mx.get_default_group_size(qt)
    K = blk * int(rng.integers(1, 2048 // blk + 1)) if blk == 256 else 32 * int(rng.integers(1, 65))
    M = int(rng.choice([1, 2, 3, 4, 5, 8, 13, 16, 17, 31, 32, 33, 47, 64, 65, 96, 128, 130, 200, 256, 257, 300]))
    N = int(rng.integers(1, 700))
    path = int(rng.choice([mx.PATH_AUTO, mx.PATH_AUTO, mx.PATH_MFMA] + ([mx.PATH_GEMV] if M <= 64 else [])))
    ydt = str(rng.choice(["bf16", "f16", "f32"]))
    xdt = mx.BF16 if ydt != "f16" else int(rng.choice([mx.BF16, mx.F16]))
    use_ws = bool(rng.integers(2))
    use_bias = bool(rng.integers(2))
    return qt, M, N, K, path, ydt, xdt, use_ws, use_bias


@pytest.mark.parametrize("seed", list(range(128)))
def test_random_call_matches_oracle(cuda, seed):
    import torch
    qt, M, N, K, path, ydt, xdt, use_ws, use_bias = _case(seed)
    w = mx.synth_gguf(qt, N, K, 1000 + seed)
    pw = mx.pack_weights(w, N, K, qt, device=cuda)
    bits = mx.synth_act(M * K, xdt, 2000 + seed)
    x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda)
    x = x.view(torch.bfloat16 if xdt == mx.BF16 else torch.float16)
    xf = (orc.bf16_bits_to_f32(bits) if xdt == mx.BF16 else orc.f16_bits_to_f32(bits)).reshape(M, K)
    bias = torch.linspace(-1, 1, N, device=cuda).to(torch.bfloat16) if use_bias else None
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[ydt]
    ycode = {"bf16": mx.BF16, "f16": mx.F16, "f32": mx.F32}[ydt]
    need = mx.workspace_size(qt, N, K, M) if use_ws else 0
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=cuda)
    L = mx.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run():
        y = torch.empty((M, N), dtype=tdt, device=cuda)
        rc = L.mlxr_qgemm_run_ws(int(qt), N, K, 0, pw.data_ptr(), x.data_ptr(), xdt,
                                 bias.data_ptr() if bias is not None else None, mx.BF16, y.data_ptr(), ycode, M,
                                 path, ws.data_ptr() if need else None, need, s)
        assert rc == 0, (L.mlxr_qgemm_last_error(), qt, M, N, K, path)
        return y

    y1, y2 = run(), run()
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    gemv = path == mx.PATH_GEMV or (path == mx.PATH_AUTO and mx.auto_path(qt, N, K, M) == mx.PATH_GEMV)
    bf = bias.float().cpu().numpy() if bias is not None else None
    yh = y1.float().cpu().numpy()
    exact = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bf)
    if gemv:
        ref = exact
    else:
        ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bf, w_to_bf16=xdt == mx.BF16, w_to_f16=xdt == mx.F16)
    label = (str(qt), M, N, K, path, ydt, xdt, use_ws, use_bias)
    # half-precision outputs add their own rounding (2^-9 / 2^-12 relative) to the contract
    assert orc.rel_err(yh, ref) <= TOL, label
    assert orc.normwise_rel_err(yh, exact) <= TOL, label


@pytest.mark.parametrize("seed", list(range(40)))
def test_random_grouped_call_matches_oracle(cuda, seed):
    """One to five weights sharing X (random types and N, so some share a launch and some
    run alone), with or without the workspace the library asks for: every output against
    the oracle as above, and the call repeated gives the same bits."""
    import torch
    rng = np.random.default_rng(5000 + seed)
    kq = bool(rng.integers(2))
    K = 256 * int(rng.integers(1, 9)) if kq else 32 * int(rng.integers(1, 65))
    pool = TYPES[:3] if kq else TYPES[3:]
    n = int(rng.integers(1, 6))
    specs = [(pool[int(rng.integers(len(pool)))], int(rng.integers(1, 600))) for _ in range(n)]
    M = int(rng.choice([1, 2, 4, 8, 33, 64, 100, 256, 300]))
    use_ws = bool(rng.integers(2))
    gg = [mx.synth_gguf(qt, N, K, 6000 + 16 * seed + i) for i, (qt, N) in enumerate(specs)]
    pws = [mx.pack_weights(g, N, K, qt, device=cuda) for g, (qt, N) in zip(gg, specs)]
    bits = mx.synth_act(M * K, mx.BF16, 7000 + seed)
    x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)
    xf = orc.bf16_bits_to_f32(bits).reshape(M, K)
    ys = mx.q_gemm_dequant_grouped(x, pws, out_dtype=torch.float32, workspace=use_ws)
    ys2 = mx.q_gemm_dequant_grouped(x, pws, out_dtype=torch.float32, workspace=use_ws)
    torch.cuda.synchronize()
    for i, ((qt, N), y, y2) in enumerate(zip(specs, ys, ys2)):
        label = (i, str(qt), M, N, K, use_ws)
        assert torch.equal(y, y2), label
        yh = y.cpu().numpy()
        exact = orc.gemm_f64(int(qt), M, N, K, gg[i], xf)
        ref = exact if M <= 4 else orc.gemm_f64(int(qt), M, N, K, gg[i], xf, w_to_bf16=True)
        assert orc.rel_err(yh, ref) <= TOL, label
        assert orc.normwise_rel_err(yh, exact) <= TOL, label


@pytest.mark.parametrize("seed", list(range(32)))
def test_random_swiglu_matches_oracle(cuda, seed):
    """The fused gate/up/gating entry at random M (the GEMV, skinny and tiled kernels), type,
    N and K, with and without its workspace: h against swish(g) * u of the oracle's g and u
    (over the operands each kernel multiplies)."""
    import torch
    rng = np.random.default_rng(8000 + seed)
    qt = TYPES[int(rng.integers(len(TYPES)))]
    blk = mx.get_default_group_size(qt)
    K = blk * int(rng.integers(1, 2048 // blk + 1)) if blk == 256 else 32 * int(rng.integers(1, 65))
    N = int(rng.integers(1, 600))
    M = int(rng.choice([1, 3, 4, 5, 8, 16, 31, 32, 33, 64, 100, 256]))
    use_ws = bool(rng.integers(2))
    wg = mx.synth_gguf(qt, N, K, 9000 + seed)
    wu = mx.synth_gguf(qt, N, K, 9500 + seed)
    pg = mx.pack_weights(wg, N, K, qt, device=cuda)
    pu = mx.pack_weights(wu, N, K, qt, device=cuda)
    bits = mx.synth_act(M * K, mx.BF16, 9900 + seed)
    x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)
    xf = orc.bf16_bits_to_f32(bits).reshape(M, K)
    h = mx.q_gemm_swiglu(x, pg, pu, out_dtype=torch.float32, workspace=use_ws)
    h2 = mx.q_gemm_swiglu(x, pg, pu, out_dtype=torch.float32, workspace=use_ws)
    torch.cuda.synchronize()
    label = (str(qt), M, N, K, use_ws)
    assert torch.equal(h, h2), label
    rb = M > 4
    g = orc.gemm_f64(int(qt), M, N, K, wg, xf, w_to_bf16=rb).astype(np.float64)
    u = orc.gemm_f64(int(qt), M, N, K, wu, xf, w_to_bf16=rb).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    assert orc.rel_err(h.cpu().numpy(), ref) <= TOL, label


@pytest.mark.parametrize("seed", list(range(16)))
def test_random_staged_skinny_call_matches_oracle(cuda, seed):
    """Random shapes in the range where the narrow skinny kernel stages its activations in
    LDS (M <= 8 through the MFMA path, thousands of rows, K of 4096 or a little less or more):
    the staged call gives the same bits as the global-read one, and both are within the
    contract of the oracle over the bf16-rounded weights."""
    import torch
    rng = np.random.default_rng(12000 + seed)
    qt = TYPES[int(rng.integers(len(TYPES)))]
    blk = mx.get_default_group_size(qt)
    K = 4096 + blk * int(rng.integers(-2, 3))
    M = int(rng.integers(1, 9))
    N = int(rng.integers(6000, 16000))
    use_bias = bool(rng.integers(2))
    ydt = str(rng.choice(["bf16", "f16", "f32"]))
    w = mx.synth_gguf(qt, N, K, 13000 + seed)
    pw = mx.pack_weights(w, N, K, qt, device=cuda)
    bits = mx.synth_act(M * K, mx.BF16, 14000 + seed)
    x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)
    xf = orc.bf16_bits_to_f32(bits).reshape(M, K)
    bias = torch.linspace(-1, 1, N, device=cuda).to(torch.bfloat16) if use_bias else None
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[ydt]
    ys = {}
    try:
        for on in (True, False):
            mx.qgemm.test_skinny_stage(on)
            ys[on] = mx.q_gemm_dequant(x, pw, M, N, K, qt, bias=bias, out_dtype=tdt, path=mx.PATH_MFMA)
    finally:
        mx.qgemm.test_skinny_stage(True)
    torch.cuda.synchronize()
    label = (str(qt), M, N, K, use_bias, ydt)
    assert torch.equal(ys[True], ys[False]), label
    bf = bias.float().cpu().numpy() if bias is not None else None
    ref = orc.gemm_f64(int(qt), M, N, K, w, xf, bias=bf, w_to_bf16=True)
    assert orc.rel_err(ys[True].float().cpu().numpy(), ref) <= TOL, label


@pytest.mark.parametrize("chunk", list(range(8)))
def test_random_calls_against_dequantized_weights(cuda, chunk):
    """50 seeded random calls per chunk, wider than the oracle cases (M to 600, N to 15000,
    K to 16384, fp16 activations, workspaces of random bytes or one byte short of the size
    asked for): each against an fp64 product over the library's own dequantized weights
    (bit-exact to the oracle by the dequant tests; rounded to the activation type where an
    MFMA kernel consumes them), within the 5e-3 contract, and bit-identical on repeat."""
    import torch
    fails = []
    for it in range(50 * chunk, 50 * chunk + 50):
        rng = np.random.default_rng(20000 + it)
        qt = TYPES[int(rng.integers(len(TYPES)))]
        blk = mx.get_default_group_size(qt)
        K = blk * int(rng.integers(1, (16384 if rng.random() < 0.2 else 4096) // blk + 1))
        M = int(rng.choice([1, 2, 4, 5, 7, 8, 9, 16, 17, 31, 32, 33, 48, 64, 65, 128, 200, 256, 300, 600]))
        N = int(rng.integers(1, 3000)) if rng.random() < 0.7 else int(rng.integers(3000, 15000))
        path = int(rng.choice([mx.PATH_AUTO, mx.PATH_AUTO, mx.PATH_MFMA] + ([mx.PATH_GEMV] if M <= 64 else [])))
        xdt = mx.BF16 if rng.random() < 0.8 else mx.F16
        ydt = int(rng.choice([mx.BF16, mx.F16, mx.F32]))
        wsmode = int(rng.integers(3))  # none, the size asked for (random bytes), one byte short
        pw = mx.pack_weights(mx.synth_gguf(qt, N, K, 30000 + it), N, K, qt, device=cuda)
        g = torch.Generator(device=cuda).manual_seed(40000 + it)
        x = (torch.randn(M, K, device=cuda, generator=g) * 0.7).to(torch.bfloat16 if xdt == mx.BF16 else torch.float16)
        bias = torch.randn(N, device=cuda, generator=g).to(torch.bfloat16) if rng.random() < 0.5 else None
        need = mx.workspace_size(qt, N, K, M)
        nb = 0 if wsmode == 0 or need == 0 else (need if wsmode == 1 else need - 1)
        ws = torch.randint(0, 256, (max(nb, 1),), dtype=torch.uint8, device=cuda, generator=g)
        tdt = {mx.BF16: torch.bfloat16, mx.F16: torch.float16, mx.F32: torch.float32}[ydt]
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        ys = []
        for _ in range(2):
            y = torch.empty((M, N), dtype=tdt, device=cuda)
            rc = mx.lib().mlxr_qgemm_run_ws(int(qt), N, K, 0, pw.data_ptr(), x.data_ptr(), xdt,
                                            bias.data_ptr() if bias is not None else None, mx.BF16, y.data_ptr(),
                                            ydt, M, path, ws.data_ptr() if nb else None, nb, s)
            assert rc == 0, (mx.lib().mlxr_qgemm_last_error(), it)
            ys.append(y)
        wd = mx.dequantize(pw, torch.float32)
        if not (path == mx.PATH_GEMV or (path == mx.PATH_AUTO and mx.auto_path(qt, N, K, M) == mx.PATH_GEMV)):
            wd = wd.to(x.dtype).float()
        ref = x.double() @ wd.double().T
        if bias is not None:
            ref += bias.double()
        err = ((ys[0].double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        label = (it, str(qt), M, N, K, path, xdt, ydt, wsmode, bias is not None)
        if not torch.equal(ys[0], ys[1]) or not err <= TOL:
            fails.append((label, err))
    assert not fails, fails
