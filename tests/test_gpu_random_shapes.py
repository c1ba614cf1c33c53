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
    gemv = path == mx.PATH_GEMV or (path == mx.PATH_AUTO and M <= 4)
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
