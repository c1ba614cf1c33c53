"""mlxr_qgemm_run_noalloc (the entry point that allocates nothing: split-K partials in the
library's fixed per-GPU scratch array) against mlxr_qgemm_run_ws with a caller workspace of
the same size, through the C ABI: bit for bit, on two calls in a row (the second with a
smaller input), and the error for a plan that needs more scratch than the array holds."""
import ctypes

import numpy as np
import pytest

import mlxr_amd as mx
from mlxr_amd import qgemm

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20  # MLXR_NOALLOC_SCRATCH_BYTES
Q4K = int(mx.QuantType.Q4_K)


def _need(N, K, M):
    n = ctypes.c_size_t(0)
    assert qgemm.lib().mlxr_qgemm_workspace_size(Q4K, N, K, M, ctypes.byref(n)) == 0
    return n.value


def _x(torch, M, K, seed, cuda):
    bits = mx.synth_act(M * K, mx.BF16, seed)
    return torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)


def _run(torch, fn_noalloc, pw, x, N, K, M, ws=None):
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=x.device)
    lib = qgemm.lib()
    args = (Q4K, N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, None, mx.F32, y.data_ptr(), mx.F32, M, 0)
    if fn_noalloc:
        rc = lib.mlxr_qgemm_run_noalloc(*args, None)
    else:
        rc = lib.mlxr_qgemm_run_ws(*args, ws.data_ptr(), ws.numel(), None)
    assert rc == 0, qgemm.lib().mlxr_qgemm_last_error()
    torch.cuda.synchronize()
    return y


def test_noalloc_equals_workspace_entry_point(cuda):
    import torch
    N, K = 4096, 4096
    w = mx.synth_gguf(Q4K, N, K, 5)
    pw = mx.pack_weights(w, N, K, Q4K, device=cuda)
    ws = torch.empty(SCRATCH, dtype=torch.uint8, device=cuda)
    # first call: prefill rows whose tiled launch splits K; second: a smaller batched-decode
    # input whose skinny launch splits K too (down shape), so the array is reused
    cases = [(N, K, 512, pw, 11), (4096, 14336, 8, None, 12)]
    for N_, K_, M, p, seed in cases:
        if p is None:
            p = mx.pack_weights(mx.synth_gguf(Q4K, N_, K_, 6), N_, K_, Q4K, device=cuda)
        need = _need(N_, K_, M)
        assert 0 < need <= SCRATCH, (M, need)
        x = _x(torch, M, K_, seed, cuda)
        y0 = _run(torch, True, p, x, N_, K_, M)
        y1 = _run(torch, False, p, x, N_, K_, M, ws)
        assert torch.equal(y0, y1), M
        assert torch.isfinite(y0).all()


def test_noalloc_without_split_and_too_large(cuda):
    import torch
    N, K = 512, 1024
    pw = mx.pack_weights(mx.synth_gguf(Q4K, N, K, 7), N, K, Q4K, device=cuda)
    x = _x(torch, 1, K, 13, cuda)
    assert _need(N, K, 1) == 0  # GEMV: no scratch at all
    y0 = _run(torch, True, pw, x, N, K, 1)
    y1 = _run(torch, False, pw, x, N, K, 1, torch.empty(16, dtype=torch.uint8, device=cuda))
    assert torch.equal(y0, y1)
    # a plan needing more than the array (Llama-3-8B down at M = 1024 splits K four
    # ways: 64 MiB of partials): a clear error, nothing launched
    N2, K2, M2 = 4096, 14336, 1024
    assert _need(N2, K2, M2) > SCRATCH
    pw2 = mx.pack_weights(mx.synth_gguf(Q4K, N2, K2, 8), N2, K2, Q4K, device=cuda)
    x2 = _x(torch, M2, K2, 14, cuda)
    y = torch.zeros((M2, N2), dtype=torch.float32, device=cuda)
    rc = qgemm.lib().mlxr_qgemm_run_noalloc(Q4K, N2, K2, 0, pw2.data_ptr(), x2.data_ptr(), mx.BF16, None, mx.F32,
                                            y.data_ptr(), mx.F32, M2, 0, None)
    assert rc == -1
    assert b"scratch" in qgemm.lib().mlxr_qgemm_last_error()
    torch.cuda.synchronize()
    assert not y.any()
