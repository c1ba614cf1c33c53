"""The SwiGLU MLP (mlxr_qgemm_mlp_ex): y = down . (swish(x . gate^T) * (x . up^T)).

The default runs the fused gate/up/gating launch and the down projection.  In the
one-launch mode (M = 1) the whole MLP is one launch whose down workgroups wait at
device-scope counters for the gate/up workgroups (reference core/kernels/metal/swiglu_mlp_fused.metal:110-131
fuses the same chain).  Checked three ways: bit for bit against the two-launch chain
(mlxr_qgemm_swiglu, then the down GEMV), stage by stage against the oracle (h against fp64
gating of the oracle's projections, y against the oracle's down over that h, y normwise
against the all-fp64 MLP), and through graph replays with changing inputs (so a stale h or
a counter left non-zero would show)."""
import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc

pytestmark = pytest.mark.gpu

TOL = 5e-3
Q = mx.QuantType
ONE = mx.qgemm.MLP_ONE_LAUNCH


def _swiglu64(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


def _bf16_round(a):
    import torch
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _weights(cuda, qgu, qd, H, I, seed):
    wg, wu, wd = mx.synth_gguf(qgu, I, H, seed), mx.synth_gguf(qgu, I, H, seed + 1), mx.synth_gguf(qd, H, I, seed + 2)
    return (wg, wu, wd), tuple(mx.pack_weights(w, N, K, qt, device=cuda)
                               for w, N, K, qt in ((wg, I, H, qgu), (wu, I, H, qgu), (wd, H, I, qd)))


def _act(torch, M, K, seed, cuda):
    bits = mx.synth_act(M * K, mx.BF16, seed)
    return (torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16),
            orc.bf16_bits_to_f32(bits).reshape(M, K))


def _check_oracle(qgu, qd, H, I, raw, xf, wb, y, h):
    """Stage by stage against the oracle, both error metrics: h (the kernel's own, read back
    from the workspace or the chain) against fp64 gating of the oracle's gate/up, and y
    against the oracle's down over that h; plus y normwise against the all-fp64 chain with
    h rounded to bf16 (elementwise that comparison is not meaningful: one bf16 rounding
    step of an h element moves small outputs by several per cent)."""
    wg, wu, wd = raw
    M = xf.shape[0]
    g = orc.gemm_f64(int(qgu), M, I, H, wg, xf, w_to_bf16=wb)
    u = orc.gemm_f64(int(qgu), M, I, H, wu, xf, w_to_bf16=wb)
    h64 = _swiglu64(g, u)
    assert orc.rel_err(h, h64) <= TOL
    assert orc.rel_err(y, orc.gemm_f64(int(qd), M, H, I, wd, h, w_to_bf16=wb)) <= TOL
    y64 = orc.gemm_f64(int(qd), M, H, I, wd, _bf16_round(h64), w_to_bf16=wb)
    assert orc.normwise_rel_err(y, y64) <= TOL


def _ws_h(ws, M, I):
    """The gated intermediate h the MLP left in its workspace (bf16, after the sync region)."""
    import torch
    o = mx.qgemm.MLP_H_OFFSET
    return ws.buf[o:o + 2 * M * I].view(torch.bfloat16).float().reshape(M, I).cpu().numpy()


def _chain(torch, x, pg, pu, pd, out_dtype):
    h = mx.q_gemm_swiglu(x, pg, pu)
    return mx.q_gemm_dequant(h, pd, x.shape[0], pd.N, pd.K, pd.qtype, out_dtype=out_dtype)


@pytest.mark.parametrize("qgu,qd,H,I", [(Q.Q4_K, Q.Q4_K, 1024, 2048), (Q.Q4_K, Q.Q6_K, 768, 1280),
                                        (Q.Q6_K, Q.Q6_K, 512, 2816), (Q.Q8_0, Q.Q8_0, 1024, 1536),
                                        (Q.Q5_K, Q.Q6_K, 1024, 2048), (Q.Q4_0, Q.Q4_0, 640, 1024),
                                        (Q.Q4_1, Q.Q6_K, 1024, 768)])
def test_mlp_m1_one_launch_equals_chain_and_oracle(cuda, qgu, qd, H, I):
    import torch
    raw, (pg, pu, pd) = _weights(cuda, qgu, qd, H, I, 300 + H + I)
    ws = mx.MlpWorkspace(cuda)
    for seed in (1, 2):  # two inputs through one workspace: the second must not see the first's h
        x, xf = _act(torch, 1, H, 400 + seed, cuda)
        for odt in (torch.bfloat16, torch.float32):
            y = mx.q_gemm_mlp(x, pg, pu, pd, ws, out_dtype=odt, mode=ONE)
            assert torch.equal(y, _chain(torch, x, pg, pu, pd, odt)), (seed, odt)
        _check_oracle(qgu, qd, H, I, raw, xf, False, y.cpu().numpy(), _ws_h(ws, 1, I))
    ws.status()


def test_mlp_llama3_8b_full_size(cuda):
    """Llama-3-8B MLP (hidden 4096, intermediate 14336, Q4_K) at M = 1 against the oracle on
    every output, and against the chain bit for bit."""
    import torch
    H, I = 4096, 14336
    raw, (pg, pu, pd) = _weights(cuda, Q.Q4_K, Q.Q4_K, H, I, 501)
    x, xf = _act(torch, 1, H, 502, cuda)
    ws = mx.MlpWorkspace(cuda)
    y = mx.q_gemm_mlp(x, pg, pu, pd, ws, mode=ONE)
    assert torch.equal(y, _chain(torch, x, pg, pu, pd, torch.bfloat16))
    assert torch.equal(y, mx.q_gemm_mlp(x, pg, pu, pd, ws))  # the default (two launches)
    _check_oracle(Q.Q4_K, Q.Q4_K, H, I, raw, xf, False, y.float().cpu().numpy(), _ws_h(ws, 1, I))
    ws.status()


@pytest.mark.parametrize("M", [2, 4, 8, 40, 130])
def test_mlp_batched_matches_oracle(cuda, M):
    """Above M = 1 the MLP runs as the fused gate/up/gating launch and the down projection."""
    import torch
    H, I = 1024, 2048
    raw, (pg, pu, pd) = _weights(cuda, Q.Q4_K, Q.Q6_K, H, I, 600)
    x, xf = _act(torch, M, H, 601 + M, cuda)
    ws = mx.MlpWorkspace(cuda)
    y = mx.q_gemm_mlp(x, pg, pu, pd, ws, out_dtype=torch.float32)
    assert torch.equal(y, _chain(torch, x, pg, pu, pd, torch.float32))
    _check_oracle(Q.Q4_K, Q.Q6_K, H, I, raw, xf, M > 4, y.cpu().numpy(), _ws_h(ws, M, I))


def test_mlp_graph_replays_with_changing_input(cuda):
    """The one-launch MLP captured in a graph: each replay, with a new input copied in
    between and eager work between replays, equals the eager result for that input -- so
    the counters are back at zero after every launch and h is never read stale."""
    import torch
    H, I = 1024, 4096
    _, (pg, pu, pd) = _weights(cuda, Q.Q4_K, Q.Q4_K, H, I, 700)
    ws = mx.MlpWorkspace(cuda)
    xs = [_act(torch, 1, H, 701 + i, cuda)[0] for i in range(4)]
    eager = [mx.q_gemm_mlp(x, pg, pu, pd, ws, mode=ONE).clone() for x in xs]
    xin = xs[0].clone()
    yout = torch.empty((1, H), dtype=torch.bfloat16, device=cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mx.q_gemm_mlp(xin, pg, pu, pd, ws, out=yout, mode=ONE)  # workspace sized outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mx.q_gemm_mlp(xin, pg, pu, pd, ws, out=yout, mode=ONE)
    for rep in range(3):
        for i, x in enumerate(xs):
            xin.copy_(x)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yout, eager[i]), (rep, i)
            _chain(torch, x, pg, pu, pd, torch.bfloat16)  # eager work between replays
    ws.status()


def test_mlp_wait_timeout_is_reported_and_recovers(cuda):
    """With the wait bound lowered to one tick the down workgroups give up at once: the
    launch still ends, mlxr_qgemm_mlp_status reports MLXR_E_TIMEOUT (and clears it), and
    the next launch on the same workspace -- bound restored -- is exact again (the
    counters were returned to zero by the last workgroup)."""
    import torch
    H, I = 4096, 14336
    _, (pg, pu, pd) = _weights(cuda, Q.Q4_K, Q.Q4_K, H, I, 800)
    x, _ = _act(torch, 1, H, 801, cuda)
    ws = mx.MlpWorkspace(cuda)
    ref = _chain(torch, x, pg, pu, pd, torch.bfloat16)
    try:
        mx.qgemm.test_set_mlp_spin_limit(1)
        mx.q_gemm_mlp(x, pg, pu, pd, ws, mode=ONE)
        torch.cuda.synchronize()
    finally:
        mx.qgemm.test_set_mlp_spin_limit(0)
    with pytest.raises(mx.QGemmError) as ei:
        ws.status()
    assert ei.value.code == -6
    ws.status()  # cleared
    for _ in range(2):
        y = mx.q_gemm_mlp(x, pg, pu, pd, ws, mode=ONE)
        assert torch.equal(y, ref)
    ws.status()


def test_mlp_argument_errors(cuda):
    import torch
    _, (pg, pu, pd) = _weights(cuda, Q.Q4_K, Q.Q4_K, 512, 1024, 900)
    x, _ = _act(torch, 1, 512, 901, cuda)
    with pytest.raises(mx.QGemmError):
        mx.q_gemm_mlp(x, pg, pu, pg, mx.MlpWorkspace(cuda))  # down of the wrong shape
    lib = mx.lib()
    # a workspace smaller than asked for is refused
    rc = lib.mlxr_qgemm_mlp(3, 3, 512, 1024, pg.data_ptr(), pu.data_ptr(), pd.data_ptr(), x.data_ptr(), 2,
                            x.data_ptr(), 2, 1, x.data_ptr(), 16, None)
    assert rc == -1 and b"workspace" in lib.mlxr_qgemm_last_error()
