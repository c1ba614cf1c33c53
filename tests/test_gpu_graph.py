"""hipGraph capture of the library's launches (the 70B-layer configuration captures its
seven GEMMs in one graph).  Every replay, with eager work and synchronisations in between,
must equal the eager result bit for bit."""
import numpy as np
import pytest

import mlxr_amd as mx

pytestmark = pytest.mark.gpu

SPECS = [("q", 512, 1024, 3), ("v", 256, 1024, 4), ("down", 1024, 2048, 4), ("tl", 256, 512, 2)]


@pytest.mark.parametrize("M", [1, 3, 256])
def test_graph_replays_match_eager(cuda, M):
    import torch
    ws = {n: mx.pack_weights(mx.synth_gguf(qt, N, K, 7 + i), N, K, qt, device=cuda)
          for i, (n, N, K, qt) in enumerate(SPECS)}
    xs = {}
    for n, N, K, qt in SPECS:
        bits = mx.synth_act(M * K, mx.BF16, 11 + K)
        xs[n] = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)
    ys = {n: torch.empty((M, N), dtype=torch.bfloat16, device=cuda) for n, N, K, qt in SPECS}

    def layer():
        for n, N, K, qt in SPECS:
            mx.q_gemm_dequant(xs[n], ws[n], M, N, K, qt, out=ys[n])

    layer()
    torch.cuda.synchronize()
    ref = {n: ys[n].clone() for n in ys}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # capture on the stream that ran the warm-up call: the library's split-K workspace is
    # per stream and is allocated outside capture
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        layer()
    for it in range(4):
        for y in ys.values():
            y.fill_(float(it + 1))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n in ys:
            assert torch.equal(ys[n], ref[n]), (it, n)


@pytest.mark.parametrize("M", [1, 8, 130, 512])
def test_graph_mlp_and_grouped_replays_match_eager(cuda, M):
    """A decoder layer's matmul calls as a decode or prefill engine captures them: grouped
    q/k/v, the fused gate+up+SwiGLU and the down projection (split-K workspaces from torch's
    allocator inside the capture at the sizes that split).  Replays with eager work between
    them equal the eager result bit for bit."""
    import torch
    Q4K = int(mx.QuantType.Q4_K)
    H, F = 512, 1536
    W = {n: mx.pack_weights(mx.synth_gguf(Q4K, N, K, 21 + i), N, K, Q4K, device=cuda)
         for i, (n, N, K) in enumerate((("q", H, H), ("k", H // 4, H), ("v", H // 4, H), ("gate", F, H),
                                        ("up", F, H), ("down", H, F)))}
    bits = mx.synth_act(M * H, mx.BF16, 31 + M)
    x = torch.from_numpy(bits.view(np.int16).reshape(M, H)).to(cuda).view(torch.bfloat16)
    qkv = [torch.empty((M, W[n].N), dtype=torch.bfloat16, device=cuda) for n in ("q", "k", "v")]
    y = torch.empty((M, H), dtype=torch.bfloat16, device=cuda)
    h = torch.empty((M, F), dtype=torch.bfloat16, device=cuda)

    def layer():
        mx.q_gemm_dequant_grouped(x, [W["q"], W["k"], W["v"]], outs=qkv)
        mx.q_gemm_swiglu(x, W["gate"], W["up"], out=h)
        mx.q_gemm_dequant(h, W["down"], M, H, F, Q4K, out=y)

    layer()
    torch.cuda.synchronize()
    ref = [t.clone() for t in qkv + [h, y]]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        layer()
    for it in range(4):
        for t in qkv + [h, y]:
            t.fill_(float(it + 1))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k, (t, r) in enumerate(zip(qkv + [h, y], ref)):
            assert torch.equal(t, r), (it, k)
