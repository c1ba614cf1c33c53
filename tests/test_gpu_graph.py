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
