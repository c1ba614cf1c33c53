"""Quantized weights from a .gguf file on disk go through the mapped reader, the upload and
the matmul, and give exactly the results of the same blocks packed from host memory."""
import numpy as np
import pytest

import mlxr_amd as mx
from mlxr_amd import gguf
from oracle import orc
from tests import gguf_writer as gw

pytestmark = pytest.mark.gpu
TOL = 5e-3


def test_gguf_upload_matches_pack(cuda, tmp_path):
    import torch
    T = gguf.GGMLType
    specs = [("blk.0.attn_q.weight", T.Q4_K, mx.QuantType.Q4_K, 256, 1024),
             ("blk.0.attn_v.weight", T.Q6_K, mx.QuantType.Q6_K, 128, 512),
             ("blk.0.ffn_down.weight", T.Q8_0, mx.QuantType.Q8_0, 96, 1056),
             ("blk.1.attn_q.weight", T.Q4_0, mx.QuantType.Q4_0, 64, 544),
             ("blk.1.attn_k.weight", T.Q4_1, mx.QuantType.Q4_1, 80, 256),
             ("blk.1.ffn_up.weight", T.Q5_K, mx.QuantType.Q5_K, 72, 768)]
    w = gw.Writer(3, alignment=64)
    w.add("general.architecture", gw.STR, "llama")
    blocks = {}
    for i, (name, gt, qt, N, K) in enumerate(specs):
        blocks[name] = mx.synth_gguf(qt, N, K, 300 + i)
        w.add_tensor(name, [K, N], gt, blocks[name].tobytes())
    w.add_tensor("output_norm.weight", [4096], T.F32, np.ones(4096, np.float32).tobytes())
    p = tmp_path / "w.gguf"
    p.write_bytes(w.to_bytes()[0])
    with gguf.GGUFFile(str(p)) as g:
        with pytest.raises(mx.QGemmError):
            g.upload("output_norm.weight", device=cuda)  # not a quantized matmul weight
        for i, (name, gt, qt, N, K) in enumerate(specs):
            pw = g.upload(name, device=cuda)
            assert (pw.qtype, pw.N, pw.K) == (qt, N, K)
            ref_pw = mx.pack_weights(blocks[name], N, K, qt, device=cuda)
            # same planes (the bytes between 256-aligned planes are padding, never written)
            assert torch.equal(mx.dequantize(pw).view(torch.int32), mx.dequantize(ref_pw).view(torch.int32))
            for M in (1, 37, 300):
                bits = mx.synth_act(M * K, mx.BF16, 400 + M)
                x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(cuda).view(torch.bfloat16)
                y = mx.q_gemm_dequant(x, pw, M, N, K, qt, out_dtype=torch.float32)
                ref = orc.gemm_f64(int(qt), M, N, K, blocks[name], orc.bf16_bits_to_f32(bits).reshape(M, K),
                                   w_to_bf16=M > 4)
                assert orc.rel_err(y.cpu().numpy(), ref) <= TOL, (name, M)
