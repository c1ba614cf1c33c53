"""The packed HBM layout (mlxr_amd/csrc/qgemm_layout.h), stated in numpy by
tests/packref.py, decodes back to exactly the oracle's GGUF dequantization.  The GPU pack
kernels are compared byte for byte against packref (tests/test_gpu_parity.py), so this
closes the chain GGUF -> packed -> weights on the CPU."""
import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc
from tests import packref


def _nibbles(words):
    """[..., 4] pair-interleaved u32 words -> [..., 32] values 0..15 in weight order."""
    out = np.empty(words.shape[:-1] + (32,), np.uint32)
    for e in range(32):
        out[..., e] = (words[..., e >> 3] >> np.uint32(packref.pi_shift(e & 7))) & 15
    return out


def decode(qt, N, K, planes):
    if qt == 3:
        nsb = K // 256
        q = _nibbles(planes[0].view(np.uint32).reshape(N, nsb, 8, 4)).astype(np.float32)
        h = planes[1].view(np.uint16).reshape(N, nsb, 8).astype(np.uint32)
        dd = np.zeros((N, nsb), np.uint32)
        for j in range(8):
            dd |= ((h[..., j] >> 12) & 15) << np.uint32(4 * j)
        d = (dd & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
        dmin = (dd >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
        sc = (h & 63).astype(np.float32)
        m = ((h >> 6) & 63).astype(np.float32)
        dsc = (d[..., None] * sc)[..., None]          # exact
        dm = (dmin[..., None] * m)[..., None]         # exact
        return (dsc * q - dm).reshape(N, K)           # one rounding, as in the formula
    if qt == 4:
        nsb = K // 256
        lo = _nibbles(planes[0].view(np.uint32).reshape(N, nsb, 8, 4))
        hw = planes[1].view(np.uint32).reshape(N, nsb, 8, 2)
        hi = np.empty_like(lo)
        for e in range(32):
            hi[..., e] = (hw[..., e >> 4] >> np.uint32(packref.q6h_shift(e))) & 3
        q = (lo | (hi << 4)).astype(np.int32) - 32
        sc = planes[2].view(np.int8).reshape(N, nsb, 8, 2).astype(np.float32)
        d = planes[3].view(np.float16).reshape(N, nsb).astype(np.float32)
        ds = d[..., None, None] * sc                  # [N, nsb, 8, 2]
        w = np.repeat(ds, 16, axis=-1) * q.astype(np.float32)
        return w.reshape(N, K)
    if qt == 10:
        nsb = K // 256
        q = _nibbles(planes[0].view(np.uint32).reshape(N, nsb, 8, 4))
        hw = planes[1].view(np.uint32).reshape(N, nsb, 8)
        for e in range(32):
            q[..., e] |= ((hw >> np.uint32(packref.q5h_bit(e))) & 1) << 4
        q = q.astype(np.float32)
        h = planes[2].view(np.uint16).reshape(N, nsb, 8).astype(np.uint32)
        dd = np.zeros((N, nsb), np.uint32)
        for j in range(8):
            dd |= ((h[..., j] >> 12) & 15) << np.uint32(4 * j)
        d = (dd & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
        dmin = (dd >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
        dsc = (d[..., None] * (h & 63).astype(np.float32))[..., None]
        dm = (dmin[..., None] * ((h >> 6) & 63).astype(np.float32))[..., None]
        return (dsc * q - dm).reshape(N, K)
    if qt in (0, 1):
        nb = K // 32
        q = _nibbles(planes[0].view(np.uint32).reshape(N, nb, 4)).astype(np.float32)
        hdr = planes[1].view(np.float16).reshape(N, nb, 1 if qt == 0 else 2).astype(np.float32)
        d = hdr[..., 0:1]
        if qt == 0:
            return ((q - np.float32(8)) * d).reshape(N, K)  # exact
        return (q * d + hdr[..., 1:2]).reshape(N, K)      # product exact, one rounding
    nb = K // 32
    q = planes[0].view(np.int8).reshape(N, nb, 32).astype(np.float32)
    d = planes[1].view(np.float16).reshape(N, nb).astype(np.float32)
    return (q * d[..., None]).reshape(N, K)


@pytest.mark.parametrize("qt,N,K", [(3, 8, 1024), (4, 6, 768), (2, 5, 256), (3, 1, 256), (0, 7, 96), (1, 5, 320), (10, 6, 768)])
def test_packed_layout_decodes_to_oracle(qt, N, K):
    w = mx.synth_gguf(qt, N, K, 100 + qt)
    got = decode(qt, N, K, packref.planes(qt, N, K, w))
    np.testing.assert_array_equal(got.view(np.uint32), orc.dequant(qt, N, K, w).view(np.uint32))


@pytest.mark.parametrize("qt,N,K", [(3, 14336, 4096), (4, 1024, 8192), (2, 2048, 2048), (0, 4096, 4096),
                                    (1, 1024, 2080), (10, 1024, 4096)])
def test_packed_size_is_gguf_size(qt, N, K):
    planes = packref.planes(qt, N, K, np.zeros(mx.gguf_size(qt, N, K), np.uint8))
    assert sum(p.size for p in planes) == mx.gguf_size(qt, N, K)
    assert packref.pack(qt, N, K, np.zeros(mx.gguf_size(qt, N, K), np.uint8)).size == mx.packed_size(qt, N, K)
