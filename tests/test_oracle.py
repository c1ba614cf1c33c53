"""Pins the CPU oracle (oracle/orc.c) before it is trusted as the checker.

The reference has no test, fixture or golden vector for q_gemm numerics, so each oracle
function is pinned against what the mathematics and the GGUF format fix:
  - fp16 -> fp32: exhaustively against numpy, and the reference's own powf formulation
    (q_gemm_dequant_primitive.mm:141-165) agrees on every non-NaN code;
  - fp32 -> fp16 / bf16 round-to-nearest-even: against numpy / torch casts;
  - Q8_0 / Q4_K / Q6_K dequant: hand-derived known answers that isolate every bit field
    (one-hot scale bits, single ql/qh bits, scale-group index), an independent
    per-element decoder, and extreme scales;
  - the GEMMs: integer-valued special cases that are exact in any order (so the result
    must equal numpy's int64 matmul bit for bit), linearity, and fp64 numpy on the
    dequantized weights.
"""
import numpy as np
import pytest

import mlxr_amd as mx
from oracle import orc

Q80, Q4K, Q6K = 2, 3, 4


# ----------------------------------------------------------------------- conversions

def test_f16_to_f32_exhaustive():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_reference_fp16_formula_agrees_exhaustively():
    """The reference's powf-based fp16_to_fp32 (.mm:141-165) equals the bit conversion."""
    l = orc.lib()
    for c in range(65536):
        a, b = l.orc_f16_to_f32(c), l.orc_ref_fp16_to_fp32(c)
        if np.isnan(a):
            assert np.isnan(b)
        else:
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), hex(c)


def _edge_floats():
    rng = np.random.default_rng(1)
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, 6.0e-5,
         np.inf, -np.inf, 3.0e38]
    # exact fp16 halfway points: (h + 0.5 ulp) for random normal fp16 values
    h = rng.integers(0x0400, 0x7bff, 2000).astype(np.uint16).view(np.float16).astype(np.float64)
    ulp = np.spacing(h.astype(np.float16)).astype(np.float64)
    v += list(h + ulp / 2) + list(-(h + ulp / 2))
    v += list(rng.standard_normal(5000) * 10.0 ** rng.integers(-9, 5, 5000))
    return np.array(v, dtype=np.float32)


def test_f32_to_f16_rne():
    l = orc.lib()
    vals = _edge_floats()
    got = np.array([l.orc_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_rne():
    torch = pytest.importorskip("torch")
    l = orc.lib()
    rng = np.random.default_rng(2)
    vals = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000).astype(np.float32)
    # exact halfway cases between bf16 neighbours, both parities
    base = (rng.integers(0, 1 << 15, 4000).astype(np.uint32) << 16) | 0x8000
    vals = np.concatenate([vals, base.view(np.float32), np.array([0.0, -0.0, np.inf, -np.inf], np.float32)])
    vals = vals[np.isfinite(vals) | np.isinf(vals)]
    got = np.array([l.orc_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------------- sizes

def test_block_geometry_and_sizes():
    l = orc.lib()
    assert [l.orc_block_bytes(t) for t in (Q80, Q4K, Q6K)] == [34, 144, 210]
    assert [l.orc_block_elems(t) for t in (Q80, Q4K, Q6K)] == [32, 256, 256]
    # GGUF weight byte counts of the benchmark configurations (N·K/256·144 for Q4_K, N·K/32·34 for Q8_0)
    assert l.orc_weight_bytes(Q80, 2048, 2048) == 4456448
    assert l.orc_weight_bytes(Q4K, 4096, 4096) == 9437184
    assert l.orc_weight_bytes(Q4K, 1024, 4096) == 2359296
    assert l.orc_weight_bytes(Q4K, 14336, 4096) == 33030144
    assert l.orc_weight_bytes(Q4K, 4096, 14336) == 33030144
    assert l.orc_weight_bytes(Q6K, 1024, 8192) == 6881280
    assert l.orc_weight_bytes(Q6K, 8192, 28672) == 192675840


# ----------------------------------------------------------------------- block builders

def f16(v):
    return np.float16(v).view(np.uint16)


def q8_block(d_bits, qs):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[2:] = np.asarray(qs, np.int8).view(np.uint8)
    return b


def q4k_block(d_bits, dmin_bits, scales12, qs128):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin_bits], np.uint16).view(np.uint8)
    b[4:16] = scales12
    b[16:] = qs128
    return b


def q6k_block(ql, qh, sc, d_bits):
    b = np.zeros(210, np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([d_bits], np.uint16).view(np.uint8)
    return b


# ----------------------------------------------------------------------- Q8_0

def test_q8_0_known_answers():
    qs = np.arange(-16, 16)
    qs[0], qs[-1] = -127, 127
    for d in (1.0, 65504.0, 2.0 ** -24, 0.0, -0.5):
        blk = q8_block(f16(d), qs)
        got = orc.dequant(Q80, 1, 32, blk)[0]
        np.testing.assert_array_equal(got, qs.astype(np.float32) * np.float32(d))


# ---------------------------------------------------------------- Q4_0 / Q4_1

def q4_block(qt, d_bits, qs, m_bits=0):
    hb = np.array([d_bits] if qt == 0 else [d_bits, m_bits], np.uint16).view(np.uint8)
    return np.concatenate([hb, np.asarray(qs, np.uint8)])


def test_q4_0_element_order_and_values():
    # byte j = lo | hi << 4 with lo = j, hi = 15 - j: element j = j - 8, element j+16 = 7 - j
    qs = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    for d in (1.0, -0.5, 65504.0, 2.0 ** -24, 0.0):
        got = orc.dequant(0, 1, 32, q4_block(0, f16(d), qs))[0]
        want = np.array([j - 8 for j in range(16)] + [7 - j for j in range(16)], np.float32) * np.float32(d)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))  # incl. sign of zero


def test_q4_1_element_order_and_values():
    qs = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    for d, m in ((1.0, 0.0), (0.25, -3.0), (2.0 ** -14, 1.5), (0.0, -2.0), (3.0, -0.0)):
        got = orc.dequant(1, 1, 32, q4_block(1, f16(d), qs, f16(m)))[0]
        q = np.array(list(range(16)) + [15 - j for j in range(16)], np.float64)
        want = (q * d + m).astype(np.float32)  # q*d is exact, so the fp64 sum rounds once
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qt", [0, 1])
def test_q4_gguf_order_vs_reference_cpu_order(qt):
    """The reference's CPU routines (q_gemm_dequant_primitive.mm:189-216) give the same
    32 values in interleaved order: theirs[2i] = gguf[i], theirs[2i+1] = gguf[i+16]."""
    blk = mx.synth_gguf(qt, 1, 32, 9 + qt)
    g = orc.dequant(qt, 1, 32, blk)[0]
    r = orc.dequant_refcpu_q4(qt, blk)
    np.testing.assert_array_equal(r[0::2], g[:16])
    np.testing.assert_array_equal(r[1::2], g[16:])


@pytest.mark.parametrize("qt", [0, 1])
def test_q4_matches_elementwise_decoder(qt):
    N, K = 3, 128
    w = mx.synth_gguf(qt, N, K, 40 + qt)
    hb = 2 if qt == 0 else 4
    b = w.reshape(N, K // 32, hb + 16)
    out = np.empty((N, K), np.float32)
    for n in range(N):
        for blk in range(K // 32):
            d = np.float32(b[n, blk, 0:2].view(np.float16)[0])
            m = np.float32(b[n, blk, 2:4].view(np.float16)[0]) if qt == 1 else None
            for e in range(32):
                byte = int(b[n, blk, hb + (e % 16)])
                q = (byte & 15) if e < 16 else (byte >> 4)
                out[n, 32 * blk + e] = np.float32(q - 8) * d if qt == 0 else np.float32(np.float64(q) * d + m)
    np.testing.assert_array_equal(orc.dequant(qt, N, K, w).view(np.uint32), out.view(np.uint32))


# ----------------------------------------------------------------------- Q5_K

def q5k_block(d_bits, dmin_bits, scales, qh, qs):
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin_bits], np.uint16).view(np.uint8)
    b[4:16] = scales
    b[16:48] = qh
    b[48:176] = qs
    return b


_UNIT_SCALES = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)  # sc_j = 1, m_j = 0


@pytest.mark.parametrize("bit", range(8))
def test_q5k_single_qh_bit(bit):
    """qh[l] bit b is the fifth bit of element 32b + l (chunk b/2, high half if b odd)."""
    for l in (0, 7, 31):
        qh = np.zeros(32, np.uint8)
        qh[l] = 1 << bit
        got = orc.dequant(10, 1, 256, q5k_block(f16(1.0), f16(1.0), _UNIT_SCALES, qh, np.zeros(128, np.uint8)))[0]
        want = np.zeros(256, np.float32)
        want[32 * bit + l] = 16.0
        np.testing.assert_array_equal(got, want)


def test_q5k_matches_elementwise_decoder():
    N, K = 2, 512
    w = mx.synth_gguf(10, N, K, 71)
    b = w.reshape(N, K // 256, 176)
    out = np.empty((N, K), np.float32)
    for n in range(N):
        for s in range(K // 256):
            blk = b[n, s]
            d = np.float32(blk[0:2].view(np.float16)[0])
            dmin = np.float32(blk[2:4].view(np.float16)[0])
            sc = blk[4:16]
            for e in range(256):
                c, half, l = e // 64, (e // 32) % 2, e % 32
                j = 2 * c + half
                if j < 4:
                    scj, mj = sc[j] & 63, sc[j + 4] & 63
                else:
                    scj = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4)
                    mj = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
                byte = int(blk[48 + 32 * c + l])
                q = ((byte >> 4) if half else (byte & 15)) | (((int(blk[16 + l]) >> j) & 1) << 4)
                out[n, 256 * s + e] = np.float32(np.float64(d * np.float32(scj)) * q - np.float64(dmin * np.float32(mj)))
    np.testing.assert_array_equal(orc.dequant(10, N, K, w).view(np.uint32), out.view(np.uint32))


# ----------------------------------------------------------------------- Q4_K

# One-hot scale bits, derived by hand from the GGUF 12-byte packing: sub-blocks 0..3 keep
# their 6-bit scale in bytes 0..3 and 6-bit min in bytes 4..7 (bits 0..5); sub-blocks 4..7
# keep the low 4 bits of scale/min in the low/high nibble of bytes 8..11 and the top 2
# bits in bits 6..7 of bytes 0..3 (scale) / 4..7 (min).
def _q4k_onehot_expect(i, b):
    """(kind, sub-block, value) set by scales[i] = 1 << b."""
    if i < 4:
        return ("sc", i, 1 << b) if b < 6 else ("sc", i + 4, 1 << (b - 2))
    if i < 8:
        return ("m", i - 4, 1 << b) if b < 6 else ("m", i, 1 << (b - 2))
    return ("sc", i - 4, 1 << b) if b < 4 else ("m", i - 4, 1 << (b - 4))


@pytest.mark.parametrize("i", range(12))
@pytest.mark.parametrize("b", range(8))
def test_q4k_scale_bits_one_hot(i, b):
    s = np.zeros(12, np.uint8)
    s[i] = 1 << b
    blk = q4k_block(f16(1.0), f16(1.0), s, np.full(128, 0x11, np.uint8))  # q = 1 everywhere
    got = orc.dequant(Q4K, 1, 256, blk)[0]
    kind, j, val = _q4k_onehot_expect(i, b)
    exp = np.zeros(256, np.float32)  # w = sc*1 - m
    exp[32 * j:32 * j + 32] = val if kind == "sc" else -val
    np.testing.assert_array_equal(got, exp)


def test_q4k_element_order():
    """Chunk c (64 weights) takes qs[32c..32c+31]: low nibbles give weights 64c..64c+31,
    high nibbles 64c+32..64c+63 (unit scales, zero mins, d = 1 -> w = q)."""
    s = np.zeros(12, np.uint8)
    s[0:4] = 1       # sc 0..3 = 1
    s[8:12] = 0x01   # sc 4..7 = 1, m 4..7 = 0
    rng = np.random.default_rng(3)
    qs = rng.integers(0, 256, 128).astype(np.uint8)
    got = orc.dequant(Q4K, 1, 256, q4k_block(f16(1.0), f16(1.0), s, qs))[0]
    exp = np.empty(256, np.float32)
    for c in range(4):
        exp[64 * c:64 * c + 32] = qs[32 * c:32 * c + 32] & 15
        exp[64 * c + 32:64 * c + 64] = qs[32 * c:32 * c + 32] >> 4
    np.testing.assert_array_equal(got, exp)


def test_q4k_extremes():
    s = np.full(12, 0xFF, np.uint8)  # every scale and min = 63
    d, dmin = 0.001, 0.002
    dq, dmq = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    for qbyte, q in ((0x00, 0), (0xFF, 15)):
        got = orc.dequant(Q4K, 1, 256, q4k_block(f16(d), f16(dmin), s, np.full(128, qbyte, np.uint8)))[0]
        exp = np.float32(np.float32(dq * 63) * q - np.float32(dmq * 63))
        np.testing.assert_array_equal(got, np.full(256, exp, np.float32))
    got = orc.dequant(Q4K, 1, 256, q4k_block(0, 0, s, np.full(128, 0x5A, np.uint8)))[0]
    assert np.all(got == 0)


def _q4k_decode_elementwise(blk):
    """Independent decoder: for each weight e, find its nibble and its (scale, min) bits."""
    d = np.float32(blk[0:2].view(np.float16)[0])
    dmin = np.float32(blk[2:4].view(np.float16)[0])
    s = [int(x) for x in blk[4:16]]
    bits = sum(s[k] << (8 * k) for k in range(12))  # 96-bit little-endian integer
    out = np.empty(256, np.float32)
    for e in range(256):
        c, within = divmod(e, 64)
        hi = within >= 32
        byte = int(blk[16 + 32 * c + within % 32])
        q = byte >> 4 if hi else byte & 15
        j = 2 * c + int(hi)
        if j < 4:
            sc, m = (bits >> (8 * j)) & 63, (bits >> (8 * (j + 4))) & 63
        else:
            lo_sc = (bits >> (8 * (j + 4))) & 15
            lo_m = (bits >> (8 * (j + 4) + 4)) & 15
            sc = lo_sc | (((bits >> (8 * (j - 4) + 6)) & 3) << 4)
            m = lo_m | (((bits >> (8 * j + 6)) & 3) << 4)
        out[e] = np.float32(np.float32(d * np.float32(sc)) * np.float32(q) - np.float32(dmin * np.float32(m)))
    return out


def test_q4k_matches_elementwise_decoder():
    w = mx.synth_gguf(Q4K, 3, 512, 17)
    got = orc.dequant(Q4K, 3, 512, w)
    blocks = w.reshape(6, 144)
    ref = np.concatenate([_q4k_decode_elementwise(b) for b in blocks]).reshape(3, 512)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ----------------------------------------------------------------------- Q6_K

@pytest.mark.parametrize("i", [0, 5, 31, 32, 63, 64, 100, 127])
@pytest.mark.parametrize("b", range(8))
def test_q6k_single_ql_bit(i, b):
    """ql byte 64h + r: low nibble is the low 4 bits of weight 128h + r, high nibble of
    weight 128h + r + 64.  All other weights have q = 0 -> w = -32 (d = 1, scales 1)."""
    ql = np.zeros(128, np.uint8)
    ql[i] = 1 << b
    got = orc.dequant(Q6K, 1, 256, q6k_block(ql, np.zeros(64, np.uint8), np.ones(16), f16(1.0)))[0]
    exp = np.full(256, -32.0, np.float32)
    h, r = divmod(i, 64)
    e = 128 * h + r + (64 if b >= 4 else 0)
    exp[e] = (1 << (b % 4)) - 32
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("i", [0, 7, 31, 32, 63])
@pytest.mark.parametrize("b", range(8))
def test_q6k_single_qh_bit(i, b):
    """qh byte 32h + l: bits 2t..2t+1 are the high 2 bits of weight 128h + 32t + l."""
    qh = np.zeros(64, np.uint8)
    qh[i] = 1 << b
    got = orc.dequant(Q6K, 1, 256, q6k_block(np.zeros(128, np.uint8), qh, np.ones(16), f16(1.0)))[0]
    exp = np.full(256, -32.0, np.float32)
    h, l = divmod(i, 32)
    e = 128 * h + 32 * (b // 2) + l
    exp[e] = (16 << (b % 2)) - 32
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("g", range(16))
def test_q6k_scale_group(g):
    """Weight e uses scales[e // 16]; scales at the int8 range ends -32 and 31."""
    sc = np.ones(16, np.int64)
    sc[g] = -32
    sc[(g + 5) % 16] = 31
    ql = np.full(128, 0x77, np.uint8)  # low 4 bits 7
    got = orc.dequant(Q6K, 1, 256, q6k_block(ql, np.zeros(64, np.uint8), sc, f16(0.5)))[0]
    exp = np.repeat(sc.astype(np.float32), 16) * np.float32(0.5) * np.float32(7 - 32)
    np.testing.assert_array_equal(got, exp)


def _q6k_decode_elementwise(blk):
    d = np.float32(blk[208:210].view(np.float16)[0])
    sc = blk[192:208].view(np.int8)
    out = np.empty(256, np.float32)
    for e in range(256):
        h, r = divmod(e, 128)
        t, l = divmod(r, 32)
        qlb = int(blk[64 * h + l + 32 * (t & 1)])
        lo = (qlb >> 4) if t >= 2 else (qlb & 15)
        hi = (int(blk[128 + 32 * h + l]) >> (2 * t)) & 3
        out[e] = np.float32(d * np.float32(sc[e // 16])) * np.float32((lo | (hi << 4)) - 32)
    return out


def test_q6k_matches_elementwise_decoder():
    w = mx.synth_gguf(Q6K, 2, 768, 19)
    got = orc.dequant(Q6K, 2, 768, w)
    ref = np.concatenate([_q6k_decode_elementwise(b) for b in w.reshape(6, 210)]).reshape(2, 768)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ----------------------------------------------------------------------- GEMMs

def _integer_q4k(N, K, seed):
    """Q4_K weights that dequantize to w = q (d = 1, every scale 1, every min 0)."""
    rng = np.random.default_rng(seed)
    blocks = []
    for _ in range(N * K // 256):
        s = np.zeros(12, np.uint8)
        s[0:4] = 1
        s[8:12] = 1
        blocks.append(q4k_block(f16(1.0), f16(0.0), s, rng.integers(0, 256, 128).astype(np.uint8)))
    return np.concatenate(blocks)


@pytest.mark.parametrize("M,N,K", [(1, 8, 256), (3, 16, 512), (5, 7, 768)])
def test_gemm_integer_case_is_exact(M, N, K):
    """Integer weights and small integer activations: every partial sum is an integer
    below 2^24, so any summation order is exact and y must equal numpy's int64 matmul."""
    w = _integer_q4k(N, K, M + N)
    wq = orc.dequant(Q4K, N, K, w)
    assert np.all(wq == np.round(wq)) and wq.min() >= 0 and wq.max() <= 15
    x = np.random.default_rng(K).integers(-8, 9, (M, K)).astype(np.float32)
    ref = (x.astype(np.int64) @ wq.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(orc.gemm_f64(Q4K, M, N, K, w, x), ref)
    np.testing.assert_array_equal(orc.eval_cpu(Q4K, M, N, K, w, x), ref)
    bias = np.arange(N, dtype=np.float32)
    np.testing.assert_array_equal(orc.eval_cpu(Q4K, M, N, K, w, x, bias), ref + bias)
    np.testing.assert_array_equal(orc.gemm_f64(Q4K, M, N, K, w, x, bias), ref + bias)


@pytest.mark.parametrize("qt,K", [(Q80, 256), (Q4K, 512), (Q6K, 512)])
def test_gemm_against_numpy_fp64(qt, K):
    M, N = 4, 24
    w = mx.synth_gguf(qt, N, K, 23)
    x = orc.bf16_bits_to_f32(mx.synth_act(M * K, mx.BF16, 29)).reshape(M, K)
    wd = orc.dequant(qt, N, K, w).astype(np.float64)
    ref = (x.astype(np.float64) @ wd.T).astype(np.float32)
    np.testing.assert_allclose(orc.gemm_f64(qt, M, N, K, w, x), ref, rtol=0, atol=1e-6 * np.abs(ref).max())
    assert orc.normwise_rel_err(orc.eval_cpu(qt, M, N, K, w, x), ref) < 1e-5
    # rows subset and column sample agree with the full results
    np.testing.assert_array_equal(orc.gemm_f64(qt, M, N, K, w, x, m0=1, m1=3), orc.gemm_f64(qt, M, N, K, w, x)[1:3])
    cols = orc.eval_cpu_cols(qt, M, N, K, 8, 16, w, x)
    np.testing.assert_array_equal(cols[:, 8:16], orc.eval_cpu(qt, M, N, K, w, x)[:, 8:16])


def test_gemm_bf16_weight_rounding():
    torch = pytest.importorskip("torch")
    M, N, K = 2, 8, 512
    w = mx.synth_gguf(Q4K, N, K, 31)
    x = orc.bf16_bits_to_f32(mx.synth_act(M * K, mx.BF16, 37)).reshape(M, K)
    wb = torch.from_numpy(orc.dequant(Q4K, N, K, w)).to(torch.bfloat16).double().numpy()
    ref = (x.astype(np.float64) @ wb.T).astype(np.float32)
    np.testing.assert_allclose(orc.gemm_f64(Q4K, M, N, K, w, x, w_to_bf16=True), ref, rtol=1e-6, atol=1e-7)


def test_gemm_f16_weight_rounding():
    """w_to_f16 rounds the exact weights to fp16 (RNE), the operand of the fp16 MFMA path:
    numpy's float16 cast of the dequantized weights, then fp64."""
    M, N, K = 2, 8, 512
    for qt, seed in ((Q4K, 33), (Q80, 35)):
        w = mx.synth_gguf(qt, N, K, seed)
        x = orc.f16_bits_to_f32(mx.synth_act(M * K, mx.F16, 39)).reshape(M, K)
        wh = orc.dequant(qt, N, K, w).astype(np.float16).astype(np.float64)
        ref = (x.astype(np.float64) @ wh.T).astype(np.float32)
        np.testing.assert_allclose(orc.gemm_f64(qt, M, N, K, w, x, w_to_f16=True), ref, rtol=1e-6, atol=1e-7)
        # and it is not the bf16 rounding
        assert not np.array_equal(orc.gemm_f64(qt, M, N, K, w, x, w_to_f16=True),
                                  orc.gemm_f64(qt, M, N, K, w, x, w_to_bf16=True))


def test_elementwise_rel_err_known_answers():
    ref = np.array([100.0, -50.0, 0.5, 0.0, 1e-3])
    # 0.5, 0.0 and 1e-3 are below 1e-2 * 100 and do not count, however wrong
    y = np.array([101.0, -50.0, 9.0, 7.0, 5.0])
    assert orc.elementwise_rel_err(y, ref) == pytest.approx(0.01)
    y = np.array([100.0, -49.0, 0.5, 0.0, 1e-3])
    assert orc.elementwise_rel_err(y, ref) == pytest.approx(0.02)
    assert orc.elementwise_rel_err(ref, ref) == 0.0
    assert orc.elementwise_rel_err(np.ones(3), np.zeros(3)) == 0.0
    # the floor is relative to the largest |ref|: 2 qualifies at floor 1e-2 of 100
    assert orc.elementwise_rel_err(np.array([100.0, 3.0]), np.array([100.0, 2.0])) == pytest.approx(0.5)
    assert orc.rel_err(np.array([100.0, 3.0]), np.array([100.0, 2.0])) == pytest.approx(0.5)
    assert orc.rel_err(np.array([101.0, 2.0]), np.array([100.0, 2.0])) == pytest.approx(0.01)


def test_gemm_linearity():
    M, N, K = 3, 16, 512
    w = mx.synth_gguf(Q6K, N, K, 41)
    rng = np.random.default_rng(43)
    x1, x2 = rng.standard_normal((2, M, K)).astype(np.float32)
    y = orc.gemm_f64(Q6K, M, N, K, w, x1 + x2)
    y12 = orc.gemm_f64(Q6K, M, N, K, w, x1).astype(np.float64) + orc.gemm_f64(Q6K, M, N, K, w, x2)
    assert orc.normwise_rel_err(y, y12) < 1e-6


def test_unsupported_types_rejected():
    assert orc.lib().orc_dequant(8, 1, 256, None, None) == -1  # Q2_K has no oracle here
    assert orc.lib().orc_dequant(Q4K, 1, 300, None, None) == -1  # K not a block multiple
