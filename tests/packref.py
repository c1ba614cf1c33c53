"""numpy statement of the packed HBM layout (test helper).

Builds, from GGUF block bytes, the exact bytes the library's pack kernels must produce,
following the layout description in mlxr_amd/csrc/qgemm_layout.h.  Independent of the
HIP pack kernels, so a GPU test can compare them byte for byte.
"""
import numpy as np


def _align256(v):
    return (v + 255) & ~255


def pi_shift(e):
    return 4 * ((e >> 1) + 4 * (e & 1))


def q5h_bit(e):
    return 2 * (e >> 3) + ((e >> 1) & 1) + 8 * (((e >> 2) & 1) + 2 * (e & 1))


def q6h_shift(e):
    return 2 * ((e & 7) >> 1) + 16 * (e & 1) + 8 * ((e >> 3) & 1)


def _words_from_nibbles(nib):
    """nib [..., 32] values 0..15 -> [..., 4] uint32 pair-interleaved words."""
    nib = nib.astype(np.uint32).reshape(nib.shape[:-1] + (4, 8))
    w = np.zeros(nib.shape[:-1], dtype=np.uint32)
    for i in range(8):
        w |= nib[..., i] << np.uint32(pi_shift(i))
    return w


def q4k_scale_min(s):
    """s [..., 12] uint8 -> (sc, m) [..., 8] (GGUF 6-bit packing)."""
    s = s.astype(np.uint32)
    sc = np.zeros(s.shape[:-1] + (8,), np.uint32)
    m = np.zeros_like(sc)
    for j in range(4):
        sc[..., j] = s[..., j] & 63
        m[..., j] = s[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
        m[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, m


def planes(qtype, N, K, gguf):
    g = np.asarray(gguf, dtype=np.uint8)
    if qtype == 3:  # Q4_K
        nsb = K // 256
        b = g.reshape(N, nsb, 144)
        sc, m = q4k_scale_min(b[..., 4:16])
        dd = (b[..., 0].astype(np.uint32) | (b[..., 1].astype(np.uint32) << 8)
              | (b[..., 2].astype(np.uint32) << 16) | (b[..., 3].astype(np.uint32) << 24))
        hdr = np.zeros((N, nsb, 8), np.uint16)
        for j in range(8):
            hdr[..., j] = (sc[..., j] | (m[..., j] << 6) | (((dd >> np.uint32(4 * j)) & 15) << 12)).astype(np.uint16)
        hdr = hdr.view(np.uint8).reshape(N, nsb, 16)
        qs = b[..., 16:144].reshape(N, nsb, 4, 32)
        nib = np.stack([qs & 15, qs >> 4], axis=3).reshape(N, nsb, 8, 32)  # sub-block 2c, 2c+1
        words = _words_from_nibbles(nib)  # [N, nsb, 8, 4]
        return [words.view(np.uint8).reshape(-1), hdr.reshape(-1)]
    if qtype == 10:  # Q5_K: Q4_K header and nibbles, fifth bits in q5h_bit order
        nsb = K // 256
        b = g.reshape(N, nsb, 176)
        sc, m = q4k_scale_min(b[..., 4:16])
        dd = (b[..., 0].astype(np.uint32) | (b[..., 1].astype(np.uint32) << 8)
              | (b[..., 2].astype(np.uint32) << 16) | (b[..., 3].astype(np.uint32) << 24))
        hdr = np.zeros((N, nsb, 8), np.uint16)
        for j in range(8):
            hdr[..., j] = (sc[..., j] | (m[..., j] << 6) | (((dd >> np.uint32(4 * j)) & 15) << 12)).astype(np.uint16)
        qh = b[..., 16:48].astype(np.uint32)          # [N, nsb, 32]: bit j of byte l -> sub-block j, elem l
        qs = b[..., 48:176].reshape(N, nsb, 4, 32)
        nib = np.stack([qs & 15, qs >> 4], axis=3).reshape(N, nsb, 8, 32)
        words = _words_from_nibbles(nib)
        hw = np.zeros((N, nsb, 8), np.uint32)
        for j in range(8):
            for e in range(32):
                hw[..., j] |= ((qh[..., e] >> np.uint32(j)) & 1) << np.uint32(q5h_bit(e))
        return [words.view(np.uint8).reshape(-1), hw.view(np.uint8).reshape(-1), hdr.view(np.uint8).reshape(-1)]
    if qtype == 4:  # Q6_K
        nsb = K // 256
        b = g.reshape(N, nsb, 210)
        ql, qh = b[..., 0:128], b[..., 128:192]
        lo = np.zeros((N, nsb, 256), np.uint8)
        hi = np.zeros((N, nsb, 256), np.uint8)
        for h in range(2):
            for r in range(64):  # ql byte 64h+r: low nibble -> 128h+r, high -> 128h+r+64
                lo[..., 128 * h + r] = ql[..., 64 * h + r] & 15
                lo[..., 128 * h + r + 64] = ql[..., 64 * h + r] >> 4
            for l in range(32):  # qh byte 32h+l: bits 2t..2t+1 -> 128h+32t+l
                for t in range(4):
                    hi[..., 128 * h + 32 * t + l] = (qh[..., 32 * h + l] >> (2 * t)) & 3
        lw = _words_from_nibbles(lo.reshape(N, nsb, 8, 32))
        hw = np.zeros((N, nsb, 8, 2), np.uint32)
        hs = hi.reshape(N, nsb, 8, 32).astype(np.uint32)
        for e in range(32):
            hw[..., e >> 4] |= hs[..., e] << np.uint32(q6h_shift(e))
        return [lw.view(np.uint8).reshape(-1), hw.view(np.uint8).reshape(-1),
                b[..., 192:208].reshape(-1).copy(), b[..., 208:210].reshape(-1).copy()]
    if qtype in (0, 1):  # Q4_0 / Q4_1: byte j holds elements j (low) and j + 16 (high)
        nb = K // 32
        hb = 2 if qtype == 0 else 4
        b = g.reshape(N, nb, hb + 16)
        qs = b[..., hb:]
        nib = np.concatenate([qs & 15, qs >> 4], axis=-1).reshape(N, nb, 1, 32)
        words = _words_from_nibbles(nib)  # [N, nb, 1, 4]
        return [words.view(np.uint8).reshape(-1), b[..., 0:hb].reshape(-1).copy()]
    if qtype == 2:  # Q8_0
        nb = K // 32
        b = g.reshape(N, nb, 34)
        return [b[..., 2:34].reshape(-1).copy(), b[..., 0:2].reshape(-1).copy()]
    raise ValueError(qtype)


def pack(qtype, N, K, gguf):
    ps = planes(qtype, N, K, gguf)
    total = 0
    offs = []
    for p in ps:
        offs.append(total)
        total = _align256(total + p.size)
    out = np.zeros(total, np.uint8)
    for o, p in zip(offs, ps):
        out[o:o + p.size] = p
    return out
