// Register dequantization of packed weights into MFMA operand words, shared by the MFMA
// GEMM (qgemm_tile_kernel.h) and the dequant entry point (qgemm_pack.hip), so the values the
// GEMM multiplies are exactly the ones mlxr_qgemm_dequant returns.
//
// A "word" is 8 consecutive weights of a 32-weight sub-block (word kk = weights 8kk ..
// 8kk+7) as four packed pairs of the MFMA element type (bf16, or fp16 for fp16
// activations).  Each value is the exact GGUF fp32 weight, rounded to nearest even:
//   Q4_K  fma(d*sc, q, -(dmin*m))       (d*sc, q*d*sc and dmin*m exact; one rounding)
//   Q5_K  as Q4_K with q in 0..31
//   Q6_K  (d*sc) * (q - 32)             (exact; q - 32 formed exactly in fp32)
//   Q8_0  d * q                         (exact)
//   Q4_0  (q - 8) * d                   (exact)
//   Q4_1  fma(q, d, m)                  (q*d exact; one rounding)
// (the products keep the sign of zero of the GGUF formulas, which an fma with an
// offset term would not: fma(a, 32, -32a) is +0 for negative a).  The GEMM kernels take
// the MM variant: for Q6_K, Q8_0 and Q4_0 it forms the same values with one fma
// (fma(a, q, -c*a) rounds a*q - c*a, which is exactly a*(q - c), once), one operation per
// weight fewer; only an exact zero may differ in sign, which no product sum can see.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;

enum XType : int { X_BF16 = 0, X_F16 = 1 };

// Two floats -> packed pair of the MFMA element type, round to nearest even.
template <int XT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (XT == X_BF16) {
    return pack_bf16x2(lo, hi);
  } else {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
}

// An empty asm that makes later uses of v depend on this point in the program (used to
// order work against explicit waits and inside the MFMA stream).
template <typename T>
__device__ __forceinline__ void pin(T& v) {
  asm volatile("" : "+v"(v));
}

template <int QT>
struct Raw;
template <>
struct Raw<QT_Q4_K> {
  u32x4_t q;
  __device__ void pin_all() { pin(q); }
};
template <>
struct Raw<QT_Q6_K> {
  u32x4_t ql;
  u32x2_t qh;
  __device__ void pin_all() {
    pin(ql);
    pin(qh);
  }
};
template <>
struct Raw<QT_Q8_0> {
  u32x4_t a, b;
  uint32_t d;
  __device__ void pin_all() {
    pin(a);
    pin(b);
    pin(d);
  }
};

// Q5_K: the Q4_K nibbles plus the sub-block's fifth bits (q5h_bit order).
template <>
struct Raw<QT_Q5_K> {
  u32x4_t q;
  uint32_t qh;
  __device__ void pin_all() {
    pin(q);
    pin(qh);
  }
};

// Q4_0 / Q4_1: one 32-weight block (4 pair-interleaved words) and its scale word
// (fp16 d, plus fp16 m in the high half for Q4_1).
template <>
struct Raw<QT_Q4_0> {
  u32x4_t q;
  uint32_t d;
  __device__ void pin_all() {
    pin(q);
    pin(d);
  }
};
template <>
struct Raw<QT_Q4_1> {
  u32x4_t q;
  uint32_t d;
  __device__ void pin_all() {
    pin(q);
    pin(d);
  }
};

// Header bytes of one super-block as loaded; decoded once per four steps.
template <int QT>
struct Hdr {
  u32x4_t h;   // Q4_K: 8 x u16 lane-sliced entries; Q6_K: 16 int8 scales
  uint32_t d;  // Q6_K: fp16 d
  __device__ void pin_all() {
    pin(h);
    if constexpr (QT == QT_Q6_K) pin(d);
  }
};
// Decoded per-sub-block factors for the four sub-blocks (h, h+2, h+4, h+6) a lane owns
// in the current super-block.
template <int QT>
struct Scales {
  float a[4], b[4];  // Q4_K: d*sc, -(dmin*m).  Q6_K: d*sc of the two 16-weight groups.
};

template <int QT>
__device__ __forceinline__ void decode_hdr(const Hdr<QT>& h, int half, Scales<QT>& s) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    const uint32_t dd = q4k_dd(make_uint4(h.h[0], h.h[1], h.h[2], h.h[3]));
    const float d = f16_bits_to_f32(dd & 0xffffu), dmin = f16_bits_to_f32(dd >> 16);
    const uint32_t w[4] = {h.h[0], h.h[1], h.h[2], h.h[3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // entry j = 2q + half sits in word q, half `half`
      const uint32_t f = (half ? (w[q] >> 16) : w[q]) & 0xfffu;
      s.a[q] = d * (float)(f & 63u);
      s.b[q] = -(dmin * (float)(f >> 6));
    }
  } else if constexpr (QT == QT_Q6_K) {
    const float d = f16_bits_to_f32(h.d & 0xffffu);
    const uint32_t w[4] = {h.h[0], h.h[1], h.h[2], h.h[3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // sub-block j = 2q + half uses scales 2j, 2j + 1: bytes 4q + 2half, +1 = word q
      const uint32_t v = half ? (w[q] >> 16) : w[q];
      s.a[q] = d * (float)(int8_t)(v & 0xffu);
      s.b[q] = d * (float)(int8_t)((v >> 8) & 0xffu);
    }
  }
}

// Word kk of a sub-block is computed as a prelude and four quarter tasks (one packed
// pair each: weights (0,1), (2,3), (4,5), (6,7) of the word), so the GEMM can spread the
// work one task per MFMA.  q selects the sub-block's scales (sub-block 2q + half of the
// super-block, see decode_hdr).
template <int QT>
struct WordTmp {
  uint32_t u0, u1;
  float a, c;
};

template <int QT, int kk, bool MM = false>
__device__ __forceinline__ void word_prelude(const Raw<QT>& r, const Scales<QT>& s, int q, uint32_t nib,
                                             WordTmp<QT>& t) {
  if constexpr (QT == QT_Q4_K) {
    uint32_t w = r.q[kk];
    pin(w);
    t.u0 = w & nib;
    t.u1 = (w >> 4) & nib;
    t.a = s.a[q];
    t.c = s.b[q];
  } else if constexpr (QT == QT_Q5_K) {
    // the fifth bits of word kk's nibble bytes sit at bits 2kk (+1 for u1) + 8b of qh
    uint32_t w = r.q[kk], hb = r.qh;
    pin(w);
    pin(hb);
    constexpr int sh = 2 * kk - 4;  // moves bit 2kk + 8b to bit 4 + 8b
    const uint32_t h0 = sh >= 0 ? (hb >> sh) : (hb << (-sh));
    const uint32_t h1 = sh + 1 >= 0 ? (hb >> (sh + 1)) : (hb << (-(sh + 1)));
    t.u0 = (w & nib) | (h0 & 0x10101010u);
    t.u1 = ((w >> 4) & nib) | (h1 & 0x10101010u);
    t.a = s.a[q];
    t.c = s.b[q];
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    uint32_t w = r.q[kk];
    pin(w);
    t.u0 = w & nib;
    t.u1 = (w >> 4) & nib;
    t.a = f16_bits_to_f32(r.d & 0xffffu);
    t.c = QT == QT_Q4_0 ? (MM ? -8.f * t.a : 8.f) : f16_bits_to_f32(r.d >> 16);
  } else if constexpr (QT == QT_Q6_K) {
    // the six-bit values of the word in the Q4_K byte order (u0: weights 0, 4, 1, 5; u1:
    // 2, 6, 3, 7): low nibbles from ql, then the two high bits from qh, where after the
    // shift by 8(kk & 1) weight 2s has its bits at 2s and weight 2s+1 at 16 + 2s
    uint32_t lw = r.ql[kk], hv = r.qh[kk >> 1];
    pin(lw);
    pin(hv);
    const uint32_t x = (kk & 1) ? (hv >> 8) : hv;
    t.u0 = (lw & nib) | ((x << 4) & 0x00300030u) | ((x << 8) & 0x30003000u);
    t.u1 = ((lw >> 4) & nib) | ((x << 2) & 0x00300030u) | ((x << 6) & 0x30003000u);
    t.a = (kk < 2) ? s.a[q] : s.b[q];
    t.c = MM ? -32.f * t.a : 32.f;
  } else {
    uint32_t w0 = kk < 2 ? r.a[2 * kk] : r.b[2 * kk - 4];
    uint32_t w1 = kk < 2 ? r.a[2 * kk + 1] : r.b[2 * kk - 3];
    pin(w0);
    pin(w1);
    t.u0 = w0 ^ 0x80808080u;
    t.u1 = w1 ^ 0x80808080u;
    t.a = f16_bits_to_f32(r.d & 0xffffu);
    t.c = MM ? -128.f * t.a : 128.f;
  }
}

template <int QT, int XT, int kk, int qq, bool MM = false>
__device__ __forceinline__ uint32_t word_quarter(const WordTmp<QT>& t, uint32_t nib) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K || QT == QT_Q4_1) {
    // u0 bytes: weights 0, 4, 1, 5; u1 bytes: 2, 6, 3, 7
    const uint32_t v = (qq & 1) ? t.u1 : t.u0;
    const int sh = (qq & 2) ? 8 : 0;
    return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                     __builtin_fmaf(t.a, (float)((v >> (16 + sh)) & 0xffu), t.c));
  } else if constexpr (QT == QT_Q4_0) {
    const uint32_t v = (qq & 1) ? t.u1 : t.u0;
    const int sh = (qq & 2) ? 8 : 0;
    if constexpr (MM)
      return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                       __builtin_fmaf(t.a, (float)((v >> (16 + sh)) & 0xffu), t.c));
    return pack2<XT>(((float)((v >> sh) & 0xffu) - t.c) * t.a, ((float)((v >> (16 + sh)) & 0xffu) - t.c) * t.a);
  } else if constexpr (QT == QT_Q6_K) {
    // bytes as Q4_K's (see word_prelude)
    const uint32_t v = (qq & 1) ? t.u1 : t.u0;
    const int sh = (qq & 2) ? 8 : 0;
    if constexpr (MM)
      return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                       __builtin_fmaf(t.a, (float)((v >> (16 + sh)) & 0xffu), t.c));
    return pack2<XT>(t.a * ((float)((v >> sh) & 0xffu) - t.c), t.a * ((float)((v >> (16 + sh)) & 0xffu) - t.c));
  } else {
    // bytes hold q + 128 (sign bits flipped in the prelude)
    const uint32_t v = (qq < 2) ? t.u0 : t.u1;
    const int sh = (qq & 1) ? 16 : 0;
    if constexpr (MM)
      return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                       __builtin_fmaf(t.a, (float)((v >> (sh + 8)) & 0xffu), t.c));
    return pack2<XT>(((float)((v >> sh) & 0xffu) - t.c) * t.a, ((float)((v >> (sh + 8)) & 0xffu) - t.c) * t.a);
  }
}

// The whole word (dequant entry point; MM: GEMM kernels).
template <int QT, int XT, int kk, bool MM = false>
__device__ __forceinline__ uint4 dequant_word(const Raw<QT>& r, const Scales<QT>& s, int q, uint32_t nib) {
  WordTmp<QT> t;
  word_prelude<QT, kk, MM>(r, s, q, nib, t);
  return make_uint4(word_quarter<QT, XT, kk, 0, MM>(t, nib), word_quarter<QT, XT, kk, 1, MM>(t, nib),
                    word_quarter<QT, XT, kk, 2, MM>(t, nib), word_quarter<QT, XT, kk, 3, MM>(t, nib));
}

// Plain (compiler-visible) loads of sub-block sb of row n and of its super-block header,
// for the dequant entry point.
template <int QT>
__device__ __forceinline__ void load_sub_plain(const PlanePtrs& P, int K, int n, int sb, Raw<QT>& r, Hdr<QT>& h) {
  const size_t nsub = (size_t)(K >> 5), nsb = (size_t)(K >> 8);
  const size_t s = (size_t)n * nsub + (size_t)sb;
  const size_t g = (size_t)n * nsb + (size_t)(sb >> 3);
  if constexpr (QT == QT_Q4_K) {
    r.q = *(const u32x4_t*)(P.p[0] + s * 16);
    h.h = *(const u32x4_t*)(P.p[1] + g * 16);
  } else if constexpr (QT == QT_Q5_K) {
    r.q = *(const u32x4_t*)(P.p[0] + s * 16);
    r.qh = *(const uint32_t*)(P.p[1] + s * 4);
    h.h = *(const u32x4_t*)(P.p[2] + g * 16);
  } else if constexpr (QT == QT_Q4_0) {
    r.q = *(const u32x4_t*)(P.p[0] + s * 16);
    r.d = *(const uint16_t*)(P.p[1] + s * 2);
  } else if constexpr (QT == QT_Q4_1) {
    r.q = *(const u32x4_t*)(P.p[0] + s * 16);
    r.d = *(const uint32_t*)(P.p[1] + s * 4);
  } else if constexpr (QT == QT_Q6_K) {
    r.ql = *(const u32x4_t*)(P.p[0] + s * 16);
    r.qh = *(const u32x2_t*)(P.p[1] + s * 8);
    h.h = *(const u32x4_t*)(P.p[2] + g * 16);
    h.d = *(const uint16_t*)(P.p[3] + g * 2);
  } else {
    r.a = *(const u32x4_t*)(P.p[0] + s * 32);
    r.b = *(const u32x4_t*)(P.p[0] + s * 32 + 16);
    r.d = *(const uint16_t*)(P.p[1] + s * 2);
  }
}

// The 32 weights of sub-block sb of row n as four words of element type XT.
template <int QT, int XT>
__device__ __forceinline__ void dequant_sub_words(const PlanePtrs& P, int K, int n, int sb, uint32_t nib, uint4* out) {
  Raw<QT> r;
  Hdr<QT> h;
  load_sub_plain<QT>(P, K, n, sb, r, h);
  Scales<QT> sc;
  decode_hdr<QT>(h, sb & 1, sc);
  const int q = (sb & 7) >> 1;
  out[0] = dequant_word<QT, XT, 0>(r, sc, q, nib);
  out[1] = dequant_word<QT, XT, 1>(r, sc, q, nib);
  out[2] = dequant_word<QT, XT, 2>(r, sc, q, nib);
  out[3] = dequant_word<QT, XT, 3>(r, sc, q, nib);
}

}  // namespace mlxr
