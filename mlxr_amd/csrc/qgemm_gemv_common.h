// Device building blocks of the no-MFMA GEMV kernels (qgemm_gemv.hip, qgemm_mlp.hip):
// weight-chunk loads from the packed planes, decoding into bf16/fp16 magic pairs, the
// per-sub-block contribution with the folded offset/min correction, and wavefront sums.
// Everything sits in an anonymous namespace: each kernel file instantiates its own copy.
#pragma once
#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {
namespace {

enum XType : int { X_BF16 = 0, X_F16 = 1 };

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;


template <int XT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (XT == X_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c,
                                  false);
}

// sum over pairs [i0, i1) of dot2(x[i], w[i]); two chains for ILP.
template <int XT, int I0, int I1>
__device__ __forceinline__ float dot_range(const uint32_t* x, const uint32_t* w) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = I0; i < I1; i += 2) {
    s0 = dot2<XT>(x[i], w[i], s0);
    if (i + 1 < I1) s1 = dot2<XT>(x[i + 1], w[i + 1], s1);
  }
  return s0 + s1;
}
template <int XT, int I0, int I1>
__device__ __forceinline__ float sum_range(const uint32_t* x) {
  constexpr uint32_t ONE = (XT == X_BF16) ? 0x3F803F80u : 0x3C003C00u;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = I0; i < I1; i += 2) {
    s0 = dot2<XT>(x[i], ONE, s0);
    if (i + 1 < I1) s1 = dot2<XT>(x[i + 1], ONE, s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ float dpp_row_sum(float v) {
  // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror 4, row_ror 8: every lane of a
  // 16-lane row ends with the row's total.
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_row_sum(v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (a + b) + (c + d);
}

// Sum over the 64 lanes: DPP adds within rows of 16 (quad swaps, half-row and row
// mirrors), then row_bcast:15 / row_bcast:31 carry the row totals upward so lane 63 holds
// the wavefront total; returned as a uniform value.
__device__ __forceinline__ float wave_total(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *(const uint4*)p; }

// Weights of one row and one sub-block, as loaded from HBM.
template <int QT>
struct WLoad;
template <>
struct WLoad<QT_Q4_K> {
  uint4 q;
  uint32_t h;  // this lane's u16 of the lane-sliced header
};
template <>
struct WLoad<QT_Q6_K> {
  uint4 ql;
  uint2 qh;
  uint32_t sc;  // two int8 scales in the low 16 bits
  uint32_t d;   // fp16 bits
};
template <>
struct WLoad<QT_Q8_0> {
  uint4 a, b;
  uint32_t d;
};
template <>
struct WLoad<QT_Q5_K> {
  uint4 q;
  uint32_t qh;  // fifth bits
  uint32_t h;   // this lane's u16 of the lane-sliced header
};
template <>
struct WLoad<QT_Q4_0> {
  uint4 q;
  uint32_t d;  // fp16 bits
};
template <>
struct WLoad<QT_Q4_1> {
  uint4 q;
  uint32_t d;  // fp16 d | fp16 m << 16
};

template <bool NT>
__device__ __forceinline__ uint4 ldw16(const uint8_t* p) {
  typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v[0], v[1], v[2], v[3]);
  } else {
    return *(const uint4*)p;
  }
}

template <int QT, bool NT = false>
__device__ __forceinline__ void load_w(const PlanePtrs& P, int K, int n, int sb, WLoad<QT>& w) {
  const size_t nsub = (size_t)(K >> 5);
  if constexpr (QT == QT_Q4_K) {
    const size_t nsb = (size_t)(K >> 8);
    w.q = ldw16<NT>(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.h = *(const uint16_t*)(P.p[1] + ((size_t)n * nsb + (sb >> 3)) * 16 + 2 * (sb & 7));
  } else if constexpr (QT == QT_Q6_K) {
    const size_t nsb = (size_t)(K >> 8);
    w.ql = ldw16<NT>(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.qh = *(const uint2*)(P.p[1] + ((size_t)n * nsub + sb) * 8);
    w.sc = *(const uint16_t*)(P.p[2] + ((size_t)n * nsb + (sb >> 3)) * 16 + 2 * (sb & 7));
    w.d = *(const uint16_t*)(P.p[3] + ((size_t)n * nsb + (sb >> 3)) * 2);
  } else if constexpr (QT == QT_Q5_K) {
    const size_t nsb = (size_t)(K >> 8);
    w.q = ldw16<NT>(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.qh = *(const uint32_t*)(P.p[1] + ((size_t)n * nsub + sb) * 4);
    w.h = *(const uint16_t*)(P.p[2] + ((size_t)n * nsb + (sb >> 3)) * 16 + 2 * (sb & 7));
  } else if constexpr (QT == QT_Q4_0) {
    w.q = ldw16<NT>(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.d = *(const uint16_t*)(P.p[1] + ((size_t)n * nsub + sb) * 2);
  } else if constexpr (QT == QT_Q4_1) {
    w.q = ldw16<NT>(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.d = *(const uint32_t*)(P.p[1] + ((size_t)n * nsub + sb) * 4);
  } else {
    const uint8_t* q = P.p[0] + ((size_t)n * nsub + sb) * 32;
    w.a = ldw16<NT>(q);
    w.b = ldw16<NT>(q + 16);
    w.d = *(const uint16_t*)(P.p[1] + ((size_t)n * nsub + sb) * 2);
  }
}
template <int QT>
__device__ __forceinline__ void zero_w(WLoad<QT>& w) {
  if constexpr (QT == QT_Q4_K) {
    w.q = make_uint4(0, 0, 0, 0);
    w.h = 0;
  } else if constexpr (QT == QT_Q6_K) {
    w.ql = make_uint4(0, 0, 0, 0);
    w.qh = make_uint2(0, 0);
    w.sc = 0;
    w.d = 0;
  } else if constexpr (QT == QT_Q5_K) {
    w.q = make_uint4(0, 0, 0, 0);
    w.qh = 0;
    w.h = 0;
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    w.q = make_uint4(0, 0, 0, 0);
    w.d = 0;
  } else {
    w.a = make_uint4(0, 0, 0, 0);
    w.b = make_uint4(0, 0, 0, 0);
    w.d = 0;
  }
}

// Decoded weights of one row/sub-block: 16 magic pairs + scale factors.
struct WDec {
  uint32_t p[16];
  float s0, s1;  // Q4_K: d*sc, dmin*m.  Q6_K: d*sc(group 0), d*sc(group 1).  Q8_0: d, -
                 // Q4_0: d, 8d.  Q4_1: d, -m  (so Q4_0/Q4_1/Q4_K share one contribution)
};

// Fifth bits of pair s of word t of a Q5_K sub-block, at bits 4 and 20 (q5h_bit order).
__device__ __forceinline__ uint32_t q5_pair_bits(uint32_t qh, int t, int s) {
  const int r = 2 * t + (s & 1) + 8 * (s >> 1) - 4;
  return (r >= 0 ? (qh >> r) : (qh << (-r))) & 0x00100010u;
}

template <int QT, int XT>
__device__ __forceinline__ void decode_w(const WLoad<QT>& w, int j, WDec& o) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    constexpr uint32_t MAGIC = (XT == X_BF16) ? 0x43004300u : 0x64006400u;
    const uint32_t qw[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        o.p[4 * t + s] = ((qw[t] >> (4 * s)) & 0x000F000Fu) | MAGIC;
        if constexpr (QT == QT_Q5_K) o.p[4 * t + s] |= q5_pair_bits(w.qh, t, s);
      }
    // d | dmin << 16: nibble j of it sits in bits 12..15 of lane j's entry; OR the eight
    // lanes of the super-block together (xor 1, xor 2 within quads, then mirror within 8).
    uint32_t dd = (w.h >> 12) << (4 * j);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0xB1, 0xF, 0xF, false);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0x4E, 0xF, 0xF, false);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0x141, 0xF, 0xF, false);
    o.s0 = f16_bits_to_f32(dd & 0xffffu) * (float)(w.h & 63u);
    o.s1 = f16_bits_to_f32(dd >> 16) * (float)((w.h >> 6) & 63u);
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    constexpr uint32_t MAGIC = (XT == X_BF16) ? 0x43004300u : 0x64006400u;
    const uint32_t qw[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) o.p[4 * t + s] = ((qw[t] >> (4 * s)) & 0x000F000Fu) | MAGIC;
    o.s0 = f16_bits_to_f32(w.d & 0xffffu);
    o.s1 = QT == QT_Q4_0 ? 8.f * o.s0 : -f16_bits_to_f32(w.d >> 16);
  } else if constexpr (QT == QT_Q6_K) {
    constexpr uint32_t MAGIC = (XT == X_BF16) ? 0x43004300u : 0x64006400u;
    const uint32_t lw[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t hv = (t & 2) ? w.qh.y : w.qh.x;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int rs = 8 * (t & 1) + 2 * s - 4;  // bring bits 2s(+16) of the t-half to 4(+20)
        const uint32_t hs = rs >= 0 ? (hv >> rs) : (hv << (-rs));
        o.p[4 * t + s] = ((lw[t] >> (4 * s)) & 0x000F000Fu) | (hs & 0x00300030u) | MAGIC;
      }
    }
    const float d = f16_bits_to_f32(w.d);
    o.s0 = d * (float)(int8_t)(w.sc & 0xffu);
    o.s1 = d * (float)(int8_t)((w.sc >> 8) & 0xffu);
  } else {
    const uint32_t qw[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
    if constexpr (XT == X_F16) {
      // int8 q -> u = q + 128 -> fp16 (1024 + u) via byte permute with 0x64 high bytes.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t u = qw[i] ^ 0x80808080u;
        o.p[2 * i + 0] = __builtin_amdgcn_perm(u, 0x64646464u, 0x00050004u);
        o.p[2 * i + 1] = __builtin_amdgcn_perm(u, 0x64646464u, 0x00070006u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o.p[i] = qw[i];  // raw int8, fp32 path below
    }
    o.s0 = f16_bits_to_f32(w.d);
    o.s1 = 0.f;
  }
}

// Contribution of one decoded row/sub-block against one activation sub-block.
template <int QT, int XT>
__device__ __forceinline__ float contrib(const uint32_t* xv, const WDec& w, float X0, float X1) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K || QT == QT_Q4_0 || QT == QT_Q4_1) {
    constexpr float OFF = (XT == X_BF16) ? 128.f : 1024.f;
    const float S = dot_range<XT, 0, 16>(xv, w.p);
    return w.s0 * (S - OFF * (X0 + X1)) - w.s1 * (X0 + X1);
  } else if constexpr (QT == QT_Q6_K) {
    constexpr float OFF = (XT == X_BF16) ? 160.f : 1056.f;  // magic + 32
    const float S0 = dot_range<XT, 0, 8>(xv, w.p);
    const float S1 = dot_range<XT, 8, 16>(xv, w.p);
    return w.s0 * (S0 - OFF * X0) + w.s1 * (S1 - OFF * X1);
  } else {
    if constexpr (XT == X_F16) {
      const float S = dot_range<XT, 0, 16>(xv, w.p);
      return w.s0 * (S - 1152.f * (X0 + X1));
    } else {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t q2 = w.p[j >> 1] >> (16 * (j & 1));
        const float q0 = (float)(int)(int8_t)(q2 & 0xffu);
        const float q1 = (float)(int)(int8_t)((q2 >> 8) & 0xffu);
        s0 = __builtin_fmaf(bf16_bits_to_f32(xv[j] & 0xffffu), q0, s0);
        s1 = __builtin_fmaf(bf16_bits_to_f32(xv[j] >> 16), q1, s1);
      }
      return w.s0 * (s0 + s1);
    }
  }
}


// Variant for M <= 4 (the decode shapes).  Each wavefront owns a contiguous run of rows
// and walks them as a flat sequence of (row, segment) chunks, D-1 chunks of loads in
// flight ahead of the one being reduced.  Weight loads are raw buffer loads whose row /
// segment offset is a scalar (SGPR) and whose lane offset is fixed, so a chunk costs no
// vector address arithmetic; lanes past the end of K get an offset beyond the buffer and
// read zeros.  The activations (and their per-sub-block sums) are staged once per
// workgroup in LDS as [m][segment][quarter][lane] so each chunk reads them with
// conflict-free 16-byte LDS loads at immediate offsets.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t OOB = 0x80000000u;  // voffset that is out of range of every buffer

__device__ __forceinline__ rsrc_t make_rsrc(const void* ptr, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)bytes, 0x00020000);
}

template <int QT>
struct CLoad;
// 16-bit fields stay 16-bit until decoded: widening them in the loop latch would make
// the compiler wait for the loads in flight.
template <>
struct CLoad<QT_Q4_K> {
  uint4 q;
  uint16_t h;
};
template <>
struct CLoad<QT_Q6_K> {
  uint4 ql;
  uint2 qh;
  uint16_t sc, d;
};
template <>
struct CLoad<QT_Q8_0> {
  uint4 a, b;
  uint16_t d;
};
template <>
struct CLoad<QT_Q5_K> {
  uint4 q;
  uint32_t qh;
  uint16_t h;
};
template <>
struct CLoad<QT_Q4_0> {
  uint4 q;
  uint16_t d;
};
template <>
struct CLoad<QT_Q4_1> {
  uint4 q;
  uint32_t d;
};


// One weight of a (possibly grouped) launch.  Weights in one launch share K, the quant
// type and the activations; each owns a contiguous range of wavefronts.
struct LdsGroup {
  PlanePtrs P;
  uint32_t psize[4];  // plane sizes in bytes (all < 2^31)
  void* y;
  const void* bias;
  int N, rows_per_wave, wave_start, y_dtype, bias_dtype;
};

constexpr int MAX_GROUPS = 4;

struct LdsParams {
  const void* x;
  int M, K, ngroups;
  uint32_t cmask, cmagic;  // 0x000F000F and the bf16/fp16 magic, passed at run time
  LdsGroup g[MAX_GROUPS];
};

template <int QT, int WPOL>
__device__ __forceinline__ void load_chunk(const rsrc_t* R, int row, int seg, int nsub, int nsb,
                                           int lane, bool ok, CLoad<QT>& b) {
  const uint32_t sbase = (uint32_t)row * (uint32_t)nsub + (uint32_t)seg * 64u;  // first sub-block
  const uint32_t gbase = (uint32_t)row * (uint32_t)nsb + (uint32_t)seg * 8u;    // first super-block
  if constexpr (QT == QT_Q4_K) {
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 16 : OOB, sbase * 16u, WPOL);
    b.q = make_uint4(q[0], q[1], q[2], q[3]);
    b.h = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? lane * 2 : OOB, gbase * 16u, WPOL);
  } else if constexpr (QT == QT_Q6_K) {
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 16 : OOB, sbase * 16u, WPOL);
    b.ql = make_uint4(q[0], q[1], q[2], q[3]);
    const u32x2_t h = __builtin_amdgcn_raw_buffer_load_b64(R[1], ok ? lane * 8 : OOB, sbase * 8u, WPOL);
    b.qh = make_uint2(h[0], h[1]);
    b.sc = __builtin_amdgcn_raw_buffer_load_b16(R[2], ok ? lane * 2 : OOB, gbase * 16u, WPOL);
    b.d = __builtin_amdgcn_raw_buffer_load_b16(R[3], ok ? (lane >> 3) * 2 : OOB, gbase * 2u, WPOL);
  } else if constexpr (QT == QT_Q5_K) {
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 16 : OOB, sbase * 16u, WPOL);
    b.q = make_uint4(q[0], q[1], q[2], q[3]);
    b.qh = __builtin_amdgcn_raw_buffer_load_b32(R[1], ok ? lane * 4 : OOB, sbase * 4u, WPOL);
    b.h = __builtin_amdgcn_raw_buffer_load_b16(R[2], ok ? lane * 2 : OOB, gbase * 16u, WPOL);
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 16 : OOB, sbase * 16u, WPOL);
    b.q = make_uint4(q[0], q[1], q[2], q[3]);
    if constexpr (QT == QT_Q4_0) b.d = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? lane * 2 : OOB, sbase * 2u, WPOL);
    else b.d = __builtin_amdgcn_raw_buffer_load_b32(R[1], ok ? lane * 4 : OOB, sbase * 4u, WPOL);
  } else {
    const u32x4_t q0 = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 32 : OOB, sbase * 32u, WPOL);
    const u32x4_t q1 = __builtin_amdgcn_raw_buffer_load_b128(R[0], ok ? lane * 32 + 16 : OOB, sbase * 32u, WPOL);
    b.a = make_uint4(q0[0], q0[1], q0[2], q0[3]);
    b.b = make_uint4(q1[0], q1[1], q1[2], q1[3]);
    b.d = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? lane * 2 : OOB, sbase * 2u, WPOL);
  }
}

template <int QT, int XT>
__device__ __forceinline__ void decode_chunk(const CLoad<QT>& b, int j, uint32_t MASK, uint32_t MAGIC, WDec& o) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    const uint32_t qw[4] = {b.q.x, b.q.y, b.q.z, b.q.w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if constexpr (QT == QT_Q5_K) o.p[4 * t + s] = and_or(qw[t] >> (4 * s), MASK, MAGIC | q5_pair_bits(b.qh, t, s));
        else o.p[4 * t + s] = and_or(qw[t] >> (4 * s), MASK, MAGIC);
      }
    // d | dmin << 16: nibble j of it sits in bits 12..15 of lane j's entry; OR the eight
    // lanes of the super-block together (xor 1, xor 2 within quads, then mirror within 8).
    const uint32_t hv = b.h;
    uint32_t dd = (hv >> 12) << (4 * j);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0xB1, 0xF, 0xF, false);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0x4E, 0xF, 0xF, false);
    dd |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)dd, 0x141, 0xF, 0xF, false);
    o.s0 = f16_bits_to_f32(dd & 0xffffu) * (float)(hv & 63u);
    o.s1 = f16_bits_to_f32(dd >> 16) * (float)((hv >> 6) & 63u);
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    const uint32_t qw[4] = {b.q.x, b.q.y, b.q.z, b.q.w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) o.p[4 * t + s] = and_or(qw[t] >> (4 * s), MASK, MAGIC);
    const uint32_t dv = b.d;
    o.s0 = f16_bits_to_f32(dv & 0xffffu);
    o.s1 = QT == QT_Q4_0 ? 8.f * o.s0 : -f16_bits_to_f32(dv >> 16);
  } else if constexpr (QT == QT_Q6_K) {
    WLoad<QT_Q6_K> w;
    w.ql = b.ql;
    w.qh = b.qh;
    w.sc = b.sc;
    w.d = b.d;
    decode_w<QT, XT>(w, j, o);
  } else {
    WLoad<QT_Q8_0> w;
    w.a = b.a;
    w.b = b.b;
    w.d = b.d;
    decode_w<QT, XT>(w, j, o);
  }
}


}  // namespace
}  // namespace mlxr
