// Device helpers shared by the pack, dequant, GEMV and MFMA kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qgemm_layout.h"

namespace mlxr {

// Cache policy bits of buffer loads (the aux operand): 0 default, 2 non-temporal (nt).
constexpr int POL_DEFAULT = 0, POL_NT = 2;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;

// Element types (values of MLXR_F32 / MLXR_F16 / MLXR_BF16).
enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}
// Round-to-nearest-even conversions (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
// Two floats -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float load_scalar(const void* p, int dtype, size_t i) {
  if (dtype == DT_F32) return ((const float*)p)[i];
  if (dtype == DT_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
__device__ __forceinline__ void store_scalar(void* p, int dtype, size_t i, float v) {
  if (dtype == DT_F32) ((float*)p)[i] = v;
  else if (dtype == DT_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}

// Shift that brings the nibble of weight e (0..7) of a pair-interleaved word to bit 0.
__host__ __device__ constexpr int pi_shift(int e) { return 4 * ((e >> 1) + 4 * (e & 1)); }
// Bit of the 2-bit high field of weight e (0..31 in a Q6_K sub-block) in its qh word
// (word index e/16).
__host__ __device__ constexpr int q6h_shift(int e) {
  return 2 * ((e & 7) >> 1) + 16 * (e & 1) + 8 * ((e >> 3) & 1);
}

// Bit of the fifth bit of weight e (0..31 in a Q5_K sub-block) in its qh word.
__host__ __device__ constexpr int q5h_bit(int e) {
  return 2 * (e >> 3) + ((e >> 1) & 1) + 8 * (((e >> 2) & 1) + 2 * (e & 1));
}

// Q4_K lane-sliced header (8 x u16 per super-block): d | dmin << 16 from the high
// nibbles of all eight entries.
__device__ __forceinline__ uint32_t q4k_dd(const uint4& h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t dd = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) dd |= ((w[j >> 1] >> (16 * (j & 1) + 12)) & 15u) << (4 * j);
  return dd;
}

// Raw packed bytes of one 32-weight sub-block (what a loader prefetches).
template <int QT>
struct RawSub;
template <>
struct RawSub<QT_Q4_K> {
  uint4 q;  // 4 pair-interleaved words
  uint4 h;  // the super-block's 8 x u16 lane-sliced header
};
template <>
struct RawSub<QT_Q6_K> {
  uint4 ql;
  uint2 qh;
  uint32_t sc;  // two int8 scales (groups 2j, 2j+1) in the low 16 bits
  uint32_t d;   // fp16 bits
};
template <>
struct RawSub<QT_Q8_0> {
  uint4 a, b;
  uint32_t d;
};

template <>
struct RawSub<QT_Q5_K> {
  uint4 q;      // low nibbles, as Q4_K
  uint32_t qh;  // fifth bits (q5h_bit order)
  uint4 h;      // the super-block's lane-sliced header, as Q4_K
};
template <>
struct RawSub<QT_Q4_0> {
  uint4 q;     // 4 pair-interleaved words
  uint32_t d;  // fp16 bits
};
template <>
struct RawSub<QT_Q4_1> {
  uint4 q;
  uint32_t d;  // fp16 d | fp16 m << 16
};

template <int QT>
__device__ __forceinline__ void load_raw_sub(const uint8_t* const* planes, int K, int n, int sb, RawSub<QT>& r) {
  const size_t nsub = (size_t)(K / 32);
  if constexpr (QT == QT_Q4_K) {
    const size_t nsb = (size_t)(K / 256);
    r.q = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    r.h = *(const uint4*)(planes[1] + ((size_t)n * nsb + (sb >> 3)) * 16);
  } else if constexpr (QT == QT_Q5_K) {
    const size_t nsb = (size_t)(K / 256);
    r.q = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    r.qh = *(const uint32_t*)(planes[1] + ((size_t)n * nsub + sb) * 4);
    r.h = *(const uint4*)(planes[2] + ((size_t)n * nsb + (sb >> 3)) * 16);
  } else if constexpr (QT == QT_Q6_K) {
    const size_t nsb = (size_t)(K / 256);
    r.ql = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    r.qh = *(const uint2*)(planes[1] + ((size_t)n * nsub + sb) * 8);
    r.sc = *(const uint16_t*)(planes[2] + ((size_t)n * nsb + (sb >> 3)) * 16 + 2 * (sb & 7));
    r.d = *(const uint16_t*)(planes[3] + ((size_t)n * nsb + (sb >> 3)) * 2);
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {  // block index == sub-block index
    r.q = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    if constexpr (QT == QT_Q4_0) r.d = *(const uint16_t*)(planes[1] + ((size_t)n * nsub + sb) * 2);
    else r.d = *(const uint32_t*)(planes[1] + ((size_t)n * nsub + sb) * 4);
  } else {  // Q8_0: block index == sub-block index
    const uint8_t* qs = planes[0] + ((size_t)n * nsub + sb) * 32;
    r.a = *(const uint4*)qs;
    r.b = *(const uint4*)(qs + 16);
    r.d = *(const uint16_t*)(planes[1] + ((size_t)n * nsub + sb) * 2);
  }
}

// fp32 weights of one sub-block, exactly as the GGUF formulas define (every product
// below is exact in fp32; Q4_K rounds once, in the fma).  j = sub-block index within its
// super-block (sb % 8).
template <int QT>
__device__ __forceinline__ void dequant_raw(const RawSub<QT>& r, int j, float* w) {
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    const uint32_t dd = q4k_dd(r.h);
    const uint32_t hw[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
    const uint32_t f = (hw[j >> 1] >> (16 * (j & 1))) & 0xfffu;
    const float dsc = f16_bits_to_f32(dd & 0xffffu) * (float)(f & 63u);
    const float dm = f16_bits_to_f32(dd >> 16) * (float)(f >> 6);
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      uint32_t v = (qw[e >> 3] >> pi_shift(e & 7)) & 15u;
      if constexpr (QT == QT_Q5_K) v |= ((r.qh >> q5h_bit(e)) & 1u) << 4;
      w[e] = __builtin_fmaf(dsc, (float)v, -dm);
    }
  } else if constexpr (QT == QT_Q6_K) {
    const float d = f16_bits_to_f32(r.d);
    const float ds0 = d * (float)(int8_t)(r.sc & 0xffu), ds1 = d * (float)(int8_t)((r.sc >> 8) & 0xffu);
    const uint32_t lw[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};
    const uint32_t hw[2] = {r.qh.x, r.qh.y};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t lo = (lw[e >> 3] >> pi_shift(e & 7)) & 15u;
      const uint32_t hi = (hw[e >> 4] >> q6h_shift(e)) & 3u;
      w[e] = (e < 16 ? ds0 : ds1) * (float)((int)(lo | (hi << 4)) - 32);
    }
  } else if constexpr (QT == QT_Q4_0 || QT == QT_Q4_1) {
    const float d = f16_bits_to_f32(r.d & 0xffffu);
    const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t v = (qw[e >> 3] >> pi_shift(e & 7)) & 15u;
      if constexpr (QT == QT_Q4_0) w[e] = (float)((int)v - 8) * d;
      else w[e] = __builtin_fmaf((float)v, d, f16_bits_to_f32(r.d >> 16));
    }
  } else {
    const float d = f16_bits_to_f32(r.d);
    const uint32_t qw[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int v = (int)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xffu);
      w[e] = (float)v * d;
    }
  }
}

// (v & mask) | bits in one VALU op; the compiler otherwise emits an and plus an or.
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(bits));
  return r;
}

// swish(g) * u = g / (1 + exp(-g)) * u in fp32: the gating of the SwiGLU MLP
// (reference core/graph/layers.cpp:391-414).  The quotient uses the hardware reciprocal
// (v_rcp_f32, 1 ulp) instead of the IEEE division sequence, which is about ten
// instructions and made the tiled GEMM's fused epilogue 8 k clocks per tile longer.
__device__ __forceinline__ float swiglu1(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)) * u;
}

}  // namespace mlxr
