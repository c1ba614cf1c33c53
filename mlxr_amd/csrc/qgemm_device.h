// Device helpers shared by the pack, dequant, GEMV and MFMA kernels (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qgemm_layout.h"

namespace mlxr {

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
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
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

// Q4_K lane-sliced header (8 x u16 per super-block): d | dmin << 16 from the high
// nibbles of all eight entries.
__device__ __forceinline__ uint32_t q4k_dd(const uint4& h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t dd = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) dd |= ((w[j >> 1] >> (16 * (j & 1) + 12)) & 15u) << (4 * j);
  return dd;
}

// Dequantize sub-block `sb` (32 weights along K) of row n to fp32, exactly as the GGUF
// formulas define (every product below is exact in fp32; Q4_K rounds once in the fma).
template <int QT>
__device__ __forceinline__ void dequant_sub_f32(const uint8_t* const* planes, int K, int n,
                                                int sb, float* w) {
  const size_t nsub = (size_t)(K / 32);
  if constexpr (QT == QT_Q4_K) {
    const size_t nsb = (size_t)(K / 256);
    const uint4 q = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    const uint4 h = *(const uint4*)(planes[1] + ((size_t)n * nsb + (sb >> 3)) * 16);
    const uint32_t dd = q4k_dd(h);
    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
    const uint32_t f = (hw[(sb & 7) >> 1] >> (16 * (sb & 1))) & 0xfffu;
    const float dsc = f16_bits_to_f32(dd & 0xffffu) * (float)(f & 63u);
    const float dm = f16_bits_to_f32(dd >> 16) * (float)(f >> 6);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t v = (qw[e >> 3] >> pi_shift(e & 7)) & 15u;
      w[e] = __builtin_fmaf(dsc, (float)v, -dm);
    }
  } else if constexpr (QT == QT_Q6_K) {
    const size_t nsb = (size_t)(K / 256);
    const uint4 ql = *(const uint4*)(planes[0] + ((size_t)n * nsub + sb) * 16);
    const uint2 qh = *(const uint2*)(planes[1] + ((size_t)n * nsub + sb) * 8);
    const int8_t* sc = (const int8_t*)(planes[2] + ((size_t)n * nsb + (sb >> 3)) * 16) + 2 * (sb & 7);
    const float d = f16_bits_to_f32(*(const uint16_t*)(planes[3] + ((size_t)n * nsb + (sb >> 3)) * 2));
    const float ds0 = d * (float)sc[0], ds1 = d * (float)sc[1];
    const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t hw[2] = {qh.x, qh.y};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t lo = (lw[e >> 3] >> pi_shift(e & 7)) & 15u;
      const uint32_t hi = (hw[e >> 4] >> q6h_shift(e)) & 3u;
      w[e] = (e < 16 ? ds0 : ds1) * (float)((int)(lo | (hi << 4)) - 32);
    }
  } else {  // Q8_0: block index == sub-block index
    const int8_t* qs = (const int8_t*)(planes[0] + ((size_t)n * nsub + sb) * 32);
    const float d = f16_bits_to_f32(*(const uint16_t*)(planes[1] + ((size_t)n * nsub + sb) * 2));
    const uint4 a = *(const uint4*)qs;
    const uint4 b = *(const uint4*)(qs + 16);
    const uint32_t qw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int v = (int)(int8_t)((qw[e >> 2] >> (8 * (e & 3))) & 0xffu);
      w[e] = (float)v * d;
    }
  }
}

}  // namespace mlxr
