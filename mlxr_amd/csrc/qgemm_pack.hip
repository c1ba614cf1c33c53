// One-time repack of GGUF blocks into the planar layout, and the dequant kernel.
//
// Reference counterparts: the block records of core/kernels/primitives/
// q_gemm_dequant_primitive.mm:29-57 (GGUF block_q4_0 / q4_1 / q8_0 / q4_K / q6_K), the
// upload the reference skips at daemon/server/model_loader.cpp:236-245, and the CPU
// dequant routines at q_gemm_dequant_primitive.mm:189-225.
#include "qgemm_device.h"
#include "qgemm_internal.h"
#include "qgemm_wdequant.h"

namespace mlxr {

namespace {

__device__ __forceinline__ uint32_t rd_u8(const uint8_t* p, int i) { return p[i]; }
__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p, int i) {
  return (uint32_t)p[i] | ((uint32_t)p[i + 1] << 8);
}

// One thread per (row, super-block).  Source: 144-byte block_q4_K records.
__global__ void pack_q4k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs_out,
                                uint8_t* __restrict__ hdr_out, int N, int nsb) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nsb) return;
  const uint8_t* b = src + idx * 144;
  const uint8_t* s = b + 4;
  const uint8_t* q = b + 16;
  // header: u16 j = sc_j | m_j << 6 | (nibble j of d | dmin << 16) << 12
  const uint32_t dd = rd_u16(b, 0) | (rd_u16(b, 2) << 16);
  uint16_t* h = (uint16_t*)(hdr_out + idx * 16);
  for (int j = 0; j < 8; ++j) {
    uint32_t sc, m;
    if (j < 4) {
      sc = s[j] & 63u;
      m = s[j + 4] & 63u;
    } else {
      sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
      m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
    h[j] = (uint16_t)(sc | (m << 6) | (((dd >> (4 * j)) & 15u) << 12));
  }
  // qs: sub-block j = 64-chunk j/2, low (j even) or high (j odd) nibbles
  uint32_t* o = (uint32_t*)(qs_out + idx * 128);
  for (int j = 0; j < 8; ++j) {
    const int c = j >> 1, hi = j & 1;
    for (int t = 0; t < 4; ++t) {
      uint32_t w = 0;
      for (int e = 0; e < 8; ++e) {
        const uint32_t byte = rd_u8(q, 32 * c + 8 * t + e);
        const uint32_t v = hi ? (byte >> 4) : (byte & 15u);
        w |= v << pi_shift(e);
      }
      o[4 * j + t] = w;
    }
  }
}

// One thread per (row, super-block).  Source: 176-byte block_q5_K records
// {d, dmin, scales[12], qh[32], qs[128]}: header and qs as Q4_K; the fifth bit of element
// l of sub-block j is bit j of qh[l].
__global__ void pack_q5k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs_out,
                                uint8_t* __restrict__ qh_out, uint8_t* __restrict__ hdr_out, int N, int nsb) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nsb) return;
  const uint8_t* b = src + idx * 176;
  const uint8_t* s = b + 4;
  const uint8_t* qh = b + 16;
  const uint8_t* q = b + 48;
  const uint32_t dd = rd_u16(b, 0) | (rd_u16(b, 2) << 16);
  uint16_t* h = (uint16_t*)(hdr_out + idx * 16);
  for (int j = 0; j < 8; ++j) {
    uint32_t sc, m;
    if (j < 4) {
      sc = s[j] & 63u;
      m = s[j + 4] & 63u;
    } else {
      sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
      m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
    h[j] = (uint16_t)(sc | (m << 6) | (((dd >> (4 * j)) & 15u) << 12));
  }
  uint32_t* o = (uint32_t*)(qs_out + idx * 128);
  uint32_t* oh = (uint32_t*)(qh_out + idx * 32);
  for (int j = 0; j < 8; ++j) {
    const int c = j >> 1, hi = j & 1;
    uint32_t hw = 0;
    for (int t = 0; t < 4; ++t) {
      uint32_t w = 0;
      for (int e = 0; e < 8; ++e) {
        const uint32_t byte = rd_u8(q, 32 * c + 8 * t + e);
        w |= (hi ? (byte >> 4) : (byte & 15u)) << pi_shift(e);
        hw |= ((rd_u8(qh, 8 * t + e) >> j) & 1u) << q5h_bit(8 * t + e);
      }
      o[4 * j + t] = w;
    }
    oh[j] = hw;
  }
}

// One thread per (row, super-block).  Source: 210-byte block_q6_K records.
__global__ void pack_q6k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ ql_out,
                                uint8_t* __restrict__ qh_out, uint8_t* __restrict__ sc_out,
                                uint8_t* __restrict__ d_out, int N, int nsb) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nsb) return;
  const uint8_t* b = src + idx * 210;
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  uint32_t* lo = (uint32_t*)(ql_out + idx * 128);
  uint32_t* ho = (uint32_t*)(qh_out + idx * 64);
  for (int j = 0; j < 8; ++j) {  // 32-weight sub-block j = weights 32j..32j+31
    const int h = j >> 2, t4 = j & 3;
    uint32_t lw[4] = {0u, 0u, 0u, 0u}, hw[2] = {0u, 0u};
    for (int e = 0; e < 32; ++e) {
      const uint32_t l4 = (rd_u8(ql, 64 * h + e + 32 * (t4 & 1)) >> (4 * (t4 >> 1))) & 15u;
      const uint32_t h2 = (rd_u8(qh, 32 * h + e) >> (2 * t4)) & 3u;
      lw[e >> 3] |= l4 << pi_shift(e & 7);
      hw[e >> 4] |= h2 << q6h_shift(e);
    }
    for (int t = 0; t < 4; ++t) lo[4 * j + t] = lw[t];
    ho[2 * j + 0] = hw[0];
    ho[2 * j + 1] = hw[1];
  }
  for (int i = 0; i < 16; ++i) sc_out[idx * 16 + i] = b[192 + i];
  d_out[idx * 2 + 0] = b[208];
  d_out[idx * 2 + 1] = b[209];
}

// One thread per (row, block).  Source: 34-byte block_q8_0 records.
__global__ void pack_q80_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs_out,
                                uint8_t* __restrict__ d_out, int N, int nb) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nb) return;
  const uint8_t* b = src + idx * 34;
  uint32_t* o = (uint32_t*)(qs_out + idx * 32);
  for (int t = 0; t < 8; ++t)
    o[t] = rd_u8(b, 2 + 4 * t) | (rd_u8(b, 3 + 4 * t) << 8) | (rd_u8(b, 4 + 4 * t) << 16) |
           (rd_u8(b, 5 + 4 * t) << 24);
  d_out[idx * 2 + 0] = b[0];
  d_out[idx * 2 + 1] = b[1];
}

// One thread per (row, block).  Source: 18-byte block_q4_0 or 20-byte block_q4_1 records;
// GGUF element e < 16 is the low nibble of byte e, e >= 16 the high nibble of byte e - 16.
template <int QT>
__global__ void pack_q4_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs_out,
                               uint8_t* __restrict__ d_out, int N, int nb) {
  constexpr int HB = QT == QT_Q4_1 ? 4 : 2;  // header bytes (d, and m for Q4_1)
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nb) return;
  const uint8_t* b = src + idx * (HB + 16);
  const uint8_t* q = b + HB;
  uint32_t* o = (uint32_t*)(qs_out + idx * 16);
  for (int t = 0; t < 4; ++t) {
    uint32_t w = 0;
    for (int e = 0; e < 8; ++e) {
      const int el = 8 * t + e;
      const uint32_t byte = rd_u8(q, el & 15);
      w |= (el < 16 ? (byte & 15u) : (byte >> 4)) << pi_shift(e);
    }
    o[t] = w;
  }
  for (int i = 0; i < HB; ++i) d_out[idx * HB + i] = b[i];
}

// One thread per (row, 32-weight sub-block): 32 outputs.
template <int QT>
__global__ void dequant_kernel(PlanePtrs P, int N, int K, void* __restrict__ out, int out_dtype, uint32_t nib) {
  const int nsub = K / 32;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * nsub) return;
  const int n = (int)(idx / nsub), sb = (int)(idx % nsub);
  RawSub<QT> r;
  load_raw_sub<QT>(P.p, K, n, sb, r);
  const size_t o = (size_t)n * K + (size_t)sb * 32;
  if (out_dtype == DT_F32) {
    float w[32];
    dequant_raw<QT>(r, sb & 7, w);
    float4* dst = (float4*)((float*)out + o);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  } else {
    // the routine the MFMA GEMM uses to build its weight operands
    uint4 v[4];
    dequant_sub_words<QT, X_BF16>(P, K, n, sb, nib, v);
    uint4* dst = (uint4*)((uint16_t*)out + o);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = v[i];
  }
}

}  // namespace

hipError_t launch_pack(const PackedLayout& L, const uint8_t* gguf_dev, uint8_t* packed_dev,
                       hipStream_t s) {
  const int threads = 256;
  if (L.qtype == QT_Q4_K) {
    const int nsb = L.K / 256;
    const size_t total = (size_t)L.N * nsb;
    pack_q4k_kernel<<<dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s>>>(
        gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1], L.N, nsb);
  } else if (L.qtype == QT_Q5_K) {
    const int nsb = L.K / 256;
    const size_t total = (size_t)L.N * nsb;
    pack_q5k_kernel<<<dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s>>>(
        gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1], packed_dev + L.off[2], L.N, nsb);
  } else if (L.qtype == QT_Q6_K) {
    const int nsb = L.K / 256;
    const size_t total = (size_t)L.N * nsb;
    pack_q6k_kernel<<<dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s>>>(
        gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1], packed_dev + L.off[2],
        packed_dev + L.off[3], L.N, nsb);
  } else if (L.qtype == QT_Q4_0 || L.qtype == QT_Q4_1) {
    const int nb = L.K / 32;
    const size_t total = (size_t)L.N * nb;
    const dim3 grid((unsigned)((total + threads - 1) / threads));
    if (L.qtype == QT_Q4_0)
      pack_q4_kernel<QT_Q4_0><<<grid, dim3(threads), 0, s>>>(gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1],
                                                             L.N, nb);
    else
      pack_q4_kernel<QT_Q4_1><<<grid, dim3(threads), 0, s>>>(gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1],
                                                             L.N, nb);
  } else {
    const int nb = L.K / 32;
    const size_t total = (size_t)L.N * nb;
    pack_q80_kernel<<<dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s>>>(
        gguf_dev, packed_dev + L.off[0], packed_dev + L.off[1], L.N, nb);
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const PackedLayout& L, const uint8_t* packed_dev, void* out, int out_dtype,
                          hipStream_t s) {
  const PlanePtrs P = plane_ptrs(L, packed_dev);
  const size_t total = (size_t)L.N * (L.K / 32);
  const int threads = 256;
  const dim3 grid((unsigned)((total + threads - 1) / threads));
  if (L.qtype == QT_Q4_K)
    dequant_kernel<QT_Q4_K><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  else if (L.qtype == QT_Q6_K)
    dequant_kernel<QT_Q6_K><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  else if (L.qtype == QT_Q5_K)
    dequant_kernel<QT_Q5_K><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  else if (L.qtype == QT_Q4_0)
    dequant_kernel<QT_Q4_0><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  else if (L.qtype == QT_Q4_1)
    dequant_kernel<QT_Q4_1><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  else
    dequant_kernel<QT_Q8_0><<<grid, dim3(threads), 0, s>>>(P, L.N, L.K, out, out_dtype, 0x0F0F0F0Fu);
  return hipGetLastError();
}

}  // namespace mlxr
