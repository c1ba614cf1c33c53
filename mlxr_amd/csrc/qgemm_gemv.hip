// Kernel (a): decode GEMV / skinny GEMM, Y[M,N] = X[M,K] . W[N,K]^T (+ bias), M <= 64.
//
// Replaces the M-small use of core/kernels/metal/q_gemm_dequant.metal:338-486 in the
// reference.  No MFMA: the weights are streamed from HBM exactly once with 16-byte loads
// (a wavefront reads 1 KiB of contiguous nibbles per instruction), two 4-bit weights are
// turned into a bf16 (or fp16) pair with one mask-and-or into a magic exponent
// (value = 128 + q for bf16, 1024 + q for fp16), multiplied with activation pairs by
// v_dot2_f32_{bf16,f16} into fp32, and the row sums are reduced across the wavefront
// with DPP row operations plus three readlanes.
//
// Per sub-block j the magic offset and the Q4_K min are folded into one correction,
//   sum_e x_e * (d*sc_j*q_e - dmin*m_j) = d*sc_j*(S_j - OFF*X_j) - dmin*m_j*X_j,
//   S_j = sum_e x_e*(OFF + q_e) (dot2 result),  X_j = sum_e x_e,
// so the weights are never materialised as floats.
//
// Work split: one workgroup = 4 wavefronts; a wavefront owns R output rows and walks K
// in segments of 64 sub-blocks (2048 weights), lane i taking sub-block 64*seg + i.  The
// lane's 32 activations are loaded once per segment and reused for all R rows.
#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {

namespace {

enum XType : int { X_BF16 = 0, X_F16 = 1 };

struct GemvParams {
  PlanePtrs P;
  const void* x;
  const void* bias;
  void* y;
  int M, N, K;
  int bias_dtype, y_dtype;
};

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

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *(const uint4*)p; }

// Weights of one row and one sub-block, as loaded from HBM.
template <int QT>
struct WLoad;
template <>
struct WLoad<QT_Q4_K> {
  uint4 q, h;
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

template <int QT>
__device__ __forceinline__ void load_w(const PlanePtrs& P, int K, int n, int sb, WLoad<QT>& w) {
  const size_t nsub = (size_t)(K >> 5);
  if constexpr (QT == QT_Q4_K) {
    const size_t nsb = (size_t)(K >> 8);
    w.q = ld16(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.h = ld16(P.p[1] + ((size_t)n * nsb + (sb >> 3)) * 16);
  } else if constexpr (QT == QT_Q6_K) {
    const size_t nsb = (size_t)(K >> 8);
    w.ql = ld16(P.p[0] + ((size_t)n * nsub + sb) * 16);
    w.qh = *(const uint2*)(P.p[1] + ((size_t)n * nsub + sb) * 8);
    w.sc = *(const uint16_t*)(P.p[2] + ((size_t)n * nsb + (sb >> 3)) * 16 + 2 * (sb & 7));
    w.d = *(const uint16_t*)(P.p[3] + ((size_t)n * nsb + (sb >> 3)) * 2);
  } else {
    const uint8_t* q = P.p[0] + ((size_t)n * nsub + sb) * 32;
    w.a = ld16(q);
    w.b = ld16(q + 16);
    w.d = *(const uint16_t*)(P.p[1] + ((size_t)n * nsub + sb) * 2);
  }
}
template <int QT>
__device__ __forceinline__ void zero_w(WLoad<QT>& w) {
  if constexpr (QT == QT_Q4_K) {
    w.q = make_uint4(0, 0, 0, 0);
    w.h = make_uint4(0, 0, 0, 0);
  } else if constexpr (QT == QT_Q6_K) {
    w.ql = make_uint4(0, 0, 0, 0);
    w.qh = make_uint2(0, 0);
    w.sc = 0;
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
};

template <int QT, int XT>
__device__ __forceinline__ void decode_w(const WLoad<QT>& w, int j, WDec& o) {
  if constexpr (QT == QT_Q4_K) {
    constexpr uint32_t MAGIC = (XT == X_BF16) ? 0x43004300u : 0x64006400u;
    const uint32_t qw[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) o.p[4 * t + s] = ((qw[t] >> (4 * s)) & 0x000F000Fu) | MAGIC;
    const uint32_t f = q4k_field(w.h.y, w.h.z, w.h.w, j);
    o.s0 = f16_bits_to_f32(w.h.x & 0xffffu) * (float)(f & 63u);
    o.s1 = f16_bits_to_f32(w.h.x >> 16) * (float)(f >> 6);
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
  if constexpr (QT == QT_Q4_K) {
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

template <int QT, int XT, int MT, int R>
__global__ __launch_bounds__(256) void qgemv_kernel(GemvParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= p.N) return;
  const int K = p.K, M = p.M;
  const int nsub = K >> 5;
  const int nseg = (nsub + 63) >> 6;
  const uint8_t* xb = (const uint8_t*)p.x;

  float acc[MT][R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int seg = 0; seg < nseg; ++seg) {
    const int sb = seg * 64 + lane;
    const bool active = sb < nsub;
    WLoad<QT> wl[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (active && row0 + r < p.N) load_w<QT>(p.P, K, row0 + r, sb, wl[r]);
      else zero_w<QT>(wl[r]);
    }
    WDec wd[R];
#pragma unroll
    for (int r = 0; r < R; ++r) decode_w<QT, XT>(wl[r], lane & 7, wd[r]);

#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) {
        uint32_t xv[16];
        if (active) {
          const uint8_t* xp = xb + ((size_t)m * K + (size_t)sb * 32) * 2;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint4 v = ld16(xp + 16 * i);
            xv[4 * i + 0] = v.x;
            xv[4 * i + 1] = v.y;
            xv[4 * i + 2] = v.z;
            xv[4 * i + 3] = v.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) xv[i] = 0u;
        }
        float X0 = 0.f, X1 = 0.f;
        if constexpr (!(QT == QT_Q8_0 && XT == X_BF16)) {
          X0 = sum_range<XT, 0, 8>(xv);
          X1 = sum_range<XT, 8, 16>(xv);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] += contrib<QT, XT>(xv, wd[r], X0, X1);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m < M) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float tot = wave_sum(acc[m][r]);
        const int n = row0 + r;
        if (lane == ((m * R + r) & 63) && n < p.N) {
          float v = tot;
          if (p.bias) v += load_scalar(p.bias, p.bias_dtype, n);
          store_scalar(p.y, p.y_dtype, (size_t)m * p.N + n, v);
        }
      }
    }
  }
}

template <int QT, int XT, int MT, int R>
hipError_t launch_t(const GemvParams& p, hipStream_t s) {
  const int rows_per_block = 4 * R;
  const dim3 grid((unsigned)((p.N + rows_per_block - 1) / rows_per_block));
  qgemv_kernel<QT, XT, MT, R><<<grid, dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

template <int QT, int XT>
hipError_t launch_x(const GemvParams& p, int R, hipStream_t s) {
  const int M = p.M;
  if (M == 1) {
    if (R >= 4) return launch_t<QT, XT, 1, 4>(p, s);
    if (R == 2) return launch_t<QT, XT, 1, 2>(p, s);
    return launch_t<QT, XT, 1, 1>(p, s);
  }
  if (M <= 2) return launch_t<QT, XT, 2, 2>(p, s);
  if (M <= 4) return launch_t<QT, XT, 4, 2>(p, s);
  if (M <= 8) return launch_t<QT, XT, 8, 2>(p, s);
  if (M <= 16) return launch_t<QT, XT, 16, 2>(p, s);
  if (M <= 32) return launch_t<QT, XT, 32, 1>(p, s);
  return launch_t<QT, XT, 64, 1>(p, s);
}

// Rows per wavefront at M = 1: as many as keep >= 16 wavefronts per CU in flight.
int pick_rows(int N) {
  if (N >= 4 * 4096) return 4;
  if (N >= 2 * 4096) return 2;
  return 1;
}

}  // namespace

hipError_t launch_gemv(const RunArgs& a, hipStream_t s) {
  GemvParams p;
  p.P = plane_ptrs(a.L, a.packed);
  p.x = a.x;
  p.bias = a.bias;
  p.y = a.y;
  p.M = a.M;
  p.N = a.L.N;
  p.K = a.L.K;
  p.bias_dtype = a.bias_dtype;
  p.y_dtype = a.y_dtype;
  const int R = pick_rows(p.N);
  const bool f16 = a.x_dtype == DT_F16;
  switch (a.L.qtype) {
    case QT_Q4_K: return f16 ? launch_x<QT_Q4_K, X_F16>(p, R, s) : launch_x<QT_Q4_K, X_BF16>(p, R, s);
    case QT_Q6_K: return f16 ? launch_x<QT_Q6_K, X_F16>(p, R, s) : launch_x<QT_Q6_K, X_BF16>(p, R, s);
    default: return f16 ? launch_x<QT_Q8_0, X_F16>(p, R, s) : launch_x<QT_Q8_0, X_BF16>(p, R, s);
  }
}

}  // namespace mlxr
