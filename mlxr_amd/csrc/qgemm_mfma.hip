// Kernel (b): prefill GEMM, Y[M,N] = X[M,K] . W[N,K]^T (+ bias) on bf16 MFMA.
//
// Replaces the large-M use of core/kernels/metal/q_gemm_dequant.metal:338-486 in the
// reference (tile loop :374-464: X tile to shared memory, W tile dequantized to shared
// memory, accumulate in fp32, bias + store :467-485).  Here each workgroup owns a
// BM x BN output tile; per 64-wide K step it stages X (bf16) into LDS, dequantizes the
// packed weight sub-blocks of its BN rows to fp32 with the exact GGUF formulas, rounds
// them to bf16 (RNE) into LDS, and feeds v_mfma_f32_32x32x16_bf16 with fp32 accumulators.
#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

struct MfmaParams {
  PlanePtrs P;
  const void* x;
  const void* bias;
  void* y;
  int M, N, K;
  int x_dtype, bias_dtype, y_dtype;
  int tiles_m, tiles_n;
};

constexpr int BK = 64;        // K elements per LDS stage (two 32-weight sub-blocks)
constexpr int LDK = BK + 8;   // LDS row pitch in bf16 elements (144 B: conflict-free b128 reads)

// fp16 activations are rounded to bf16 (RNE) when staged; bf16 ones are copied.
__device__ __forceinline__ uint32_t f16x2_to_bf16x2(uint32_t v) {
  return pack_bf16x2(f16_bits_to_f32(v & 0xffffu), f16_bits_to_f32(v >> 16));
}

template <int QT, int BM, int BN>
__global__ __launch_bounds__(256) void qgemm_mfma_kernel(MfmaParams p) {
  constexpr int TI = BM / 64, TJ = BN / 64;  // 32x32 MFMA tiles per wavefront (2x2 waves)
  __shared__ __attribute__((aligned(16))) uint16_t sA[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: consecutive workgroups on one XCD (workgroup id % 8) walk the M tiles of
  // the same N tile, so a weight tile is dequantized from one L2.
  const int ntiles = p.tiles_m * p.tiles_n;
  const int per_xcd = (ntiles + 7) / 8;
  const int b = blockIdx.x;
  int t = (b & 7) * per_xcd + (b >> 3);
  if ((ntiles & 7) != 0) t = b;  // uneven split: keep the plain order
  const int tm = t % p.tiles_m, tn = t / p.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  const int M = p.M, N = p.N, K = p.K;
  const int nsub = K >> 5;
  const int nkt = (K + BK - 1) / BK;
  const uint8_t* xb = (const uint8_t*)p.x;

  f32x16_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  for (int kt = 0; kt < nkt; ++kt) {
    // X tile: BM rows x 64 bf16 = 8 chunks of 16 B per row.
    for (int c = tid; c < BM * 8; c += 256) {
      const int r = c >> 3, kc = c & 7;
      const int gm = m0 + r, gk = kt * BK + kc * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gm < M && gk < K) {
        v = *(const uint4*)(xb + ((size_t)gm * K + gk) * 2);
        if (p.x_dtype == DT_F16) {
          v.x = f16x2_to_bf16x2(v.x);
          v.y = f16x2_to_bf16x2(v.y);
          v.z = f16x2_to_bf16x2(v.z);
          v.w = f16x2_to_bf16x2(v.w);
        }
      }
      *(uint4*)&sA[r * LDK + kc * 8] = v;
    }
    // W tile: BN rows x 2 sub-blocks, dequantized to bf16.
    for (int c = tid; c < BN * 2; c += 256) {
      const int r = c >> 1, j = c & 1;
      const int gn = n0 + r, sb = kt * 2 + j;
      uint4* dst = (uint4*)&sB[r * LDK + j * 32];
      if (gn < N && sb < nsub) {
        float w[32];
        dequant_sub_f32<QT>(p.P.p, K, gn, sb, w);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dst[i] = make_uint4(pack_bf16x2(w[8 * i + 0], w[8 * i + 1]), pack_bf16x2(w[8 * i + 2], w[8 * i + 3]),
                              pack_bf16x2(w[8 * i + 4], w[8 * i + 5]), pack_bf16x2(w[8 * i + 6], w[8 * i + 7]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = make_uint4(0, 0, 0, 0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t a[TI], bv[TJ];
      const int ko = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int row = wm * (BM / 2) + i * 32 + (lane & 31);
        a[i] = *(const bf16x8_t*)&sA[row * LDK + ko];
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int col = wn * (BN / 2) + j * 32 + (lane & 31);
        bv[j] = *(const bf16x8_t*)&sB[col * LDK + ko];
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Epilogue: accumulator v of a 32x32 tile is row 8*(v/4) + 4*(lane/32) + v%4,
  // column lane%32.
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
      if (col >= N) continue;
      const float bias = p.bias ? load_scalar(p.bias, p.bias_dtype, col) : 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M) store_scalar(p.y, p.y_dtype, (size_t)row * N + col, acc[i][j][v] + bias);
      }
    }
  }
}

template <int QT, int BM, int BN>
hipError_t launch_t(MfmaParams p, hipStream_t s) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
  qgemm_mfma_kernel<QT, BM, BN><<<grid, dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_mfma(const RunArgs& a, hipStream_t s) {
  MfmaParams p;
  p.P = plane_ptrs(a.L, a.packed);
  p.x = a.x;
  p.bias = a.bias;
  p.y = a.y;
  p.M = a.M;
  p.N = a.L.N;
  p.K = a.L.K;
  p.x_dtype = a.x_dtype;
  p.bias_dtype = a.bias_dtype;
  p.y_dtype = a.y_dtype;
  switch (a.L.qtype) {
    case QT_Q4_K: return launch_t<QT_Q4_K, 128, 128>(p, s);
    case QT_Q6_K: return launch_t<QT_Q6_K, 128, 128>(p, s);
    default: return launch_t<QT_Q8_0, 128, 128>(p, s);
  }
}

}  // namespace mlxr
