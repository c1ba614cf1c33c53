// Kernel (b): prefill GEMM, Y[M,N] = X[M,K] . W[N,K]^T (+ bias) on bf16 MFMA.
//
// Replaces the large-M use of core/kernels/metal/q_gemm_dequant.metal:338-486 in the
// reference (tile loop :374-464: X tile to shared memory, W tile dequantized to shared
// memory, accumulate in fp32, bias + store :467-485).  Here each workgroup owns a
// BM x BN output tile; per 64-wide K step it stages X (bf16) into LDS, dequantizes the
// packed weight sub-blocks of its BN rows to fp32 with the exact GGUF formulas, rounds
// them to bf16 (RNE) into LDS, and feeds v_mfma_f32_32x32x16_bf16 with fp32 accumulators.
#include <stdlib.h>

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

// Large-tile variant: BM x BN = 256 x 256 per workgroup, four wavefronts in a 2 x 2
// arrangement, each owning a 128 x 128 sub-tile as 4 x 4 accumulators of the 32x32x16
// MFMA (256 fp32 per lane, held in AGPRs).  Two LDS stages: while the MFMAs consume stage
// s, the next K step's activation chunks and raw weight sub-blocks are already in
// registers (loaded before the MFMAs), and are written -- the weights dequantized to
// bf16 -- into stage s^1 afterwards; one barrier per K step.
constexpr int BIG = 256;
constexpr int BIG_STAGE_ELEMS = 2 * BIG * LDK;                         // A + B tiles, bf16
constexpr size_t BIG_LDS_BYTES = 2 * (size_t)BIG_STAGE_ELEMS * 2;      // two stages

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
constexpr uint32_t OOB = 0x80000000u;  // voffset beyond every buffer: the load returns 0

__device__ __forceinline__ rsrc_t make_rsrc(const void* ptr, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t voff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Raw (still quantized) weight sub-block loaded through buffer resources; invalid rows
// and K tails read zeros, which dequantize to zeros.
template <int QT>
__device__ __forceinline__ void bload_raw_sub(const rsrc_t* R, int K, int n, int sb, bool ok, RawSub<QT>& r) {
  const uint32_t nsub = (uint32_t)(K >> 5), nsb = (uint32_t)(K >> 8);
  const uint32_t s = (uint32_t)n * nsub + (uint32_t)sb;   // sub-block index
  const uint32_t g = (uint32_t)n * nsb + (uint32_t)(sb >> 3);  // super-block index
  if constexpr (QT == QT_Q4_K) {
    r.q = bload16(R[0], ok ? s * 16u : OOB);
    r.h = bload16(R[1], ok ? g * 16u : OOB);
  } else if constexpr (QT == QT_Q6_K) {
    r.ql = bload16(R[0], ok ? s * 16u : OOB);
    const u32x2_t h = __builtin_amdgcn_raw_buffer_load_b64(R[1], ok ? s * 8u : OOB, 0, 0);
    r.qh = make_uint2(h[0], h[1]);
    r.sc = __builtin_amdgcn_raw_buffer_load_b16(R[2], ok ? g * 16u + 2u * (uint32_t)(sb & 7) : OOB, 0, 0);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(R[3], ok ? g * 2u : OOB, 0, 0);
  } else {
    r.a = bload16(R[0], ok ? s * 32u : OOB);
    r.b = bload16(R[0], ok ? s * 32u + 16u : OOB);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? s * 2u : OOB, 0, 0);
  }
}

struct BigParams {
  MfmaParams m;
  uint32_t psize[4];  // plane sizes in bytes (< 2^31)
  uint32_t nib;       // 0x0F0F0F0F (run-time constant for the dequant)
};

// Scheduling hints: interleave `n` MFMAs with VALU / LDS-write work of the next tile.
#define SCHED_MFMA(n) __builtin_amdgcn_sched_group_barrier(0x008, n, 0)
#define SCHED_VALU(n) __builtin_amdgcn_sched_group_barrier(0x002, n, 0)
#define SCHED_DSW(n) __builtin_amdgcn_sched_group_barrier(0x200, n, 0)
#define SCHED_DSR(n) __builtin_amdgcn_sched_group_barrier(0x100, n, 0)
#define SCHED_VMEM(n) __builtin_amdgcn_sched_group_barrier(0x020, n, 0)

template <int QT, bool XF16>
__global__ __launch_bounds__(256, 1) void qgemm_mfma_big_kernel(BigParams bp) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const MfmaParams& p = bp.m;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order: each XCD (workgroup id % 8) takes a contiguous run of tiles in
  // M-major order, so it keeps one activation panel in its L2 while walking N.
  const int ntiles = p.tiles_m * p.tiles_n;
  const int per_xcd = (ntiles + 7) >> 3;
  const int b = blockIdx.x;
  int t = (b & 7) * per_xcd + (b >> 3);
  if ((ntiles & 7) != 0) t = b;
  const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
  const int m0 = tm * BIG, n0 = tn * BIG;

  const int M = p.M, N = p.N, K = p.K;
  const int nsub = K >> 5;
  const int nkt = (K + BK - 1) / BK;
  const rsrc_t RX = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  rsrc_t R[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) R[i] = make_rsrc(p.P.p[i] ? p.P.p[i] : (const uint8_t*)p.x, bp.psize[i]);

  // Per-thread load assignment.  A: 256 rows x 8 chunks of 16 B -> rows (tid>>3)+32i,
  // chunk tid&7, i = 0..7.  B: 256 rows x 2 sub-blocks -> rows (tid>>1)+128i, sub tid&1.
  const int a_row = tid >> 3, a_kc = tid & 7;
  const int b_row = tid >> 1, b_j = tid & 1;

  struct Raw {
    uint4 a[8];
    RawSub<QT> w[2];
  };
  auto load_tiles = [&](int kt, Raw& r) {
    const int gk = kt * BK + a_kc * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int gm = m0 + a_row + 32 * i;
      r.a[i] = bload16(RX, (gm < M && gk < K) ? ((uint32_t)gm * K + gk) * 2u : OOB);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gn = n0 + b_row + 128 * i, sb = kt * 2 + b_j;
      bload_raw_sub<QT>(R, K, gn, sb, gn < N && sb < nsub, r.w[i]);
    }
  };
  // Slice q (0..3) of writing tile kt from registers into LDS stage `stage`:
  // slices 0, 1 dequantize weight sub-block 0, 1; slices 2, 3 store four activation chunks each.
  auto store_slice = [&](const Raw& r, int kt, int stage, int q) {
    uint16_t* sA = lds + stage * BIG_STAGE_ELEMS;
    uint16_t* sB = sA + BIG * LDK;
    if (q < 2) {
      uint4 v[4];
      dequant_raw_bf16<QT>(r.w[q], (kt * 2 + b_j) & 7, bp.nib, v);
      uint4* dst = (uint4*)&sB[(b_row + 128 * q) * LDK + b_j * 32];
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[c] = v[c];
    } else {
#pragma unroll
      for (int i = 4 * (q - 2); i < 4 * (q - 2) + 4; ++i) {
        uint4 v = r.a[i];
        if constexpr (XF16) {
          v.x = f16x2_to_bf16x2(v.x);
          v.y = f16x2_to_bf16x2(v.y);
          v.z = f16x2_to_bf16x2(v.z);
          v.w = f16x2_to_bf16x2(v.w);
        }
        *(uint4*)&sA[(a_row + 32 * i) * LDK + a_kc * 8] = v;
      }
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Fragment reads: lane supplies rows (lane & 31) of its 32-row slab, 8 K values at
  // offset 8 * (lane >> 5) within each 16-wide step.
  const int a_off = (wm * 128 + (lane & 31)) * LDK + (lane >> 5) * 8;
  const int b_off = (wn * 128 + (lane & 31)) * LDK + (lane >> 5) * 8;
  auto read_frags = [&](int stage, int kk, bf16x8_t* fa, bf16x8_t* fb) {
    const uint16_t* sA = lds + stage * BIG_STAGE_ELEMS;
    const uint16_t* sB = sA + BIG * LDK;
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = *(const bf16x8_t*)&sA[a_off + i * 32 * LDK + kk * 16];
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = *(const bf16x8_t*)&sB[b_off + j * 32 * LDK + kk * 16];
  };

  // One K step on LDS stage `stage`, with tile kt+1 (in `cur`) written into stage^1 and
  // tile kt+2 loaded into `nxt` underneath the MFMAs.
  auto kstep = [&](int kt, int stage, Raw& cur, Raw& nxt) {
    load_tiles(min(kt + 2, nkt - 1), nxt);
    bf16x8_t fa[2][4], fb[2][4];
    read_frags(stage, 0, fa[0], fb[0]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) read_frags(stage, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
      store_slice(cur, kt + 1, stage ^ 1, kk);
      // 16 MFMAs; the next fragments' LDS reads, this slice's VALU and its LDS writes are
      // spread between them.
      if (kk < 2) {
#pragma unroll
        for (int g = 0; g < 16; ++g) {
          SCHED_MFMA(1);
          if (kk + 1 < BK / 16 && g < 8) SCHED_DSR(1);
          SCHED_VALU(7);
          if ((g & 3) == 3) SCHED_DSW(1);
        }
      } else {
#pragma unroll
        for (int g = 0; g < 16; ++g) {
          SCHED_MFMA(1);
          if (kk + 1 < BK / 16 && g < 8) SCHED_DSR(1);
          SCHED_VALU(1);
          if ((g & 3) == 3) SCHED_DSW(1);
        }
      }
    }
    __syncthreads();
  };

  Raw r0, r1;
  load_tiles(0, r0);
  load_tiles(min(1, nkt - 1), r1);
#pragma unroll
  for (int q = 0; q < 4; ++q) store_slice(r0, 0, 0, q);
  __syncthreads();
  // r1 holds tile 1; steady state alternates the register sets.
  int kt = 0;
  for (; kt + 2 <= nkt; kt += 2) {
    kstep(kt, 0, r1, r0);
    kstep(kt + 1, 1, r0, r1);
  }
  if (kt < nkt) kstep(kt, 0, r1, r0);

  // Epilogue: accumulator v of a 32x32 tile is row 8*(v/4) + 4*(lane/32) + v%4, column lane%32.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = n0 + wn * 128 + j * 32 + (lane & 31);
    if (col >= N) continue;
    const float bias = p.bias ? load_scalar(p.bias, p.bias_dtype, col) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M) store_scalar(p.y, p.y_dtype, (size_t)row * N + col, acc[i][j][v] + bias);
      }
    }
  }
}

template <int QT, bool XF16>
hipError_t launch_big_t(const BigParams& bp, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void*)qgemm_mfma_big_kernel<QT, XF16>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)BIG_LDS_BYTES);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  qgemm_mfma_big_kernel<QT, XF16><<<dim3((unsigned)(bp.m.tiles_m * bp.m.tiles_n)), dim3(256), BIG_LDS_BYTES, s>>>(bp);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_big(MfmaParams p, const PackedLayout& L, hipStream_t s) {
  BigParams bp;
  bp.m = p;
  bp.m.tiles_m = (p.M + BIG - 1) / BIG;
  bp.m.tiles_n = (p.N + BIG - 1) / BIG;
  for (int i = 0; i < 4; ++i) bp.psize[i] = i < L.nplanes ? (uint32_t)L.size[i] : 0u;
  bp.nib = 0x0F0F0F0Fu;
  return p.x_dtype == DT_F16 ? launch_big_t<QT, true>(bp, s) : launch_big_t<QT, false>(bp, s);
}

// 32-bit buffer offsets: every plane and the activations must stay below 2 GiB.
bool big_fits(const MfmaParams& p, const PackedLayout& L) {
  for (int i = 0; i < L.nplanes; ++i)
    if (L.size[i] >= (1u << 31)) return false;
  return (size_t)p.M * p.K * 2 < (1u << 31);
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
  static const int use_tile = getenv("MLXR_MFMA_OLD") ? 0 : 1;
  if (use_tile && tile_fits(a)) return launch_tile(a, s);
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
  // 256 x 256 tiles once there are enough of them to cover the chip; 128 x 128 otherwise.
  const long big_tiles = (long)((p.M + 255) / 256) * ((p.N + 255) / 256);
  static const int force = getenv("MLXR_MFMA_TILE") ? atoi(getenv("MLXR_MFMA_TILE")) : 0;
  const bool big = big_fits(p, a.L) && (force ? force == 256 : big_tiles >= 192);
  switch (a.L.qtype) {
    case QT_Q4_K: return big ? launch_big<QT_Q4_K>(p, a.L, s) : launch_t<QT_Q4_K, 128, 128>(p, s);
    case QT_Q6_K: return big ? launch_big<QT_Q6_K>(p, a.L, s) : launch_t<QT_Q6_K, 128, 128>(p, s);
    default: return big ? launch_big<QT_Q8_0>(p, a.L, s) : launch_t<QT_Q8_0, 128, 128>(p, s);
  }
}

}  // namespace mlxr
