// Skinny GEMM for 4 < M <= 64 (batched decode): Y[M,N] = X[M,K] . W[N,K]^T (+ bias) on
// MFMA, streaming every weight byte from HBM exactly once.  Two variants: the one below
// on 32x32x16 MFMA (32 < M <= 64), and a narrow one further down on 16x16x32 MFMA for
// M <= 32 (qgemm_skinny16_kernel).
//
// At these M the VALU dot products of the GEMV kernel cost M/2 operations per weight and
// fall far behind HBM; here each weight is dequantized once in registers (the routines
// of qgemm_wdequant.h, the ones the prefill GEMM and mlxr_qgemm_dequant use) and the M
// rows of activations ride along in the MFMA: per 64-wide K step a lane decodes one
// 32-weight sub-block, about three VALU operations per weight, independent of M.
//
// Work split: a workgroup owns a slab of 32 weight rows and has W wavefronts, wavefront
// w taking the K steps [w*spw, (w+1)*spw).  Lane (n, h) of a wavefront owns weight row
// n0 + n and, in each step, sub-block h; K is permuted inside the step exactly as in the
// prefill GEMM (MFMA kk takes K positions 32h + 8kk .. +7 from both operands), so the
// lane's dequantized word kk is its MFMA operand.  The weights are the first operand
// (32 rows of N), the activations the second (32 rows of M, twice for M > 32), read from
// global memory (they are small and stay in L2).  Raw weights are loaded seven steps
// ahead, activations two, as branch-free buffer loads.  At the end the W partial tiles
// meet in LDS and are added in wavefront order.  (The narrow variant at M <= 8 can instead
// stage a wavefront's activations in LDS once, before its K loop: see XL below.)
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <utility>

#include "qgemm_device.h"
#include "qgemm_internal.h"
#include "qgemm_vmem.h"
#include "qgemm_wdequant.h"

namespace mlxr {

std::atomic<int> g_skinny_stage{1};

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

constexpr int TK = 64;
constexpr int MAXW = 8;  // wavefronts per workgroup
// raw weight ring (steps); loads run RING-1 steps ahead (Q8_0 sub-blocks are twice as
// large, so a shorter ring keeps its registers in budget)
template <int QT>
constexpr int ring_steps() { return QT == QT_Q8_0 ? 4 : 8; }

struct SkinnyParams {
  PlanePtrs P;
  uint32_t psize[4];  // plane sizes in bytes (< 2^31)
  const void* x;
  const void* bias;
  void* y;
  int M, N, K;
  int bias_dtype, y_dtype;
  int spw;  // K steps per wavefront (multiple of RING)
  int slabs;        // 32-row slabs; the grid is slabs x K splits
  int spg;          // K steps per workgroup (multiple of RING)
  float* ws;        // K splits over workgroups: fp32 partials, split s at ws + s * ws_split
  size_t ws_split;  // elements per split plane
  int ws_ld;        // workspace row stride (N; 2N for SwiGLU: gate then up columns)
  uint32_t nib;
  // SwiGLU (narrow kernel only): P2 is the up weight; a slab is 16 rows of both weights
  // (row tile 0 gate, 1 up) and the result swish(gate + bias) * (up + bias2) goes to y
  int swiglu;
  PlanePtrs P2;
  uint32_t psize2[4];
  const void* bias2;
};

// Compile-time loop: fn(integral_constant<int, i>) for i = 0 .. N-1, fully expanded.
template <typename Fn, int... I>
__device__ __forceinline__ void sfor_impl(Fn&& fn, std::integer_sequence<int, I...>) {
  (fn(std::integral_constant<int, I>()), ...);
}
template <int N, typename Fn>
__device__ __forceinline__ void sfor(Fn&& fn) {
  sfor_impl(fn, std::make_integer_sequence<int, N>());
}

template <int XT>
__device__ __forceinline__ f32x16_t mfma(const uint4& a, const uint4& b, const f32x16_t& c) {
  if constexpr (XT == X_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

template <int QT, int XT, int MB>
__global__ __launch_bounds__(64 * MAXW) void qgemm_skinny_kernel(SkinnyParams p) {
  constexpr int RING = ring_steps<QT>();
  __shared__ float red[MAXW][MB][16][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockDim.x >> 6;
  const int M = p.M, N = p.N, K = p.K;
  const int nsub = K >> 5, nsb = K >> 8;
  const int nkt = (K + TK - 1) / TK;
  const int ksplit = blockIdx.x / p.slabs;
  const int n0 = (blockIdx.x - ksplit * p.slabs) * 32;
  // M-block blockIdx.y: activation rows [m0, m0 + 64), addressed from its own base
  const int m0 = blockIdx.y * 64, Mt = M;
  const int Ml = min(64, Mt - m0);
  const uint16_t* const xb = (const uint16_t*)p.x + (size_t)m0 * (size_t)K;
  const int h = lane >> 5, n = n0 + (lane & 31);
  const bool rok = n < N;
  const uint32_t row_sub = rok ? (uint32_t)n * (uint32_t)nsub : 0u, row_sb = rok ? (uint32_t)n * (uint32_t)nsb : 0u;
  const int kg1 = min(nkt, (ksplit + 1) * p.spg);
  const int kt0 = ksplit * p.spg + wave * p.spw, kt1 = min(kg1, kt0 + p.spw);
  rsrc_t R[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) R[i] = make_rsrc(p.P.p[i] ? p.P.p[i] : (const uint8_t*)p.x, p.psize[i]);
  const rsrc_t RX = make_rsrc(xb, (uint32_t)Ml * (uint32_t)K * 2u);

  // activation rows of the second operand: m0 + mb*32 + lane%32; lane half h reads K
  // positions 32h + 8kk .. +7 of each step (kk at immediate offset 16kk)
  uint32_t xoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 32 + (lane & 31);
    xoff[mb] = m < Ml ? ((uint32_t)m * (uint32_t)K + 32u * h) * 2u : OOB;
  }
  const int ktail = K % TK;  // the 32-weight block types can end on a half step
  u32x4_t xf[4][4][MB];  // ring: step s in slot s % 4
  auto load_x = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    const bool live = kt < kt1 && !(ktail != 0 && kt == nkt - 1 && 32 * h >= ktail);
    const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane(kt * TK * 2);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t vo = live ? xoff[mb] : OOB;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) xf[slot][kk][mb] = __builtin_amdgcn_raw_buffer_load_b128(RX, vo + 16 * kk, soff, 0);
    }
  };

  Raw<QT> raw[RING];
  Hdr<QT> hdr[2];  // super-blocks of ring slots 0-3 and 4-7
  Scales<QT> sc;
  auto issue_raw = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    const int sb = 2 * kt + h;
    const bool in = kt < kt1 && sb < nsub && rok;
    load_raw<QT>(R, row_sub, sb, in, raw[slot]);
    if constexpr (is_kquant(QT) && (slot & 3) == 0) load_hdr<QT>(R, row_sb, kt >> 2, in, hdr[slot >> 2]);
  };

  f32x16_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[mb][v] = 0.f;

  // Step s issues the raw loads of step s+7 and the activations of step s+2.  The
  // prologue issues raw loads of steps kt0 .. kt0+6 and activations of kt0, kt0+1.
  sfor<RING - 1>([&](auto S_) {
    constexpr int s_ = decltype(S_)::value;
    issue_raw(kt0 + s_, std::integral_constant<int, s_>());
  });
  load_x(kt0, std::integral_constant<int, 0>());
  load_x(kt0 + 1, std::integral_constant<int, 1>());
  // step kt = kt0 + 8i + u: raw slot u, activations from xf[u % 4]
  auto step = [&](int kt, auto U) {
    constexpr int u = decltype(U)::value;
    issue_raw(kt + RING - 1, std::integral_constant<int, (u + RING - 1) % RING>());
    load_x(kt + 2, std::integral_constant<int, (u + 2) & 3>());
    if constexpr (is_kquant(QT) && (u & 3) == 0) decode_hdr<QT>(hdr[u >> 2], h, sc);
    uint4 w[4];
    w[0] = dequant_word<QT, XT, 0, true>(raw[u], sc, u & 3, p.nib);
    w[1] = dequant_word<QT, XT, 1, true>(raw[u], sc, u & 3, p.nib);
    w[2] = dequant_word<QT, XT, 2, true>(raw[u], sc, u & 3, p.nib);
    w[3] = dequant_word<QT, XT, 3, true>(raw[u], sc, u & 3, p.nib);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const u32x4_t xv = xf[u & 3][kk][mb];
        acc[mb] = mfma<XT>(w[kk], make_uint4(xv[0], xv[1], xv[2], xv[3]), acc[mb]);
      }
  };
  // whole rings, unconditionally: steps past kt1 load nothing and add zeros, and
  // straight-line code lets the compiler keep its load waits exact
  for (int kt = kt0; kt < kt1; kt += RING) {
    sfor<RING>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      step(kt + u, std::integral_constant<int, u>());
    });
  }

  // partial tiles meet in LDS; lane `lane` of the wavefront finishing M-block mb adds the
  // nw partials of its 16 accumulators in wavefront order.  Accumulator v holds Y[m][n] for m = mb*32 +
  // lane%32, n = n0 + 8(v/4) + 4(lane/32) + v%4.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int v = 0; v < 16; ++v) red[wave][mb][v][lane] = acc[mb][v];
  __syncthreads();
  // wavefront w finishes M-blocks w, w + nw, ... (a workgroup may have fewer wavefronts
  // than M-blocks when K is short)
  for (int mb = wave; mb < MB; mb += nw) {
    const int m = m0 + mb * 32 + (lane & 31);
    if (m >= Mt) continue;
    float out[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float s = 0.f;
      for (int w = 0; w < nw; ++w) s += red[w][mb][v][lane];
      out[v] = s;
    }
    const size_t rowbase = (size_t)m * N;
    if (p.ws) {  // K split over workgroups: this split's fp32 partial sums, no bias
      float* wsp = p.ws + (size_t)ksplit * p.ws_split + rowbase;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nn = n0 + 8 * q + 4 * (lane >> 5);
        if ((N & 3) == 0 && nn + 3 < N) {
          *(float4*)(wsp + nn) = make_float4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nn + e < N) wsp[nn + e] = out[4 * q + e];
        }
      }
      continue;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nn = n0 + 8 * q + 4 * (lane >> 5);
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v4[e] = out[4 * q + e] + ((p.bias && nn + e < N) ? load_scalar(p.bias, p.bias_dtype, nn + e) : 0.f);
      if ((N & 3) == 0 && nn + 3 < N && p.y_dtype != DT_F32) {
        const uint32_t lo = p.y_dtype == DT_BF16 ? pack_bf16x2(v4[0], v4[1]) : pack2<X_F16>(v4[0], v4[1]);
        const uint32_t hi = p.y_dtype == DT_BF16 ? pack_bf16x2(v4[2], v4[3]) : pack2<X_F16>(v4[2], v4[3]);
        *(uint2*)((uint16_t*)p.y + rowbase + nn) = make_uint2(lo, hi);
      } else if ((N & 3) == 0 && nn + 3 < N) {
        *(float4*)((float*)p.y + rowbase + nn) = make_float4(v4[0], v4[1], v4[2], v4[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nn + e < N) store_scalar(p.y, p.y_dtype, rowbase + nn + e, v4[e]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Narrow variant for M <= 32 on the 16x16x32 MFMA.  The activations are the second
// operand in 16-row blocks (NB of them), so at M = 8 or 16 half or none of the operand is
// padding instead of the 24 or 16 of 32 rows above, and each activation load feeds twice
// the weights: a step is 128 of K, a lane (r, j) = (lane % 16, lane / 16) owns sub-block j
// of the step for weight rows n0 + r and n0 + 16 + r, and MFMA kk takes word kk of every
// lane's sub-block (K positions 32j + 8kk .. +7 of the step, for both operands).  A
// K-quant super-block spans two steps: the lane's sub-blocks are j and 4 + j of it.
// Partial tiles of the workgroup's wavefronts meet in LDS as above.
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
constexpr int TK16 = 128;
template <int QT>
constexpr int ring16_steps() { return QT == QT_Q8_0 ? 2 : 4; }
constexpr int UNROLL16 = 4;  // steps per loop trip; steps per wavefront are a multiple

template <int XT>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (XT == X_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// Factors of sub-blocks j and 4 + j of a super-block (slots 0 and 1 of Scales): header
// entry e sits in word e / 2, half e % 2 (the layout decode_hdr reads).
template <int QT>
__device__ __forceinline__ void decode_hdr16(const Hdr<QT>& h, int j, Scales<QT>& s) {
  const uint32_t w[4] = {h.h[0], h.h[1], h.h[2], h.h[3]};
  if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
    const uint32_t dd = q4k_dd(make_uint4(w[0], w[1], w[2], w[3]));
    const float d = f16_bits_to_f32(dd & 0xffffu), dmin = f16_bits_to_f32(dd >> 16);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t v = w[2 * q + (j >> 1)];
      const uint32_t f = ((j & 1) ? (v >> 16) : v) & 0xfffu;
      s.a[q] = d * (float)(f & 63u);
      s.b[q] = -(dmin * (float)(f >> 6));
    }
  } else if constexpr (QT == QT_Q6_K) {
    const float d = f16_bits_to_f32(h.d & 0xffffu);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t v0 = w[2 * q + (j >> 1)];
      const uint32_t v = (j & 1) ? (v0 >> 16) : v0;
      s.a[q] = d * (float)(int8_t)(v & 0xffu);
      s.b[q] = d * (float)(int8_t)((v >> 8) & 0xffu);
    }
  }
}

// Staged-activation mode (XL): a wavefront's activations for its whole K range (at most
// XL_LOADS 16-byte loads per lane) are read once into LDS, so the K loop's only global loads
// are the weights.  SP = 2: a workgroup holds two slabs (SwiGLU: two 16-row slab pairs), the
// wavefronts of both walking the same K ranges, so each stage serves two wavefronts (half
// the LDS per slab, and the two share its loads).
constexpr int XL_LOADS = 16;

template <int QT, int XT, int NB, bool XL = false, int SP = 1>
__global__ __launch_bounds__(64 * MAXW) void qgemm_skinny16_kernel(SkinnyParams p) {
  static_assert(!XL || NB == 1, "staged activations cover one 16-row block");
  static_assert(SP == 1 || (SP == 2 && XL), "paired slabs share a stage");
  constexpr int D = ring16_steps<QT>();  // raw ring; loads run D - 1 steps ahead
  constexpr int RT = 2;                  // 16-row weight tiles per wavefront
  constexpr bool KQ = is_kquant(QT);
  constexpr int XD = 2;                  // activation loads run two steps ahead
  // XL: the dynamic LDS holds the wavefronts' activation stages, then the reduction
  __shared__ f32x4_t red_s[XL ? 1 : MAXW][RT * NB][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t xl_lds[];
  f32x4_t(*const red)[RT * NB][64] = XL ? reinterpret_cast<f32x4_t(*)[RT * NB][64]>(xl_lds) : red_s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockDim.x >> 6;
  // wavefront roles: slab sg of the workgroup's SP, K range wk of the slab's W
  const int W = nw / SP, sg = wave / W, wk = wave - sg * W;
  const int M = p.M, N = p.N, K = p.K;
  const int nsub = K >> 5, nsb = K >> 8;
  const int nkt = (K + TK16 - 1) / TK16;
  // each XCD (workgroup id % 8) takes a contiguous run of (K split, slab) pairs, so with K
  // split it reads the activations of one or two splits, not all of them
  const int nb = (int)gridDim.x;
  const int f = (nb & 7) == 0 ? ((int)blockIdx.x & 7) * (nb >> 3) + ((int)blockIdx.x >> 3) : (int)blockIdx.x;
  const int gpk = (p.slabs + SP - 1) / SP;  // workgroups per K split
  const int ksplit = f / gpk;
  const bool sw = p.swiglu != 0;
  // (SP = 2 with an odd slab count: the last workgroup's second slab lies past N, its rows
  // read zeros and store nothing)
  const int n0 = ((f - ksplit * gpk) * SP + sg) * (sw ? 16 : 32);
  const int r = lane & 15, j = lane >> 4;
  uint32_t row_sub[RT], row_sb[RT];
  bool rok[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int n = n0 + (sw ? 0 : 16 * t) + r;
    rok[t] = n < N;
    row_sub[t] = rok[t] ? (uint32_t)n * (uint32_t)nsub : 0u;
    row_sb[t] = rok[t] ? (uint32_t)n * (uint32_t)nsb : 0u;
  }
  const int kg1 = min(nkt, (ksplit + 1) * p.spg);
  const int kt0 = ksplit * p.spg + wk * p.spw, kt1 = min(kg1, kt0 + p.spw);
  rsrc_t R[RT][4];  // row tile t's weight (SwiGLU: tile 1 reads the up weight)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    R[0][i] = make_rsrc(p.P.p[i] ? p.P.p[i] : (const uint8_t*)p.x, p.psize[i]);
    R[1][i] = sw ? make_rsrc(p.P2.p[i] ? p.P2.p[i] : (const uint8_t*)p.x, p.psize2[i]) : R[0][i];
  }
  const rsrc_t RX = make_rsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);

  // activations: lane (m, j) of block nb reads row nb*16 + m, K 32j .. 32j+31 of the step
  uint32_t xoff[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int m = nb * 16 + r;
    xoff[nb] = m < M ? ((uint32_t)m * (uint32_t)K + 32u * (uint32_t)j) * 2u : OOB;
  }
  u32x4_t xf[XL ? 2 : 4][4][NB];  // step s in slot s % 4 (three live: loads run two steps ahead)
  // XL stage of this wavefront: step s (from kt0), row m at (s*M + m) * 256 bytes, its 16-byte
  // chunk c (K 8c .. 8c+7 of the step) at position c ^ m, so the 16 rows that one MFMA operand
  // read takes from chunk column c land in 16 different bank groups.  Lanes of rows >= M read
  // row M - 1: those lanes only feed output rows that are never stored.
  uint8_t* const xs = xl_lds + (size_t)wk * (size_t)p.spw * (size_t)M * 256u;
  uint32_t xl_off[4];
  if constexpr (XL) {
    const int rr = min(r, M - 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xl_off[kk] = (uint32_t)rr * 256u + (uint32_t)(((4 * j + kk) ^ rr) << 4);
  }
  auto load_x = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    if constexpr (XL) {
      const uint8_t* b = xs + (size_t)(kt - kt0) * (size_t)M * 256u;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) xf[slot & 1][kk][0] = *(const u32x4_t*)(b + xl_off[kk]);
      return;
    }
    const bool live = kt < kt1 && 4 * kt + j < nsub;
    const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane(kt * TK16 * 2);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint32_t vo = live ? xoff[nb] : OOB;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) xf[slot][kk][nb] = __builtin_amdgcn_raw_buffer_load_b128(RX, vo + 16 * kk, soff, 0);
    }
  };

  Raw<QT> raw[D][RT];
  Hdr<QT> hdr[KQ ? D / 2 : 1][RT];  // super-block of ring slots 2i, 2i + 1
  Scales<QT> sc[RT];
  auto issue_raw = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    const int sb = 4 * kt + j;
    const bool in = kt < kt1 && sb < nsub;
#pragma unroll
    for (int t = 0; t < RT; ++t) load_raw<QT>(R[t], row_sub[t], sb, in && rok[t], raw[slot][t]);
    if constexpr (KQ && (slot & 1) == 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) load_hdr<QT>(R[t], row_sb[t], kt >> 1, in && rok[t], hdr[slot >> 1][t]);
    }
  };

  f32x4_t acc[RT][NB];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[t][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if constexpr (XL) {
    // the whole stage (spw steps, zeros past kt1 and past K) is read before the weight ring
    // is issued, then written to LDS while the ring is in flight
    const int per = M * 4;  // 64-byte row quarters per step
    const uint32_t minv = (65536u + (uint32_t)per - 1u) / (uint32_t)per;  // exact g / per for g < 512
    u32x4_t st[XL_LOADS];
    uint32_t dst[XL_LOADS];
#pragma unroll
    for (int i = 0; i < XL_LOADS; ++i) {
      // (step, row, quarter) of this lane's 16 bytes; the SP wavefronts sharing the stage
      // take interleaved load rounds
      const int g = (i * SP + sg) * 16 + (lane >> 2);
      const int s = (int)(((uint32_t)g * minv) >> 16), rem = g - s * per;
      const int m = rem >> 2, c = 4 * (rem & 3) + (lane & 3);
      const int kt = kt0 + s;
      const bool ok = s < p.spw && kt < kt1 && 4 * kt + (c >> 2) < nsub;
      const uint32_t vo = ok ? ((uint32_t)m * (uint32_t)K + (uint32_t)kt * TK16 + 8u * (uint32_t)c) * 2u : OOB;
      st[i] = __builtin_amdgcn_raw_buffer_load_b128(RX, vo, 0, 0);
      dst[i] = s < p.spw ? (uint32_t)(s * M + m) * 256u + (uint32_t)((c ^ m) << 4) : ~0u;
    }
    sfor<D - 1>([&](auto S_) {
      constexpr int s_ = decltype(S_)::value;
      issue_raw(kt0 + s_, std::integral_constant<int, s_>());
    });
#pragma unroll
    for (int i = 0; i < XL_LOADS; ++i)
      if (dst[i] != ~0u) *(u32x4_t*)(xs + dst[i]) = st[i];
    if constexpr (SP > 1) __syncthreads();  // the stage holds the other wavefront's share too
    load_x(kt0, std::integral_constant<int, 0>());
  } else {
    sfor<D - 1>([&](auto S_) {
      constexpr int s_ = decltype(S_)::value;
      issue_raw(kt0 + s_, std::integral_constant<int, s_>());
      if constexpr (s_ < XD) load_x(kt0 + s_, std::integral_constant<int, s_>());
    });
    sfor<(XD > D - 1 ? XD - D + 1 : 0)>([&](auto S_) {
      constexpr int s_ = decltype(S_)::value + D - 1;
      load_x(kt0 + s_, std::integral_constant<int, s_>());
    });
  }
  // Step kt = kt0 + D*i + u (kt0 even, so an even u starts a super-block) issues the raw
  // loads of step kt + D - 1, then the activations of step kt + 2: the wait for the
  // activations of step kt (in-order counter) then covers raw loads issued two steps ago.
  auto step = [&](int kt, auto U) {
    constexpr int u = decltype(U)::value;
    issue_raw(kt + D - 1, std::integral_constant<int, (u + D - 1) % D>());
    // XL: the LDS read of the next step, while it lies inside this wavefront's stage
    if constexpr (XL) {
      if (kt + 1 < kt0 + p.spw) load_x(kt + 1, std::integral_constant<int, (u + 1) & 1>());
    } else {
      load_x(kt + XD, std::integral_constant<int, (u + XD) & 3>());
    }
    constexpr int ru = u % D;
    if constexpr (KQ && (u & 1) == 0) {
#pragma unroll
      for (int t = 0; t < RT; ++t) decode_hdr16<QT>(hdr[ru >> 1][t], j, sc[t]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      uint4 w[4];
      w[0] = dequant_word<QT, XT, 0, true>(raw[ru][t], sc[t], u & 1, p.nib);
      w[1] = dequant_word<QT, XT, 1, true>(raw[ru][t], sc[t], u & 1, p.nib);
      w[2] = dequant_word<QT, XT, 2, true>(raw[ru][t], sc[t], u & 1, p.nib);
      w[3] = dequant_word<QT, XT, 3, true>(raw[ru][t], sc[t], u & 1, p.nib);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[t][nb] = mfma16<XT>(w[kk], xf[XL ? (u & 1) : (u & 3)][kk][nb], acc[t][nb]);
    }
  };
  for (int kt = kt0; kt < kt1; kt += UNROLL16) {
    sfor<UNROLL16>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      step(kt + u, std::integral_constant<int, u>());
    });
  }

  // Accumulator tile (t, nb): lane holds Y[m][n .. n+3] for m = nb*16 + lane%16,
  // n = n0 + 16t + 4(lane/16) (SwiGLU: n = n0 + 4(lane/16) of weight t).
  if constexpr (XL) __syncthreads();  // the reduction reuses the activation stages
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[wave][t * NB + nb][lane] = acc[t][nb];
  __syncthreads();
  if (sw) {
    // wavefront wk of slab sg finishes M-blocks wk, wk + W, ...: gate and up sums of the
    // same outputs, over the slab's wavefronts in order
    for (int nb = wk; nb < NB; nb += W) {
      const int m = nb * 16 + r;
      if (m >= M) continue;
      const int w0 = sg * W;
      f32x4_t g = red[w0][nb][lane], u = red[w0][NB + nb][lane];
      for (int w = 1; w < W; ++w) {
        g += red[w0 + w][nb][lane];
        u += red[w0 + w][NB + nb][lane];
      }
      const int nn = n0 + 4 * j;
      if (p.ws) {  // K split over workgroups: partial sums, gate then up columns
        float* wsp = p.ws + (size_t)ksplit * p.ws_split + (size_t)m * p.ws_ld;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nn + e < N) {
            wsp[nn + e] = g[e];
            wsp[N + nn + e] = u[e];
          }
        continue;
      }
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = nn + e < N;
        const float gb = (p.bias && ok) ? load_scalar(p.bias, p.bias_dtype, nn + e) : 0.f;
        const float ub = (p.bias2 && ok) ? load_scalar(p.bias2, p.bias_dtype, nn + e) : 0.f;
        v4[e] = swiglu1(g[e] + gb, u[e] + ub);
      }
      const size_t rowbase = (size_t)m * N;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nn + e < N) store_scalar(p.y, p.y_dtype, rowbase + nn + e, v4[e]);
    }
    return;
  }
  for (int u = wk; u < RT * NB; u += W) {
    const int t = u / NB, nb = u - t * NB;
    const int m = nb * 16 + r;
    if (m >= M) continue;
    const int w0 = sg * W;
    f32x4_t sum = red[w0][u][lane];
    for (int w = 1; w < W; ++w) sum += red[w0 + w][u][lane];
    const int nn = n0 + 16 * t + 4 * j;
    const size_t rowbase = (size_t)m * N;
    if (p.ws) {  // K split over workgroups: this split's fp32 partial sums, no bias
      float* wsp = p.ws + (size_t)ksplit * p.ws_split + rowbase;
      if ((N & 3) == 0 && nn + 3 < N) {
        *(float4*)(wsp + nn) = make_float4(sum[0], sum[1], sum[2], sum[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nn + e < N) wsp[nn + e] = sum[e];
      }
      continue;
    }
    float v4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v4[e] = sum[e] + ((p.bias && nn + e < N) ? load_scalar(p.bias, p.bias_dtype, nn + e) : 0.f);
    if ((N & 3) == 0 && nn + 3 < N && p.y_dtype != DT_F32) {
      const uint32_t lo = p.y_dtype == DT_BF16 ? pack_bf16x2(v4[0], v4[1]) : pack2<X_F16>(v4[0], v4[1]);
      const uint32_t hi = p.y_dtype == DT_BF16 ? pack_bf16x2(v4[2], v4[3]) : pack2<X_F16>(v4[2], v4[3]);
      *(uint2*)((uint16_t*)p.y + rowbase + nn) = make_uint2(lo, hi);
    } else if ((N & 3) == 0 && nn + 3 < N) {
      *(float4*)((float*)p.y + rowbase + nn) = make_float4(v4[0], v4[1], v4[2], v4[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nn + e < N) store_scalar(p.y, p.y_dtype, rowbase + nn + e, v4[e]);
    }
  }
}

// Launch geometry: workgroups own 32-row slabs and, when the slabs are fewer than the CUs
// and a workspace is allowed, a K range (ks splits, each a whole number of rings); inside
// a workgroup the wavefronts split the range again, enough of them for about eight per CU.
struct SkinnyPlan {
  int ks, spg, w, spw;
};
SkinnyPlan skinny_plan(int N, int K, int ring, bool allow_split, int mblocks = 1) {
  constexpr int wpc = 8;  // wavefronts per CU aimed for
  const int cus = device_cu_count();
  const int slabs = (N + 31) / 32 * mblocks;  // workgroups per K split
  const int nkt = (K + TK - 1) / TK;
  SkinnyPlan pl;
  pl.ks = allow_split && slabs < cus ? std::max(1, std::min(cus / slabs, nkt / ring)) : 1;
  pl.spg = (((nkt + pl.ks - 1) / pl.ks) + ring - 1) / ring * ring;
  pl.ks = (nkt + pl.spg - 1) / pl.spg;
  const long want = (long)wpc * cus;
  pl.w = (int)std::min<long>(MAXW, std::max<long>(1, (want + (long)slabs * pl.ks - 1) / ((long)slabs * pl.ks)));
  pl.spw = (((pl.spg + pl.w - 1) / pl.w) + ring - 1) / ring * ring;
  pl.w = (pl.spg + pl.spw - 1) / pl.spw;
  return pl;
}

// The narrow kernels' geometry: as skinny_plan, in 128-wide steps (whole multiples of
// `unroll` per wavefront), at most `wcap` wavefronts per workgroup, the K split over
// workgroups sized for about `wpc` wavefronts per CU.
SkinnyPlan skinny16_plan(int N, int K, bool allow_split, int unroll, int wcap, int wpc) {
  const int maxw = std::max(1, std::min(wcap, MAXW));
  const int cus = device_cu_count();
  const int slabs = (N + 31) / 32;
  const int nkt = (K + TK16 - 1) / TK16;
  const long want = (long)wpc * cus;
  SkinnyPlan pl;
  pl.ks = 1;
  // split K over workgroups (partials + a reduce launch, a few us) only when the slabs
  // alone would fill less than half the target
  if (allow_split && 2L * slabs * maxw <= want)
    pl.ks = (int)std::max<long>(1, std::min<long>((want + (long)slabs * maxw - 1) / ((long)slabs * maxw),
                                                  nkt / unroll));
  pl.spg = (((nkt + pl.ks - 1) / pl.ks) + unroll - 1) / unroll * unroll;
  pl.ks = (nkt + pl.spg - 1) / pl.spg;
  pl.w = (int)std::min<long>(maxw, std::max<long>(1, (want + (long)slabs * pl.ks - 1) / ((long)slabs * pl.ks)));
  pl.spw = (((pl.spg + pl.w - 1) / pl.w) + unroll - 1) / unroll * unroll;
  pl.w = (pl.spg + pl.spw - 1) / pl.spw;
  return pl;
}

bool use_skinny16(int M) { return M <= 32; }

// Staged activations at most this many bytes per workgroup (with the reduction's static
// LDS, within a CU's 160 KiB); the launcher also requires that the whole grid still fits on
// the device at the workgroups per CU the stages leave.
constexpr size_t kXlMaxBytes = 128u * 1024u;
// Static LDS of the staged kernel (its unused reduction array of one wavefront).
constexpr size_t kXlStaticBytes = 2u * 64u * 16u;

// The narrow kernel's plan: SwiGLU slabs are 16 rows of two weights, planned as 32-row
// slabs of a problem with as many slabs.
SkinnyPlan s16_plan(const SkinnyParams& sp, bool allow_split) {
  const int Np = sp.swiglu ? 32 * ((sp.N + 15) / 16) : sp.N;
  return skinny16_plan(Np, sp.K, allow_split, UNROLL16, MAXW, 8);
}
size_t s16_ws_bytes(const SkinnyParams& sp, const SkinnyPlan& pl) {
  return pl.ks > 1 ? (size_t)pl.ks * (size_t)sp.M * (size_t)sp.N * (sp.swiglu ? 8u : 4u) : 0;
}

template <int QT, int XT>
hipError_t launch_s16(SkinnyParams sp, size_t ws_bytes, hipStream_t s) {
  sp.slabs = sp.swiglu ? (sp.N + 15) / 16 : (sp.N + 31) / 32;
  SkinnyPlan pl = s16_plan(sp, sp.ws != nullptr);
  if (s16_ws_bytes(sp, pl) > ws_bytes) pl = s16_plan(sp, false);
  sp.spg = pl.spg;
  sp.spw = pl.spw;
  sp.ws_ld = sp.swiglu ? 2 * sp.N : sp.N;
  sp.ws_split = (size_t)sp.M * (size_t)sp.ws_ld;
  float* const ws = (float*)sp.ws;
  void* const y = sp.y;
  const void* const bias = sp.bias;
  if (pl.ks == 1) sp.ws = nullptr;
  const dim3 grid((unsigned)(sp.slabs * pl.ks)), block((unsigned)(64 * pl.w));
  // Staged activations: only where a wavefront runs at least eight steps (shorter ranges
  // lose more to the staging latency than the K loop gains) and the stages do not limit how
  // many workgroups a CU holds at once; one slab per workgroup where that fits, else two
  // slabs sharing their stages (half the LDS per slab).  Same products in the same order
  // in every mode.
  const int mode = g_skinny_stage.load(std::memory_order_relaxed);  // 0 off, 2: paired first
  // wavefronts per SIMD the staged kernels' registers allow, queried once per device
  static std::atomic<int> occ_cache[2][64];
  auto simd_occupancy = [&](int sps) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
    int v = occ_cache[sps - 1][dev].load(std::memory_order_relaxed);
    if (v == 0) {
      const void* fn = sps == 1 ? (const void*)qgemm_skinny16_kernel<QT, XT, 1, true, 1>
                                : (const void*)qgemm_skinny16_kernel<QT, XT, 1, true, 2>;
      int nb = 0;  // resident four-wavefront workgroups without dynamic LDS: one wave per SIMD each
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, 256, 0) != hipSuccess || nb <= 0) nb = 1;
      v = nb;
      occ_cache[sps - 1][dev].store(v, std::memory_order_relaxed);
    }
    return v;
  };
  auto stage_fits = [&](int sps, size_t* lds) {
    const long groups = (long)(sp.slabs + sps - 1) / sps * pl.ks;
    const size_t xl_bytes = (size_t)pl.w * (size_t)pl.spw * (size_t)sp.M * 256u;
    // the stages, or the reduction of the wavefronts' partial tiles if larger
    *lds = std::max(xl_bytes, (size_t)sps * pl.w * 2u * 64u * 16u);
    if (!(sp.M <= 8 * sps && pl.w * sps <= MAXW && pl.spw >= 8 && pl.spw * sp.M * 4 <= sps * XL_LOADS * 16 &&
          *lds <= kXlMaxBytes))
      return false;
    // the whole grid resident at once: workgroups per CU by LDS, and by registers (a
    // workgroup of more than four wavefronts puts two or more on a SIMD; measured on MI355X,
    // grids past this ran a second round and lost to the global-read mode)
    const long by_lds = (long)(device_lds_limit() / (*lds + kXlStaticBytes));
    const long by_regs = simd_occupancy(sps) / ((pl.w * sps + 3) / 4);
    return std::min(by_lds, by_regs) * device_cu_count() >= groups;
  };
  size_t lds1 = 0, lds2 = 0;
  const bool fit1 = mode != 0 && stage_fits(1, &lds1), fit2 = mode != 0 && stage_fits(2, &lds2);
  const int sps = fit1 && !(mode == 2 && fit2) ? 1 : fit2 ? 2 : 0;
  if (sps) {
    const size_t lds = sps == 1 ? lds1 : lds2;
    const dim3 sgrid((unsigned)((sp.slabs + sps - 1) / sps * pl.ks)), sblock((unsigned)(64 * pl.w * sps));
    const void* const fn = sps == 1 ? (const void*)qgemm_skinny16_kernel<QT, XT, 1, true, 1>
                                    : (const void*)qgemm_skinny16_kernel<QT, XT, 1, true, 2>;
    static std::atomic<uint64_t> attr_set[2];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(attr_set[sps - 1].load(std::memory_order_acquire) & bit)) {
      // the most this kernel ever asks for, within what the device allows (the launch
      // condition above keeps every launch below both)
      const size_t cap = std::min(kXlMaxBytes, device_lds_limit() - kXlStaticBytes);
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)cap);
      if (e != hipSuccess) return e;
      attr_set[sps - 1].fetch_or(bit, std::memory_order_release);
    }
    if (sps == 1) qgemm_skinny16_kernel<QT, XT, 1, true, 1><<<sgrid, sblock, lds, s>>>(sp);
    else qgemm_skinny16_kernel<QT, XT, 1, true, 2><<<sgrid, sblock, lds, s>>>(sp);
  } else if (sp.M <= 16) {
    qgemm_skinny16_kernel<QT, XT, 1><<<grid, block, 0, s>>>(sp);
  } else {
    qgemm_skinny16_kernel<QT, XT, 2><<<grid, block, 0, s>>>(sp);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || pl.ks == 1) return e;
  if (sp.swiglu)
    return launch_splitk_reduce_swiglu(ws, sp.ws_split, pl.ks, bias, sp.bias2, sp.bias_dtype, y, sp.y_dtype, sp.M,
                                       sp.N, s);
  return launch_splitk_reduce(ws, sp.ws_split, pl.ks, bias, sp.bias_dtype, y, sp.y_dtype, sp.M, sp.N, s);
}

template <int QT, int XT>
hipError_t launch_s(SkinnyParams sp, size_t ws_bytes, hipStream_t s) {
  if (use_skinny16(sp.M)) return launch_s16<QT, XT>(sp, ws_bytes, s);
  constexpr int RING = ring_steps<QT>();
  sp.slabs = (sp.N + 31) / 32;
  const int mblocks = (sp.M + 63) / 64;
  SkinnyPlan pl = skinny_plan(sp.N, sp.K, RING, sp.ws != nullptr, mblocks);
  if (pl.ks > 1 && (size_t)pl.ks * (size_t)sp.M * (size_t)sp.N * 4u > ws_bytes)
    pl = skinny_plan(sp.N, sp.K, RING, false, mblocks);
  sp.spg = pl.spg;
  sp.spw = pl.spw;
  sp.ws_ld = sp.N;
  sp.ws_split = (size_t)sp.M * (size_t)sp.N;
  float* const ws = (float*)sp.ws;
  void* const y = sp.y;
  const void* const bias = sp.bias;
  if (pl.ks == 1) sp.ws = nullptr;
  const dim3 grid((unsigned)(sp.slabs * pl.ks), (unsigned)mblocks), block((unsigned)(64 * pl.w));
  if (sp.M <= 32) qgemm_skinny_kernel<QT, XT, 1><<<grid, block, 0, s>>>(sp);
  else qgemm_skinny_kernel<QT, XT, 2><<<grid, block, 0, s>>>(sp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || pl.ks == 1) return e;
  return launch_splitk_reduce(ws, sp.ws_split, pl.ks, bias, sp.bias_dtype, y, sp.y_dtype, sp.M, sp.N, s);
}

}  // namespace

hipError_t launch_skinny(const RunArgs& a, hipStream_t s) {
  SkinnyParams sp;
  sp.P = plane_ptrs(a.L, a.packed);
  for (int i = 0; i < 4; ++i) sp.psize[i] = i < a.L.nplanes ? (uint32_t)a.L.size[i] : 0u;
  sp.x = a.x;
  sp.bias = a.bias;
  sp.y = a.y;
  sp.M = a.M;
  sp.N = a.L.N;
  sp.K = a.L.K;
  sp.bias_dtype = a.bias_dtype;
  sp.y_dtype = a.y_dtype;
  sp.nib = 0x0F0F0F0Fu;
  sp.ws = (float*)a.ws;
  sp.swiglu = 0;
  sp.P2 = sp.P;
  for (int i = 0; i < 4; ++i) sp.psize2[i] = sp.psize[i];
  sp.bias2 = nullptr;
  const size_t wsb = a.ws ? a.ws_bytes : 0;
  const bool f16 = a.x_dtype == DT_F16;
  switch (a.L.qtype) {
    case QT_Q4_K: return f16 ? launch_s<QT_Q4_K, X_F16>(sp, wsb, s) : launch_s<QT_Q4_K, X_BF16>(sp, wsb, s);
    case QT_Q6_K: return f16 ? launch_s<QT_Q6_K, X_F16>(sp, wsb, s) : launch_s<QT_Q6_K, X_BF16>(sp, wsb, s);
    case QT_Q5_K: return f16 ? launch_s<QT_Q5_K, X_F16>(sp, wsb, s) : launch_s<QT_Q5_K, X_BF16>(sp, wsb, s);
    case QT_Q4_0: return f16 ? launch_s<QT_Q4_0, X_F16>(sp, wsb, s) : launch_s<QT_Q4_0, X_BF16>(sp, wsb, s);
    case QT_Q4_1: return f16 ? launch_s<QT_Q4_1, X_F16>(sp, wsb, s) : launch_s<QT_Q4_1, X_BF16>(sp, wsb, s);
    default: return f16 ? launch_s<QT_Q8_0, X_F16>(sp, wsb, s) : launch_s<QT_Q8_0, X_BF16>(sp, wsb, s);
  }
}

namespace {
SkinnyParams swiglu_params(const RunArgs& gate, const RunArgs& up) {
  SkinnyParams sp;
  sp.P = plane_ptrs(gate.L, gate.packed);
  sp.P2 = plane_ptrs(up.L, up.packed);
  for (int i = 0; i < 4; ++i) {
    sp.psize[i] = i < gate.L.nplanes ? (uint32_t)gate.L.size[i] : 0u;
    sp.psize2[i] = i < up.L.nplanes ? (uint32_t)up.L.size[i] : 0u;
  }
  sp.x = gate.x;
  sp.bias = gate.bias;
  sp.bias2 = up.bias;
  sp.y = gate.y;
  sp.M = gate.M;
  sp.N = gate.L.N;
  sp.K = gate.L.K;
  sp.bias_dtype = gate.bias_dtype;
  sp.y_dtype = gate.y_dtype;
  sp.nib = 0x0F0F0F0Fu;
  sp.ws = (float*)gate.ws;
  sp.swiglu = 1;
  return sp;
}
}  // namespace

bool skinny_swiglu_ok(int M) { return M <= 32; }

hipError_t launch_skinny_swiglu(const RunArgs& gate, const RunArgs& up, hipStream_t s) {
  const SkinnyParams sp = swiglu_params(gate, up);
  const size_t wsb = gate.ws ? gate.ws_bytes : 0;
  const bool f16 = gate.x_dtype == DT_F16;
  switch (gate.L.qtype) {
    case QT_Q4_K: return f16 ? launch_s16<QT_Q4_K, X_F16>(sp, wsb, s) : launch_s16<QT_Q4_K, X_BF16>(sp, wsb, s);
    case QT_Q6_K: return f16 ? launch_s16<QT_Q6_K, X_F16>(sp, wsb, s) : launch_s16<QT_Q6_K, X_BF16>(sp, wsb, s);
    case QT_Q5_K: return f16 ? launch_s16<QT_Q5_K, X_F16>(sp, wsb, s) : launch_s16<QT_Q5_K, X_BF16>(sp, wsb, s);
    case QT_Q4_0: return f16 ? launch_s16<QT_Q4_0, X_F16>(sp, wsb, s) : launch_s16<QT_Q4_0, X_BF16>(sp, wsb, s);
    case QT_Q4_1: return f16 ? launch_s16<QT_Q4_1, X_F16>(sp, wsb, s) : launch_s16<QT_Q4_1, X_BF16>(sp, wsb, s);
    default: return f16 ? launch_s16<QT_Q8_0, X_F16>(sp, wsb, s) : launch_s16<QT_Q8_0, X_BF16>(sp, wsb, s);
  }
}

size_t skinny_swiglu_workspace_bytes(int M, int N, int K) {
  SkinnyParams sp;
  sp.M = M;
  sp.N = N;
  sp.K = K;
  sp.swiglu = 1;
  return s16_ws_bytes(sp, s16_plan(sp, true));
}

bool skinny_fits(const RunArgs& a) {
  const size_t lim = operand_limit();
  if ((size_t)a.M * (size_t)a.L.K * 2u >= lim) return false;
  for (int i = 0; i < a.L.nplanes; ++i)
    if (a.L.size[i] >= lim) return false;
  return true;
}

double skinny_mb_est_us(int M, int N, int K) {
  // each 32-row slab reads its 64-row blocks of X from L2 (~7.5 TB/s device-wide), plus
  // ~8 us of launch, prologue and epilogue (measured on MI355X, Llama-3-8B shapes)
  return 8.0 + (double)((N + 31) / 32) * M * K * 2.0 / 7.5e6;
}

size_t skinny_workspace_bytes(int M, int N, int K, int qtype) {
  const SkinnyPlan pl = use_skinny16(M) ? skinny16_plan(N, K, true, UNROLL16, MAXW, 8)
                                         : skinny_plan(N, K, qtype == QT_Q8_0 ? 4 : 8, true, (M + 63) / 64);
  return pl.ks > 1 ? (size_t)pl.ks * (size_t)M * (size_t)N * 4u : 0;
}

}  // namespace mlxr
