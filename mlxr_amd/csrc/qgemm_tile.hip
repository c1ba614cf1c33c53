// Kernel (b): prefill GEMM, Y[M,N] = X[M,K] . W[N,K]^T (+ bias) on 32x32x16 MFMA.
//
// Replaces the large-M use of core/kernels/metal/q_gemm_dequant.metal:338-486 in the
// reference (tile loop :374-464: X tile to shared memory, W tile dequantized, fp32
// accumulation, bias + store :467-485).
//
// Tile: 256 (M) x 256 (N) per workgroup, K in steps of 64, four wavefronts; wavefront w
// owns the 256 x 64 slab of output columns [64w, 64w + 64) as 8 x 2 accumulators of the
// 32x32x16 MFMA (256 fp32 per lane, in AGPRs).
//
//  * Activations (shared by the four wavefronts) go HBM -> LDS by buffer_load ... lds
//    (no VGPR staging), four stages, three steps ahead.  A 256 x 64 stage is 32 KiB: row
//    r is 128 B, its 16-byte chunk c stored at position c ^ (r & 7), so the fragment
//    reads of eight consecutive rows hit eight different 16-byte bank groups.  The DMA is
//    issued from inline assembly, so the compiler (which would otherwise wait for every
//    outstanding load before each LDS read) leaves the waits to the exact vmcnt below.
//  * Weights never pass through LDS.  K is permuted inside each 64-step so that in MFMA
//    kk (0..3) lane half h supplies K positions 32h + 8kk .. +7 for both operands: lane
//    (n, h) then owns exactly sub-block h of the step for its weight rows n and n + 32,
//    dequantizes those 32 weights in registers and uses word kk of the result as the B
//    fragment of MFMA kk.  Per-super-block header work (d, dmin, six-bit scales) is done
//    once per four steps.  The raw sub-blocks are loaded four steps ahead; the dequant
//    of step k+1 runs between the MFMAs of step k.
//  * One barrier per step: a stage is refilled only after every wavefront has left it.
//
// The dequantized values are the exact GGUF fp32 weights rounded to nearest-even bf16
// (fp16 for fp16 activations, which use the fp16 MFMA); the same routine backs
// mlxr_qgemm_dequant, so they are covered by its bit-exact tests.
#include <stdlib.h>

#include <type_traits>

#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t OOB = 0x80000000u;  // voffset beyond every buffer: loads return 0
constexpr int TM = 256, TN = 256, TK = 64;
constexpr int NSTAGE = 4;
constexpr int A_STAGE = TM * TK * 2;  // bytes
constexpr int PD = 4;                 // raw weight prefetch distance (steps)
constexpr int TILE_LDS = NSTAGE * A_STAGE;

enum XType : int { X_BF16 = 0, X_F16 = 1 };

__device__ __forceinline__ rsrc_t make_rsrc(const void* ptr, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

struct TileParams {
  const void* x;
  const void* bias;
  void* y;
  const uint8_t* P[4];
  uint32_t psize[4];
  int M, N, K;
  int bias_dtype, y_dtype;
  int tiles_m, tiles_n;
  uint32_t nib;  // 0x0F0F0F0F, passed at run time (keeps the byte converts)
};

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

// ---- per-quant-type raw sub-block, header state and dequant --------------------------

// Loads from inline assembly: the compiler neither sees nor waits for them; every wait
// is an explicit s_waitcnt vmcnt(n) computed from the fixed issue order, followed by
// pin() on the registers it covers (an empty asm that makes their later uses depend on
// the wait).  Rows and sub-blocks past the end use an out-of-range offset and read 0.
__device__ __forceinline__ u32x4_t vload16(const i32x4_t& r, uint32_t voff) {
  u32x4_t v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=&v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ u32x4_t vload16_o16(const i32x4_t& r, uint32_t voff) {
  u32x4_t v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:16" : "=&v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ u32x2_t vload8(const i32x4_t& r, uint32_t voff) {
  u32x2_t v;
  asm volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen" : "=&v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ uint32_t vload_u16(const i32x4_t& r, uint32_t voff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=&v"(v) : "v"(voff), "s"(r));
  return v;
}
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

// VMEM instructions of one step's raw loads (two weight rows), and of its header loads.
template <int QT>
constexpr int raw_loads() { return QT == QT_Q4_K ? 2 : QT == QT_Q6_K ? 4 : 6; }
template <int QT>
constexpr int hdr_loads() { return QT == QT_Q4_K ? 2 : QT == QT_Q6_K ? 4 : 0; }

template <int QT>
__device__ __forceinline__ void load_raw(const i32x4_t* R, uint32_t row_sub, int sb, bool ok, Raw<QT>& r) {
  // row_sub = row * nsub (sub-block index of the row start); sb = sub-block within the row
  const uint32_t s = row_sub + (uint32_t)sb;
  if constexpr (QT == QT_Q4_K) {
    r.q = vload16(R[0], ok ? s * 16u : OOB);
  } else if constexpr (QT == QT_Q6_K) {
    r.ql = vload16(R[0], ok ? s * 16u : OOB);
    r.qh = vload8(R[1], ok ? s * 8u : OOB);
  } else {
    const uint32_t o = ok ? s * 32u : OOB;
    r.a = vload16(R[0], o);
    r.b = vload16_o16(R[0], o);
    r.d = vload_u16(R[1], ok ? s * 2u : OOB);
  }
}

template <int QT>
__device__ __forceinline__ void load_hdr(const i32x4_t* R, uint32_t row_sb, int g, bool ok, Hdr<QT>& h) {
  // row_sb = row * nsb; g = super-block within the row
  const uint32_t s = row_sb + (uint32_t)g;
  if constexpr (QT == QT_Q4_K) {
    h.h = vload16(R[1], ok ? s * 16u : OOB);
  } else if constexpr (QT == QT_Q6_K) {
    h.h = vload16(R[2], ok ? s * 16u : OOB);
    h.d = vload_u16(R[3], ok ? s * 2u : OOB);
  }
}

template <int QT>
__device__ __forceinline__ void decode_hdr(const Hdr<QT>& h, int half, Scales<QT>& s) {
  if constexpr (QT == QT_Q4_K) {
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

// B fragment kk of one sub-block: its weights 8kk .. 8kk+7, rounded to the MFMA type.
template <int QT, int XT, int kk>
__device__ __forceinline__ uint4 dequant_word(const Raw<QT>& r, const Scales<QT>& s, int q, uint32_t nib) {
  if constexpr (QT == QT_Q4_K) {
    const float a = s.a[q], b = s.b[q];
    uint32_t w = r.q[kk];
    pin(w);  // keeps this work at its place in the MFMA stream
    // pair-interleaved word: bytes of (w & nib) are weights 0, 4, 1, 5; of ((w >> 4) & nib) 2, 6, 3, 7
    const uint32_t lo = w & nib, hi = (w >> 4) & nib;
    const float e0 = __builtin_fmaf(a, (float)(lo & 0xffu), b);
    const float e4 = __builtin_fmaf(a, (float)((lo >> 8) & 0xffu), b);
    const float e1 = __builtin_fmaf(a, (float)((lo >> 16) & 0xffu), b);
    const float e5 = __builtin_fmaf(a, (float)(lo >> 24), b);
    const float e2 = __builtin_fmaf(a, (float)(hi & 0xffu), b);
    const float e6 = __builtin_fmaf(a, (float)((hi >> 8) & 0xffu), b);
    const float e3 = __builtin_fmaf(a, (float)((hi >> 16) & 0xffu), b);
    const float e7 = __builtin_fmaf(a, (float)(hi >> 24), b);
    return make_uint4(pack2<XT>(e0, e1), pack2<XT>(e2, e3), pack2<XT>(e4, e5), pack2<XT>(e6, e7));
  } else if constexpr (QT == QT_Q6_K) {
    // weights 8kk .. 8kk+7: group 0 (scale a) for kk < 2, group 1 (scale b) otherwise;
    // value d*sc*(q - 32) = fma(d*sc, q, -32*d*sc), exact
    const float a = (kk < 2) ? s.a[q] : s.b[q];
    const float c = -32.f * a;
    uint32_t lw = r.ql[kk];
    uint32_t hv = r.qh[kk >> 1];
    pin(lw);  // keeps this work at its place in the MFMA stream
    pin(hv);
    uint32_t o[4];
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      const int rs = 8 * (kk & 1) + 2 * sp - 4;
      const uint32_t hs = rs >= 0 ? (hv >> rs) : (hv << (-rs));
      const uint32_t v = ((lw >> (4 * sp)) & (nib & 0x000F000Fu)) | (hs & 0x00300030u);
      o[sp] = pack2<XT>(__builtin_fmaf(a, (float)(v & 0xffu), c), __builtin_fmaf(a, (float)((v >> 16) & 0xffu), c));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  } else {
    // int8 q -> (q + 128) by flipping the sign bits; q*d = fma(d, q + 128, -128 d), exact
    const float d = f16_bits_to_f32(r.d & 0xffffu), c = -128.f * d;
    const uint32_t w0 = kk < 2 ? r.a[2 * kk] : r.b[2 * kk - 4];
    const uint32_t w1 = kk < 2 ? r.a[2 * kk + 1] : r.b[2 * kk - 3];
    uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    pin(u0);  // keeps this work at its place in the MFMA stream
    pin(u1);
    return make_uint4(pack2<XT>(__builtin_fmaf(d, (float)(u0 & 0xffu), c), __builtin_fmaf(d, (float)((u0 >> 8) & 0xffu), c)),
                      pack2<XT>(__builtin_fmaf(d, (float)((u0 >> 16) & 0xffu), c), __builtin_fmaf(d, (float)(u0 >> 24), c)),
                      pack2<XT>(__builtin_fmaf(d, (float)(u1 & 0xffu), c), __builtin_fmaf(d, (float)((u1 >> 8) & 0xffu), c)),
                      pack2<XT>(__builtin_fmaf(d, (float)((u1 >> 16) & 0xffu), c), __builtin_fmaf(d, (float)(u1 >> 24), c)));
  }
}

// The same dequant split into a prelude and four quarter tasks (one bf16/fp16 pair
// each), so the work can be spread one task per MFMA.  Quarter order matches
// dequant_word: pairs (0,1), (2,3), (4,5), (6,7) of the word.
template <int QT>
struct WordTmp {
  uint32_t u0, u1;
  float a, c;
};

template <int QT, int kk>
__device__ __forceinline__ void word_prelude(const Raw<QT>& r, const Scales<QT>& s, int q, uint32_t nib,
                                             WordTmp<QT>& t) {
  if constexpr (QT == QT_Q4_K) {
    uint32_t w = r.q[kk];
    pin(w);
    t.u0 = w & nib;
    t.u1 = (w >> 4) & nib;
    t.a = s.a[q];
    t.c = s.b[q];
  } else if constexpr (QT == QT_Q6_K) {
    uint32_t lw = r.ql[kk], hv = r.qh[kk >> 1];
    pin(lw);
    pin(hv);
    t.u0 = lw;
    t.u1 = hv;
    t.a = (kk < 2) ? s.a[q] : s.b[q];
    t.c = -32.f * t.a;
  } else {
    uint32_t w0 = kk < 2 ? r.a[2 * kk] : r.b[2 * kk - 4];
    uint32_t w1 = kk < 2 ? r.a[2 * kk + 1] : r.b[2 * kk - 3];
    pin(w0);
    pin(w1);
    t.u0 = w0 ^ 0x80808080u;
    t.u1 = w1 ^ 0x80808080u;
    t.a = f16_bits_to_f32(r.d & 0xffffu);
    t.c = -128.f * t.a;
  }
}

template <int QT, int XT, int kk, int qq>
__device__ __forceinline__ uint32_t word_quarter(const WordTmp<QT>& t, uint32_t nib) {
  if constexpr (QT == QT_Q4_K) {
    // u0 bytes: weights 0, 4, 1, 5; u1 bytes: 2, 6, 3, 7
    const uint32_t v = (qq & 1) ? t.u1 : t.u0;
    const int sh = (qq & 2) ? 8 : 0;
    return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                     __builtin_fmaf(t.a, (float)((v >> (16 + sh)) & 0xffu), t.c));
  } else if constexpr (QT == QT_Q6_K) {
    constexpr int rs = 8 * (kk & 1) + 2 * qq - 4;
    const uint32_t hs = rs >= 0 ? (t.u1 >> rs) : (t.u1 << (-rs));
    const uint32_t v = ((t.u0 >> (4 * qq)) & (nib & 0x000F000Fu)) | (hs & 0x00300030u);
    return pack2<XT>(__builtin_fmaf(t.a, (float)(v & 0xffu), t.c), __builtin_fmaf(t.a, (float)((v >> 16) & 0xffu), t.c));
  } else {
    const uint32_t v = (qq < 2) ? t.u0 : t.u1;
    const int sh = (qq & 1) ? 16 : 0;
    return pack2<XT>(__builtin_fmaf(t.a, (float)((v >> sh) & 0xffu), t.c),
                     __builtin_fmaf(t.a, (float)((v >> (sh + 8)) & 0xffu), t.c));
  }
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

// Compile-time loop: fn(integral_constant<int, i>) for i = 0 .. N-1, fully expanded.
template <typename Fn, int... I>
__device__ __forceinline__ void sfor_impl(Fn&& fn, std::integer_sequence<int, I...>) {
  (fn(std::integral_constant<int, I>()), ...);
}
template <int N, typename Fn>
__device__ __forceinline__ void sfor(Fn&& fn) {
  sfor_impl(fn, std::make_integer_sequence<int, N>());
}

#define SCHED_MFMA(n) __builtin_amdgcn_sched_group_barrier(0x008, n, 0)
#define SCHED_VALU(n) __builtin_amdgcn_sched_group_barrier(0x002, n, 0)
#define SCHED_DSR(n) __builtin_amdgcn_sched_group_barrier(0x100, n, 0)
#define SCHED_VMEM(n) __builtin_amdgcn_sched_group_barrier(0x020, n, 0)
#define SCHED_DSW(n) __builtin_amdgcn_sched_group_barrier(0x200, n, 0)

template <int QT, int XT>
__global__ __launch_bounds__(256, 1) void qgemm_tile_kernel(TileParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Tile order: each XCD (workgroup id % 8) takes a contiguous run of tiles in M-major
  // order, so the activation panel it walks N with stays in its L2.
  const int ntiles = p.tiles_m * p.tiles_n;
  const int b = blockIdx.x;
  int t = b;
  if ((ntiles & 7) == 0) t = (b & 7) * (ntiles >> 3) + (b >> 3);
  const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
  const int m0 = tm * TM, n0 = tn * TN;
  const int M = p.M, N = p.N, K = p.K;
  const int nsub = K >> 5, nsb = K >> 8;
  const int nkt = (K + TK - 1) / TK;

  auto srsrc = [](const void* ptr, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)ptr;
    i32x4_t r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
  };
  i32x4_t R[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) R[i] = srsrc(p.P[i] ? p.P[i] : (const uint8_t*)p.x, p.psize[i]);

  // --- activations: LDS DMA.  Wave w fills slot blocks 8w .. 8w+7 of a stage (1 KiB =
  // 8 rows each); lane l of block b brings row 8b + l/8, global chunk (l%8) ^ (l/8), to
  // chunk position l%8.  Rows past M read zeros.
  uint32_t a_voff[8];
  const int a_pos = lane & 7;
  const int a_c = a_pos ^ (lane >> 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 8 * (8 * wave + i) + (lane >> 3);
    a_voff[i] = (m0 + r < M) ? ((uint32_t)(m0 + r) * (uint32_t)K + (uint32_t)a_c * 8u) * 2u : OOB;
  }
  const int ktail = K % TK;  // only Q8_0 can end on a half step (32 of 64)
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
  const i32x4_t rx = srsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  // Always eight DMA instructions per wavefront and step (steps past the end read
  // zeros into a stage nobody reads), so the wait counts below are exact.
  auto issue_a = [&](int kt) {
    const bool live = kt < nkt;
    const bool cut = ktail != 0 && kt == nkt - 1 && a_c * 8 >= ktail;
    const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane(kt * (TK * 2));
    const uint32_t dst = lds_base + (uint32_t)((kt & (NSTAGE - 1)) * A_STAGE + wave * 8 * 1024);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t vo = (live && !cut) ? a_voff[i] : OOB;
      const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane((int)(dst + i * 1024));
      asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                   :
                   : "v"(vo), "s"(rx), "s"(soff), "s"(m0v)
                   : "memory", "m0");
    }
  };

  // --- weight rows of this lane: n0 + 64*wave + (lane & 31) + 32j, sub-block half h
  const int h = lane >> 5;
  uint32_t row_sub[2], row_sb[2];
  bool rok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 64 * wave + (lane & 31) + 32 * j;
    rok[j] = n < N;
    row_sub[j] = rok[j] ? (uint32_t)n * (uint32_t)nsub : 0u;
    row_sb[j] = rok[j] ? (uint32_t)n * (uint32_t)nsb : 0u;
  }

  // Ring of raw sub-blocks: step k lives in slot k % PD.  Every index below is static
  // (the K loop is unrolled by four, PD = 4), so the ring stays in registers.
  Raw<QT> raw[PD][2];
  Hdr<QT> hdr[2];
  Scales<QT> sc[2];
  auto issue_raw = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    const int sb = 2 * kt + h;
    const bool in = kt < nkt && sb < nsub;
#pragma unroll
    for (int j = 0; j < 2; ++j) load_raw<QT>(R, row_sub[j], sb, in && rok[j], raw[slot][j]);
    if constexpr (QT != QT_Q8_0 && slot == 0) {
      // first step of a super-block (K-quant steps come in whole super-blocks of four)
#pragma unroll
      for (int j = 0; j < 2; ++j) load_hdr<QT>(R, row_sb[j], kt >> 2, in && rok[j], hdr[j]);
    }
  };

  // VMEM instructions issue_raw issues for the step with ring slot s.
  constexpr int RB = raw_loads<QT>(), RH = hdr_loads<QT>();
  auto rops = [](int slot) constexpr { return RB + (slot == 0 ? RH : 0); };
  // Wait until raw slot s (and its header) is in, pinning its registers.
  auto wait_raw = [&](auto SLOT, auto N) {
    constexpr int slot = decltype(SLOT)::value, n = decltype(N)::value;
    static_assert(n < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
    raw[slot][0].pin_all();
    raw[slot][1].pin_all();
    if constexpr (QT != QT_Q8_0 && slot == 0) {
      hdr[0].pin_all();
      hdr[1].pin_all();
    }
  };

  // B fragments of the current step, [j][kk]; slot kk is replaced by the next step's
  // word kk right after the MFMAs of slice kk have been issued.
  uint4 bf[2][4];
  auto decode_step = [&](auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;  // == step % 4 == sub-block quarter
    if constexpr (QT != QT_Q8_0 && slot == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) decode_hdr<QT>(hdr[j], h, sc[j]);
    }
  };
  auto dequant_piece = [&](auto SLOT, auto KK, auto J) {
    constexpr int slot = decltype(SLOT)::value, kk = decltype(KK)::value, j = decltype(J)::value;
    bf[j][kk] = dequant_word<QT, XT, kk>(raw[slot][j], sc[j], slot, p.nib);
  };
  auto dequant_slice = [&](auto SLOT, auto KK) {
    dequant_piece(SLOT, KK, std::integral_constant<int, 0>());
    dequant_piece(SLOT, KK, std::integral_constant<int, 1>());
  };

  f32x16_t acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // A fragment f = 8kk + i of a step: rows 32i + lane%32, K chunk 4h + kk, at its
  // swizzled position.  Fragments stream through a ring of four registers, three ahead.
  const int fr = lane & 31;
  auto read_a = [&](int stage, int f) -> uint4 {
    const int kk = f >> 3, i = f & 7;
    const int r = 32 * i + fr;
    const int c = (4 * h + kk) ^ (r & 7);
    return *(const uint4*)(lds + stage * A_STAGE + r * 128 + c * 16);
  };

  // ---- prologue: the issue order of steps -3 .. -1 (DMA of step s+3, raw loads of step
  // s+4), preceded by the raw loads of step 0, so every wait below is the steady-state one
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  issue_raw(0, I0());
  issue_a(0);
  issue_raw(1, I1());
  issue_a(1);
  issue_raw(2, I2());
  issue_a(2);
  issue_raw(3, I3());
  wait_raw(I0(), std::integral_constant<int, 24 + rops(1) + rops(2) + rops(3)>());
  decode_step(std::integral_constant<int, 0>());
  dequant_slice(std::integral_constant<int, 0>(), std::integral_constant<int, 0>());
  dequant_slice(std::integral_constant<int, 0>(), std::integral_constant<int, 1>());
  dequant_slice(std::integral_constant<int, 0>(), std::integral_constant<int, 2>());
  dequant_slice(std::integral_constant<int, 0>(), std::integral_constant<int, 3>());
  // stage 0 complete (every wavefront's DMA of it) before its first fragments are read
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(16 + rops(1) + rops(2) + rops(3)) : "memory");
  __syncthreads();
  // Activation fragments stream through a ring of four registers, three ahead, across
  // step boundaries.
  uint4 ring[4];
  ring[0] = read_a(0, 0);
  ring[1] = read_a(0, 1);
  ring[2] = read_a(0, 2);

  // Step kt (u = kt % 4), activations from LDS stage u.  64 MFMA slots, slot m = 2f + j
  // (fragment f = 8kk + i, weight column block j); program order is issue order
  // (sched_barrier fences).  Per slot: fragment f+3's LDS read (from the next step's
  // stage past f = 28), the MFMA, and at most one small VALU task for step kt+1: in slice
  // kk, slot t = m % 16 does the prelude (t = 0 / 8) or a quarter (t = 1..4 / 9..12) of
  // word kk of weight row 0 / 1; the finished words replace bf[.][kk] after the slice's
  // last MFMA.  Half way (slot 32) the wavefront waits for its DMA of stage kt+1 and
  // joins the barrier: then stage kt+1 is complete and stage kt-1 free, so the DMA of
  // step kt+3 goes into it.  The raw weights of step kt+4 are loaded at the end, into the
  // ring slot step kt just used.
  auto step = [&](int kt, auto U) {
    constexpr int u = decltype(U)::value;
    constexpr int un = (u + 1) & 3;
    using SN = std::integral_constant<int, un>;
    WordTmp<QT> wt[2];
    uint32_t nw[2][4];
    sfor<64>([&](auto MS) {
      constexpr int m = decltype(MS)::value, f = m >> 1, j = m & 1, kk = f >> 3, i = f & 7, t = m & 15;
      using KK = std::integral_constant<int, kk>;
      if constexpr (j == 0 && f + 3 < 32) ring[(f + 3) & 3] = read_a(u, f + 3);
      if constexpr (j == 0 && f + 3 >= 32) ring[(f + 3) & 3] = read_a(un, f + 3 - 32);
      acc[i][j] = mfma<XT>(bf[j][kk], ring[f & 3], acc[i][j]);
      if constexpr (m == 0) {
        // raw slot un was loaded at the end of step kt-3; since then: two steps of DMA +
        // raw loads
        wait_raw(SN(), std::integral_constant<int, 16 + rops((u + 2) & 3) + rops((u + 3) & 3)>());
        decode_step(SN());
      }
      if constexpr (m == 31) {
        // this wavefront's DMA of stage kt+1 was issued half way through step kt-2;
        // after it: the raw loads of kt+2, the DMA of stage kt+2, the raw loads of kt+3
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 + rops((u + 2) & 3) + rops((u + 3) & 3)) : "memory");
        __syncthreads();
        issue_a(kt + NSTAGE - 1);
      }
      if constexpr (t == 0 || t == 8) {
        constexpr int jw = t >> 3;
        word_prelude<QT, kk>(raw[un][jw], sc[jw], un, p.nib, wt[jw]);
      }
      if constexpr ((t >= 1 && t <= 4) || (t >= 9 && t <= 12)) {
        constexpr int jw = t >> 3, qq = (t & 7) - 1;
        nw[jw][qq] = word_quarter<QT, XT, kk, qq>(wt[jw], p.nib);
      }
      if constexpr (t == 15) {
        bf[0][kk] = make_uint4(nw[0][0], nw[0][1], nw[0][2], nw[0][3]);
        bf[1][kk] = make_uint4(nw[1][0], nw[1][1], nw[1][2], nw[1][3]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    issue_raw(kt + PD, U);
  };

  for (int kt = 0; kt < nkt; kt += 4) {
    step(kt, std::integral_constant<int, 0>());
    if (kt + 1 < nkt) step(kt + 1, std::integral_constant<int, 1>());
    if (kt + 2 < nkt) step(kt + 2, std::integral_constant<int, 2>());
    if (kt + 3 < nkt) step(kt + 3, std::integral_constant<int, 3>());
  }

  // no DMA may still be landing in LDS when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue.  The MFMAs take the weights as the first operand, so accumulator v
  // of tile (i, j) holds Y[m][n] for m = m0 + 32i + lane%32 and n = n0 + 64w + 32j +
  // 8(v/4) + 4(lane/32) + v%4: four consecutive columns per lane, stored as one 8-byte
  // (16-bit types) or 16-byte (fp32) write.
  const int nb = n0 + 64 * wave + 4 * (lane >> 5);
  float bv[2][4][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = nb + 32 * j + 8 * q + e;
        bv[j][q][e] = (p.bias && n < N) ? load_scalar(p.bias, p.bias_dtype, n) : 0.f;
      }
  const bool vec_ok = (N & 3) == 0;
  auto epi = [&](auto YTC) {
    constexpr int yt = decltype(YTC)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = m0 + 32 * i + (lane & 31);
      if (m >= M) continue;
      const size_t rowbase = (size_t)m * (size_t)N;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = nb + 32 * j + 8 * q;
          const float v0 = acc[i][j][4 * q + 0] + bv[j][q][0], v1 = acc[i][j][4 * q + 1] + bv[j][q][1];
          const float v2 = acc[i][j][4 * q + 2] + bv[j][q][2], v3 = acc[i][j][4 * q + 3] + bv[j][q][3];
          if (vec_ok && n + 3 < N) {
            if constexpr (yt == DT_F32) {
              *(float4*)((float*)p.y + rowbase + n) = make_float4(v0, v1, v2, v3);
            } else if constexpr (yt == DT_BF16) {
              *(uint2*)((uint16_t*)p.y + rowbase + n) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
            } else {
              *(uint2*)((uint16_t*)p.y + rowbase + n) = make_uint2(pack2<X_F16>(v0, v1), pack2<X_F16>(v2, v3));
            }
          } else {
            const float vv[4] = {v0, v1, v2, v3};
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < N) store_scalar(p.y, yt, rowbase + n + e, vv[e]);
          }
        }
      }
    }
  };
  if (p.y_dtype == DT_BF16) epi(std::integral_constant<int, DT_BF16>());
  else if (p.y_dtype == DT_F16) epi(std::integral_constant<int, DT_F16>());
  else epi(std::integral_constant<int, DT_F32>());
}

template <int QT, int XT>
hipError_t launch_tile_t(const TileParams& tp, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void*)qgemm_tile_kernel<QT, XT>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, TILE_LDS);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  qgemm_tile_kernel<QT, XT><<<dim3((unsigned)(tp.tiles_m * tp.tiles_n)), dim3(256), TILE_LDS, s>>>(tp);
  return hipGetLastError();
}

}  // namespace

bool tile_fits(const RunArgs& a) {
  for (int i = 0; i < a.L.nplanes; ++i)
    if (a.L.size[i] >= (1u << 31)) return false;
  return (size_t)a.M * a.L.K * 2 < (1u << 31);
}

hipError_t launch_tile(const RunArgs& a, hipStream_t s) {
  TileParams tp;
  const PlanePtrs P = plane_ptrs(a.L, a.packed);
  for (int i = 0; i < 4; ++i) {
    tp.P[i] = P.p[i];
    tp.psize[i] = i < a.L.nplanes ? (uint32_t)a.L.size[i] : 0u;
  }
  tp.x = a.x;
  tp.bias = a.bias;
  tp.y = a.y;
  tp.M = a.M;
  tp.N = a.L.N;
  tp.K = a.L.K;
  tp.bias_dtype = a.bias_dtype;
  tp.y_dtype = a.y_dtype;
  tp.tiles_m = (a.M + TM - 1) / TM;
  tp.tiles_n = (a.L.N + TN - 1) / TN;
  tp.nib = 0x0F0F0F0Fu;
  const bool f16 = a.x_dtype == DT_F16;
  switch (a.L.qtype) {
    case QT_Q4_K: return f16 ? launch_tile_t<QT_Q4_K, X_F16>(tp, s) : launch_tile_t<QT_Q4_K, X_BF16>(tp, s);
    case QT_Q6_K: return f16 ? launch_tile_t<QT_Q6_K, X_F16>(tp, s) : launch_tile_t<QT_Q6_K, X_BF16>(tp, s);
    default: return f16 ? launch_tile_t<QT_Q8_0, X_F16>(tp, s) : launch_tile_t<QT_Q8_0, X_BF16>(tp, s);
  }
}

}  // namespace mlxr
