// Kernel (b): prefill GEMM, Y[M,N] = X[M,K] . W[N,K]^T (+ bias) on 32x32x16 MFMA.
//
// Replaces the large-M use of core/kernels/metal/q_gemm_dequant.metal:338-486 in the
// reference (tile loop :374-464: X tile to shared memory, W tile dequantized, fp32
// accumulation, bias + store :467-485).
//
// Tile: BM (256 or 128) rows of M x 256 columns of N per workgroup, K in steps of 64,
// four wavefronts; wavefront w owns the BM x 64 slab of output columns [64w, 64w + 64) as
// MI x 2 accumulators of the 32x32x16 MFMA (MI = BM/32; in AGPRs).  The 128-row tile
// doubles the tile count for shapes whose 256-row tiles would leave CUs idle.
//
//  * Activations (shared by the four wavefronts) go HBM -> LDS by buffer_load ... lds
//    (no VGPR staging), four stages, three steps ahead.  A BM x 64 stage has 128-byte
//    rows; the 16-byte chunk c of row r is stored at position c ^ swz(r), so the
//    fragment reads of sixteen consecutive rows hit sixteen different 16-byte bank groups.
//    The DMA is issued from inline assembly, so the compiler (which would otherwise wait
//    for every outstanding load before each LDS read) leaves the stage waits to the
//    exact vmcnt values computed from the fixed issue order; the weight loads are
//    ordinary buffer loads the compiler waits for itself.
//  * Weights never pass through LDS.  K is permuted inside each 64-step so that in MFMA
//    kk (0..3) lane half h supplies K positions 32h + 8kk .. +7 for both operands: lane
//    (n, h) then owns exactly sub-block h of the step for its weight rows n and n + 32,
//    dequantizes those 32 weights in registers and uses word kk of the result as the B
//    fragment of MFMA kk.  Per-super-block header work (d, dmin, six-bit scales) is done
//    once per four steps.  The raw sub-blocks are loaded eight steps ahead (Q8_0: four,
//    for registers); the dequant of step k+1 is spread over the MFMAs of step k, a few
//    VALU ops per MFMA.
//  * One barrier per step, half way through it: the next stage is then complete and the
//    previous one free for the DMA three steps ahead, which goes out over the second half
//    of the step (one instruction every third MFMA slot).
//  * The MFMAs take the weights as the first operand, so each lane's accumulators hold
//    four consecutive output columns; the epilogue turns each 32 x 64 block around through
//    LDS and stores whole row segments (8 or 16 bytes per lane).
//
// The dequantized values are the exact GGUF fp32 weights rounded to nearest-even bf16
// (fp16 for fp16 activations, which use the fp16 MFMA), from the routines of
// qgemm_wdequant.h, which also back mlxr_qgemm_dequant: its bit-exact tests cover them.
#pragma once
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
namespace tile {


typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

constexpr int TN = 256, TK = 64;
constexpr int NSTAGE = 4;              // activation stages (DMA three steps ahead)
// Raw weight prefetch distance (steps; a multiple of four): eight where the ring fits
// the register budget beside the accumulators, four for Q8_0's larger sub-blocks.
template <int QT>
constexpr int prefetch_steps() { return QT == QT_Q8_0 ? 4 : 8; }

// One weight of a launch.  A launch covers up to MAX_TG weights that share X, K and the
// quant type (grouped projections): their tile columns follow each other.
constexpr int MAX_TG = 4;
struct TileGroup {
  const uint8_t* P[4];
  uint32_t psize[4];
  void* y;
  const void* bias;
  int N;
  int ldy;   // row stride of y in elements
  int tn0;   // first tile column of this weight in the launch
  int col0;  // first column of this weight in a split-K workspace row
  int bias_dtype, y_dtype;
};
struct TileParams {
  const void* x;
  int M, K;
  int tiles_m, tiles_n;  // tiles_n: over all weights of the launch
  int kps;          // K steps per split (multiple of 4); the grid is tiles x splits
  float* ws;        // split-K: fp32 partials, split s at ws + s * ws_split, rows of ws_ld
  size_t ws_split;  // elements per split plane
  int ws_ld;        // workspace row stride (the launch's total N)
  uint32_t nib;     // 0x0F0F0F0F, passed at run time (keeps the byte converts)
  int ngroups;
  // SwiGLU (gate = g[0], up = g[1], same shape): a tile is 128 output columns; wavefront
  // w's two 32-column accumulator blocks are gate and up of the same 32 columns, and the
  // epilogue stores swish(gate) * up into g[0].y (with ws: the two weights' partials side
  // by side, columns n and N + n of rows of ws_ld = 2N)
  int swiglu;
  TileGroup g[MAX_TG];
};

// LDS position of 16-byte chunk c of activation row r in a stage: c ^ swz(r).  Fragment
// reads take rows r .. r+15 of one chunk column per 16-lane phase; with 128-byte rows
// and 64 four-byte banks, row r lands in bank group 8(r & 1) + (c ^ swz(r)), so swz must
// be a bijection on the eight even and on the eight odd rows of an aligned group of 16.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

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

// SW: the SwiGLU variant (p.swiglu set; a separate instantiation, so the plain kernel's
// code and registers are those of the kernel without it).
template <int QT, int XT, int MI, bool SW>
__global__ __launch_bounds__(256, 1) void qgemm_tile_kernel(TileParams p) {
  constexpr int BM = 32 * MI;              // tile rows (M)
  constexpr int A_STAGE = BM * TK * 2;     // bytes per activation stage
  constexpr int NF = 4 * MI;               // A fragments per step
  constexpr int NSLOT = 2 * NF;            // MFMAs per step
  constexpr int SPS = NSLOT / 4;           // MFMA slots per slice kk
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Tile order: each XCD (workgroup id % 8) takes a contiguous run of the launch's
  // (K split, tile) pairs in split-major, then M-major order, so the activation panels it
  // walks N with (one per split and tile row) stay in its L2: with K split eight ways over
  // 32 tiles each XCD holds the panel of one split instead of all eight.
  const int ntiles = p.tiles_m * p.tiles_n;
  const int nb = (int)gridDim.x;
  const int f = (nb & 7) == 0 ? ((int)blockIdx.x & 7) * (nb >> 3) + ((int)blockIdx.x >> 3) : (int)blockIdx.x;
  const int split = f / ntiles;
  const int t = f - split * ntiles;
  const int tm = t / p.tiles_n, tn = t - tm * p.tiles_n;
  // the weight this tile column belongs to (scalar search), its fields selected with
  // static kernel-argument offsets so every load is issued at once
  constexpr bool sw = SW;
  int gi = 0;
#pragma unroll
  for (int g = 1; g < MAX_TG; ++g)
    if (g < p.ngroups && tn >= p.g[g].tn0) gi = g;
  if constexpr (sw) gi = 0;  // gate; block 1 reads p.g[1] (up) directly
  TileGroup G = p.g[0];
#pragma unroll
  for (int g = 1; g < MAX_TG; ++g) {
    const TileGroup& H = p.g[g];
    const bool sel = g == gi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      G.P[i] = sel ? H.P[i] : G.P[i];
      G.psize[i] = sel ? H.psize[i] : G.psize[i];
    }
    G.y = sel ? H.y : G.y;
    G.bias = sel ? H.bias : G.bias;
    G.N = sel ? H.N : G.N;
    G.ldy = sel ? H.ldy : G.ldy;
    G.tn0 = sel ? H.tn0 : G.tn0;
    G.col0 = sel ? H.col0 : G.col0;
    G.bias_dtype = sel ? H.bias_dtype : G.bias_dtype;
    G.y_dtype = sel ? H.y_dtype : G.y_dtype;
  }
  // n0: the tile's first column of weight G; wc: this wavefront's columns within it (64;
  // SwiGLU: 32 of gate and the same 32 of up)
  const int m0 = tm * BM, n0 = sw ? tn * (TN / 2) : (tn - G.tn0) * TN;
  const int wc = sw ? 32 * wave : 64 * wave;
  const int M = p.M, N = G.N, K = p.K;
  const int nsub = K >> 5, nsb = K >> 8;
  const int nkt = (K + TK - 1) / TK;
  // this workgroup's K steps [kt0, kend): kt0 is a multiple of four (super-block start)
  const int kt0 = split * p.kps, kend = min(nkt, kt0 + p.kps);

  // weight of accumulator block j (SwiGLU: block 1 reads the up weight)
  rsrc_t R[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    R[0][i] = make_rsrc(G.P[i] ? G.P[i] : (const uint8_t*)p.x, G.psize[i]);
    if constexpr (sw) R[1][i] = make_rsrc(p.g[1].P[i] ? p.g[1].P[i] : (const uint8_t*)p.x, p.g[1].psize[i]);
    else R[1][i] = R[0][i];
  }

  // --- activations: LDS DMA.  Wave w fills slot blocks MI*w .. MI*w+MI-1 of a stage
  // (1 KiB = 8 rows each); lane l of block b brings row 8b + l/8, global chunk
  // (l%8) ^ swz(row), to chunk position l%8.  Rows past M read zeros.
  uint32_t a_voff[MI];
  bool a_hi[MI];  // this lane's chunk is in the upper half of the step (K offset >= 32)
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = 8 * (MI * wave + i) + (lane >> 3);
    const int a_c = (lane & 7) ^ swz(r);
    a_hi[i] = a_c >= 4;
    a_voff[i] = (m0 + r < M) ? ((uint32_t)(m0 + r) * (uint32_t)K + (uint32_t)a_c * 8u) * 2u : OOB;
  }
  const int ktail = K % TK;  // the 32-weight block types can end on a half step (32 of 64)
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
  const i32x4_t rx = make_srsrc(p.x, (uint32_t)M * (uint32_t)K * 2u);
  // Always MI DMA instructions per wavefront and step (steps past the end read zeros
  // into a stage nobody reads), so the wait counts below are exact.
  auto issue_a1 = [&](int kt, int i) {
    const bool live = kt < kend;
    const bool last_half = ktail != 0 && kt == nkt - 1;  // ktail is 32 here
    const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane(kt * (TK * 2));
    const uint32_t dst = lds_base + (uint32_t)((kt & (NSTAGE - 1)) * A_STAGE + wave * MI * 1024);
    const uint32_t vo = (live && !(last_half && a_hi[i])) ? a_voff[i] : OOB;
    const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane((int)(dst + i * 1024));
    // M0 holds the LDS destination; nothing else in this kernel uses M0 (DS
    // instructions on gfx9+ do not), so clobbering it is safe here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(vo), "s"(rx), "s"(soff), "s"(m0v)
                 : "memory", "m0");
#pragma clang diagnostic pop
  };
  auto issue_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < MI; ++i) issue_a1(kt, i);
  };

  // --- weight rows of this lane: n0 + wc + (lane & 31) + 32j (SwiGLU: n0 + wc + (lane &
  // 31) of gate for j = 0 and of up for j = 1), sub-block half h
  const int h = lane >> 5;
  uint32_t row_sub[2], row_sb[2];
  bool rok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wc + (lane & 31) + (sw ? 0 : 32 * j);
    rok[j] = n < N;
    row_sub[j] = rok[j] ? (uint32_t)n * (uint32_t)nsub : 0u;
    row_sb[j] = rok[j] ? (uint32_t)n * (uint32_t)nsb : 0u;
  }

  // Ring of raw sub-blocks: step kt0 + k lives in slot k % PD.  Every index below is
  // static (the K loop is unrolled by PD), so the ring stays in registers.  K-quant
  // super-block headers ride with the first step of their super-block (slots 0, 4).
  constexpr int PD = prefetch_steps<QT>();
  Raw<QT> raw[PD][2];
  Hdr<QT> hdr[PD / 4][2];
  Scales<QT> sc[2];
  auto issue_raw = [&](int kt, auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;
    const int sb = 2 * kt + h;
    const bool in = kt < kend && sb < nsub;
#pragma unroll
    for (int j = 0; j < 2; ++j) load_raw<QT>(R[j], row_sub[j], sb, in && rok[j], raw[slot][j]);
    if constexpr (is_kquant(QT) && slot % 4 == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) load_hdr<QT>(R[j], row_sb[j], kt >> 2, in && rok[j], hdr[slot / 4][j]);
    }
  };

  // VMEM instructions issue_raw issues for the step with ring slot s.
  constexpr int RB = 2 * raw_loads<QT>(), RH = 2 * hdr_loads<QT>();  // two weight rows
  auto rops = [](int slot) constexpr { return RB + (slot % 4 == 0 ? RH : 0); };
  // B fragments of the current step, [j][kk]; word kk is replaced by the next step's
  // right after the MFMAs of slice kk have been issued.
  uint4 bf[2][4];
  auto decode_step = [&](auto SLOT) {
    constexpr int slot = decltype(SLOT)::value;  // step % PD; slot % 4 = sub-block quarter
    if constexpr (is_kquant(QT) && slot % 4 == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) decode_hdr<QT>(hdr[slot / 4][j], h, sc[j]);
    }
  };

  f32x16_t acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // A fragment f = MI*kk + i of a step: rows 32i + lane%32, K chunk 4h + kk, at its
  // swizzled position.
  const int fr = lane & 31;
  auto read_a = [&](int stage, int f) -> uint4 {
    const int kk = f / MI, i = f % MI;
    const int r = 32 * i + fr;
    const int c = (4 * h + kk) ^ swz(r);
    return *(const uint4*)(lds + stage * A_STAGE + r * 128 + c * 16);
  };

  // ---- prologue.  Steady state issues, in step s: the DMA of stage s+3 over the second
  // half and the raw loads of step s+PD at the end.  The prologue issues raw loads of steps
  // 0 .. PD-3, the DMAs of stages 0 and 1, raw PD-2, DMA 2, raw PD-1: after the DMA of
  // any stage k, exactly raw(k+PD-2), DMA(k+1), raw(k+PD-1) follow, as in the loop.
  sfor<PD - 2>([&](auto S_) {
    constexpr int s_ = decltype(S_)::value;
    issue_raw(kt0 + s_, std::integral_constant<int, s_>());
  });
  issue_a(kt0);
  issue_a(kt0 + 1);
  issue_raw(kt0 + PD - 2, std::integral_constant<int, PD - 2>());
  issue_a(kt0 + 2);
  issue_raw(kt0 + PD - 1, std::integral_constant<int, PD - 1>());
  decode_step(std::integral_constant<int, 0>());
  sfor<4>([&](auto KK) {
    constexpr int kk = decltype(KK)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) bf[j][kk] = dequant_word<QT, XT, kk, true>(raw[0][j], sc[j], 0, p.nib);
  });
  // stage 0 complete (every wavefront's DMA of it) before its first fragments are read
  vm_wait<2 * MI + rops(PD - 2) + rops(PD - 1)>();
  __syncthreads();
  // Activation fragments stream through a ring of four registers, three ahead, across
  // step boundaries.
  // reads from the next step's stage (fragments NF-3 .. NF-1 of a step) must come after
  // the mid-step barrier (MFMA slot NSLOT/2 - 1, fragment NF/2 - 1) that completes it
  static_assert(NF - 3 > NF / 2 - 1, "fragment lookahead overtakes the stage barrier");
  uint4 ring[4];
  ring[0] = read_a(0, 0);
  ring[1] = read_a(0, 1);
  ring[2] = read_a(0, 2);

  // Step kt (u = kt % 4), activations from LDS stage u.  NSLOT MFMA slots, slot m =
  // 2f + j (fragment f = MI*kk + i, weight column block j); program order is issue order
  // (sched_barrier fences).  Per slot: fragment f+3's LDS read (from the next step's
  // stage near the end), the MFMA, and a share of step kt+1's dequant: per slice kk ten
  // tasks (prelude and four quarters of word kk for weight rows 0 and 1) spread over
  // the slice's SPS slots; the finished words replace bf[.][kk] after the slice's last
  // MFMA.  Half way the wavefront waits for its DMA of stage kt+1 and joins the
  // barrier: then stage kt+1 is complete and stage kt-1 free, so the DMA of step kt+3
  // goes into it, over the second half.  The raw weights of step kt+PD are loaded at the
  // end, into the ring slot step kt just used.
  auto step = [&](int kt, auto U) {
    constexpr int u = decltype(U)::value;      // (kt - kt0) % PD; LDS stage u % 4
    constexpr int un = (u + 1) % PD;
    using SN = std::integral_constant<int, un>;
    WordTmp<QT> wt[2];
    uint32_t nw[2][4];
    sfor<NSLOT>([&](auto MS) {
      constexpr int m = decltype(MS)::value, f = m >> 1, j = m & 1, kk = f / MI, i = f % MI;
      constexpr int ts = m - kk * SPS;  // slot within the slice
      if constexpr (j == 0 && f + 3 < NF) ring[(f + 3) & 3] = read_a(u & 3, f + 3);
      if constexpr (j == 0 && f + 3 >= NF) ring[(f + 3) & 3] = read_a(un & 3, f + 3 - NF);
      acc[i][j] = mfma<XT>(bf[j][kk], ring[f & 3], acc[i][j]);
      if constexpr (m == 0) decode_step(SN());
      if constexpr (m == NSLOT / 2 - 1) {
        // this wavefront's DMA of stage kt+1 was issued half way through step kt-2;
        // after it: the raw loads of kt+PD-2, the DMA of stage kt+2, the raw loads of
        // kt+PD-1
        vm_wait<MI + rops((u + PD - 2) % PD) + rops((u + PD - 1) % PD)>();
        __syncthreads();
      }
      // the DMA of step kt+3, one instruction every third slot of the second half (issued
      // all at once right after the barrier, by all four wavefronts, they were 2-4% slower)
      if constexpr (m >= NSLOT / 2 && (m - NSLOT / 2) % 3 == 0 && (m - NSLOT / 2) / 3 < MI)
        issue_a1(kt + NSTAGE - 1, (m - NSLOT / 2) / 3);
      // tasks k = 0..9 of the slice (0: prelude row 0, 1-4: its quarters, 5: prelude
      // row 1, 6-9: its quarters); task k runs in slot (k * SPS) / 10
      sfor<10>([&](auto TK_) {
        constexpr int k = decltype(TK_)::value;
        if constexpr ((k * SPS) / 10 == ts) {
          constexpr int jw = k / 5, kq = k % 5;
          if constexpr (kq == 0) word_prelude<QT, kk, true>(raw[un][jw], sc[jw], un & 3, p.nib, wt[jw]);
          else nw[jw][kq - 1] = word_quarter<QT, XT, kk, kq - 1, true>(wt[jw], p.nib);
        }
      });
      if constexpr (ts == SPS - 1) {
        bf[0][kk] = make_uint4(nw[0][0], nw[0][1], nw[0][2], nw[0][3]);
        bf[1][kk] = make_uint4(nw[1][0], nw[1][1], nw[1][2], nw[1][3]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    issue_raw(kt + PD, U);
  };

  // Whole rings of PD steps, unconditionally: steps past kend load nothing (out-of-range
  // offsets: zero activations and zero weights, so they add zeros) and the loop body is one
  // straight-line path.  (With the steps past kend skipped by branches inside the body, the
  // compiler could not carry its load wait counts across the back edge and drained every
  // load, the prefetches included, at each trip.)
  for (int kt = kt0; kt < kend; kt += PD) {
    sfor<PD>([&](auto U_) {
      constexpr int u = decltype(U_)::value;
      step(kt + u, std::integral_constant<int, u>());
    });
  }

  // no DMA may still be landing in LDS when the workgroup ends
  vm_wait<0>();

  // ---- epilogue, through LDS (the activation stages are free once every wavefront is
  // past its last fragment read).  Accumulator v of tile (i, j) holds Y[m][n] for
  // m = m0 + 32i + lane%32, n = n0 + 64w + 32j + 8(v/4) + 4(lane/32) + v%4.  Per i, a
  // wavefront parks its 32 x 64 block in its own LDS area (row stride 68 floats) and
  // reads it back row-major: lane l takes columns 4(l%16) .. +3 of rows l/16 + 4r
  // (r = 0..7), so sixteen lanes cover 64 contiguous columns of one row and every store
  // is a whole row segment.  Split-K partials go to the workspace as fp32 without bias.
  __syncthreads();
  constexpr int EP_LD = 68;
  float* ep = (float*)lds + wave * (32 * EP_LD);
  const int c4 = lane & 15;
  const int ncol = n0 + wc + 4 * c4;  // first of this lane's four columns
  // output rows: y's, or the workspace's (split plane, this weight's column range)
  const int ld = p.ws ? p.ws_ld : G.ldy;
  const int cb = p.ws ? G.col0 : 0;
  const bool vec_ok = (N & 3) == 0 && ((ld | cb) & 3) == 0 && ncol + 3 < N;
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (!p.ws && G.bias) {
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e] = ncol + e < N ? load_scalar(G.bias, G.bias_dtype, ncol + e) : 0.f;
  }
  // Take the bias values here, once: with their loads still pending at the row loops
  // below, the compiler waited for every outstanding memory operation, the previous
  // block's stores included, at the start of each of the MI blocks.
#pragma unroll
  for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(bv[e]));
  void* const out = p.ws ? (void*)(p.ws + (size_t)split * p.ws_split) : G.y;
  const int yt = p.ws ? DT_F32 : G.y_dtype;
  if constexpr (sw) {
    // SwiGLU (no biases): accumulator v of blocks (i, 0) and (i, 1) holds gate and up of
    // the same output, m = m0 + 32i + lane%32, n = n0 + 32w + 8(v/4) + 4(lane/32) + v%4.
    // Per i the wavefront parks the two 32 x 32 blocks in its LDS area and stores whole
    // row segments of swish(gate) * up (or, split, of both partials): lane l takes columns
    // 4(l%8) .. +3 of rows l/8 + 8r.
    const int c8 = lane & 7;
    const int hcol = n0 + wc + 4 * c8;
    const bool hvec = (N & 3) == 0 && hcol + 3 < N;
    sfor<MI>([&](auto I_) {
      constexpr int i = decltype(I_)::value;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cc = 8 * q + 4 * (lane >> 5);  // column of accumulators 4q .. 4q+3
        *(float4*)(ep + (lane & 31) * EP_LD + cc) =
            make_float4(acc[i][0][4 * q], acc[i][0][4 * q + 1], acc[i][0][4 * q + 2], acc[i][0][4 * q + 3]);
        *(float4*)(ep + (lane & 31) * EP_LD + 32 + cc) =
            make_float4(acc[i][1][4 * q], acc[i][1][4 * q + 1], acc[i][1][4 * q + 2], acc[i][1][4 * q + 3]);
      }
      __builtin_amdgcn_wave_barrier();
      // lane l: rows mb + 8r (r = 0..3), gate and up of its four columns; all reads first
      float4 g[4], u[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        g[r] = *(const float4*)(ep + (8 * r + (lane >> 3)) * EP_LD + 4 * c8);
        u[r] = *(const float4*)(ep + (8 * r + (lane >> 3)) * EP_LD + 32 + 4 * c8);
      }
      const int mb = m0 + 32 * i + (lane >> 3);
      const bool full = hvec && m0 + 32 * i + 32 <= M;
      if (p.ws) {  // split: gate and up partials to columns n and N + n of the workspace
        float* const w0 = p.ws + (size_t)split * p.ws_split + (size_t)mb * (size_t)p.ws_ld + hcol;
        const size_t rs = 8 * (size_t)p.ws_ld;
        if (full) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            *(float4*)(w0 + r * rs) = g[r];
            *(float4*)(w0 + r * rs + N) = u[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (mb + 8 * r >= M) continue;
            const float og[4] = {g[r].x, g[r].y, g[r].z, g[r].w}, ou[4] = {u[r].x, u[r].y, u[r].z, u[r].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (hcol + e < N) {
                w0[r * rs + e] = og[e];
                w0[r * rs + N + e] = ou[e];
              }
          }
        }
      } else {
        float4 o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[r] = make_float4(swiglu1(g[r].x, u[r].x), swiglu1(g[r].y, u[r].y), swiglu1(g[r].z, u[r].z),
                             swiglu1(g[r].w, u[r].w));
        const size_t at0 = (size_t)mb * (size_t)G.ldy + (size_t)hcol, rs = 8 * (size_t)G.ldy;
        if (full) {
          if (yt == DT_BF16) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              *(uint2*)((uint16_t*)out + at0 + r * rs) =
                  make_uint2(pack_bf16x2(o[r].x, o[r].y), pack_bf16x2(o[r].z, o[r].w));
          } else if (yt == DT_F32) {
#pragma unroll
            for (int r = 0; r < 4; ++r) *(float4*)((float*)out + at0 + r * rs) = o[r];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              *(uint2*)((uint16_t*)out + at0 + r * rs) =
                  make_uint2(pack2<X_F16>(o[r].x, o[r].y), pack2<X_F16>(o[r].z, o[r].w));
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (mb + 8 * r >= M) continue;
            const float oe[4] = {o[r].x, o[r].y, o[r].z, o[r].w};
#pragma unroll 1
            for (int e = 0; e < 4; ++e)
              if (hcol + e < N) store_scalar(out, yt, at0 + r * rs + e, oe[e]);
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    });
    return;
  }
  sfor<MI>([&](auto I_) {
    constexpr int i = decltype(I_)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *(float4*)(ep + (lane & 31) * EP_LD + 32 * j + 8 * q + 4 * (lane >> 5)) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    __builtin_amdgcn_wave_barrier();
    // all eight row reads first, one wait, then the stores: lane l holds rows
    // mb + 4r (r = 0..7) of its four columns
    float4 v[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      v[r] = *(const float4*)(ep + (4 * r + (lane >> 4)) * EP_LD + 4 * c4);
      v[r] = make_float4(v[r].x + bv[0], v[r].y + bv[1], v[r].z + bv[2], v[r].w + bv[3]);
    }
    const int mb = m0 + 32 * i + (lane >> 4);
    const size_t at0 = (size_t)mb * (size_t)ld + (size_t)(cb + ncol), rs = 4 * (size_t)ld;
    if (vec_ok && m0 + 32 * i + 32 <= M) {  // whole block in range: straight-line stores
      if (yt == DT_BF16) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
          *(uint2*)((uint16_t*)out + at0 + r * rs) =
              make_uint2(pack_bf16x2(v[r].x, v[r].y), pack_bf16x2(v[r].z, v[r].w));
      } else if (yt == DT_F32) {
#pragma unroll
        for (int r = 0; r < 8; ++r) *(float4*)((float*)out + at0 + r * rs) = v[r];
      } else {
#pragma unroll
        for (int r = 0; r < 8; ++r)
          *(uint2*)((uint16_t*)out + at0 + r * rs) =
              make_uint2(pack2<X_F16>(v[r].x, v[r].y), pack2<X_F16>(v[r].z, v[r].w));
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        if (mb + 4 * r >= M) continue;
        const float o[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll 1
        for (int e = 0; e < 4; ++e)
          if (ncol + e < N) store_scalar(out, yt, at0 + r * rs + e, o[e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  });
}

template <int QT, int XT, int MI, bool SW>
hipError_t launch_tile_t(const TileParams& tp, int nblocks, hipStream_t s) {
  // activation stages, or the epilogue's four 32 x 68 fp32 blocks if larger (MI = 2)
  constexpr int lds_bytes = std::max(NSTAGE * 32 * MI * TK * 2, 4 * 32 * 68 * 4);
  // the LDS limit is a per-device attribute of the kernel: set once on each device used
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_set.load(std::memory_order_acquire) & bit)) {
    const hipError_t e = hipFuncSetAttribute((const void*)qgemm_tile_kernel<QT, XT, MI, SW>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  qgemm_tile_kernel<QT, XT, MI, SW><<<dim3((unsigned)nblocks), dim3(256), lds_bytes, s>>>(tp);
  return hipGetLastError();
}

// tp.tiles_n and the groups' tn0 are set by the caller
template <int QT, int XT>
hipError_t launch_q(TileParams tp, int bm, int S, hipStream_t s) {
  tp.tiles_m = (tp.M + bm - 1) / bm;
  const int ntiles = tp.tiles_m * tp.tiles_n;
  if (tp.swiglu) {
    if (bm == 64) return launch_tile_t<QT, XT, 2, true>(tp, ntiles * S, s);
    return bm == 128 ? launch_tile_t<QT, XT, 4, true>(tp, ntiles * S, s)
                     : launch_tile_t<QT, XT, 8, true>(tp, ntiles * S, s);
  }
  if (bm == 64) return launch_tile_t<QT, XT, 2, false>(tp, ntiles * S, s);
  return bm == 128 ? launch_tile_t<QT, XT, 4, false>(tp, ntiles * S, s)
                   : launch_tile_t<QT, XT, 8, false>(tp, ntiles * S, s);
}

// One translation unit per quant type instantiates the kernels (qgemm_tile_<type>.hip);
// bm in {64, 128, 256}, S split count, f16: fp16 activations (else bf16).
hipError_t launch_tile_q4k(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);
hipError_t launch_tile_q6k(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);
hipError_t launch_tile_q5k(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);
hipError_t launch_tile_q40(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);
hipError_t launch_tile_q41(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);
hipError_t launch_tile_q80(const TileParams& tp, int bm, int S, bool f16, hipStream_t s);

}  // namespace tile
}  // namespace mlxr
