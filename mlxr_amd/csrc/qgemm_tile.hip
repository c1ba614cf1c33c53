// Host side of kernel (b), the prefill GEMM (the kernel itself is in qgemm_tile_kernel.h,
// instantiated per quant type by qgemm_tile_<type>.hip): launch planning (tile height and
// K split), the split-K reduce kernels, chunking of problems with operands of 2 GiB or
// more, and grouped launches of several weights that share the activations.
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <utility>

#include "qgemm_device.h"
#include "qgemm_internal.h"
#include "qgemm_vmem.h"
#include "qgemm_wdequant.h"

#include "qgemm_tile_kernel.h"

namespace mlxr {

namespace {

using namespace tile;


// Tile rows and K split of a launch, from a small cost model in units of one 256-row
// tile step: a 128-row tile step costs 0.62 of it (the weight dequant is shared by half
// the rows); a round of workgroups costs its steps plus 0.8 (prologue, epilogue); a
// split launch adds the reduce kernel, about 3 us plus its partial-sum traffic at
// ~5 TB/s (one 256-row step is ~1.86 us).  Splits are whole groups of eight steps (two
// super-blocks: the kernel's loop runs whole rings of eight steps), at most kMaxSplits splits,
// and only with a workspace of S*M*N*4 bytes.
constexpr int kMaxSplits = 16;
// Cost of one K step of a tile of bm rows, in 256-row steps (measured on MI355X; 0.62 for
// 128-row tiles ranks Llama-3-70B q,k at M = 256 as measured: three splits of 128-row
// tiles 62.6 us, six of 256-row tiles 65.3 us).
constexpr double step_cost(int bm) { return bm == 256 ? 1.0 : bm == 128 ? 0.62 : 0.5; }
struct SplitPlan {
  int bm, tiles, S, kps;
};
SplitPlan plan_split(int M, int N, int K, size_t ws_bytes) {
  const int nkt = (K + TK - 1) / TK, cus = device_cu_count();
  const long tn = (N + TN - 1) / TN;
  SplitPlan best{256, 0, 1, 0};
  double best_t = 1e30;
  for (int bm : {256, 128, 64}) {
    const long tiles = ((M + bm - 1) / bm) * tn;
    for (int S = 1; S <= kMaxSplits; ++S) {
      const int kps = (((nkt + S - 1) / S) + 7) / 8 * 8;
      const int Sr = (nkt + kps - 1) / kps;  // splits actually used
      if (Sr != S) continue;
      if (S > 1 && (kps < 8 || (size_t)S * (size_t)M * (size_t)N * 4u > ws_bytes)) continue;
      const long rounds = (tiles * S + cus - 1) / cus;
      double t = (double)rounds * (kps * step_cost(bm) + 0.8);
      if (S > 1) t += (3.0 + (double)S * M * N * 8.0 / 5e6) / 1.86;
      if (t < best_t) {
        best_t = t;
        best = SplitPlan{bm, (int)tiles, S, kps};
      }
    }
  }

  if (best.kps == 0) best = SplitPlan{256, (int)(((M + 255) / 256) * tn), 1, nkt};  // not reached: S = 1 qualifies
  return best;
}


// The reduce kernels issue every load of a thread before its first add: up to eight
// splits' partials at a time and the bias values, so a thread waits for memory about once
// instead of once per split and once per bias value (a loop that adds as it loads waits for
// each load in turn).  The sums run in split order as before.
template <int VEC>
__device__ __forceinline__ void load_vec(const float* q, float* out) {
  if constexpr (VEC == 4) {
    const float4 a = *(const float4*)q;
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  } else {
    out[0] = *q;
  }
}
// `then` runs after the first eight splits' loads are issued (the caller's bias loads go
// there, so they share the first wait).
template <int VEC, typename Then>
__device__ __forceinline__ void sum_splits(const float* __restrict__ ws, size_t split_elems, int S, size_t i,
                                           float* v, Then&& then) {
  for (int s0 = 0; s0 < S; s0 += 8) {
    float q[8][VEC];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k < S) load_vec<VEC>(ws + (size_t)(s0 + k) * split_elems + i, q[k]);
    if (s0 == 0) then();
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (s0 + k < S) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = s0 + k == 0 ? q[k][e] : v[e] + q[k][e];
      }
  }
}
// VEC consecutive bias values as fp32 (0 without a bias); one dtype branch for all of them.
template <int VEC>
__device__ __forceinline__ void load_bias(const void* b, int dtype, int n, float* out) {
  if (!b) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = 0.f;
  } else if (dtype == DT_F32) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = ((const float*)b)[n + e];
  } else if (dtype == DT_F16) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = f16_bits_to_f32(((const uint16_t*)b)[n + e]);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = bf16_bits_to_f32(((const uint16_t*)b)[n + e]);
  }
}

// y = sum over splits (in split order) + bias, converted to y's dtype.  VEC consecutive
// elements per thread (VEC = 4 needs N % 4 == 0).
template <int VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, size_t split_elems, int S,
                                                            const void* bias, int bias_dtype, void* y, int y_dtype,
                                                            int N, size_t total) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (i >= total) return;
  const int n = (int)(i % (size_t)N);
  float bv[VEC], v[VEC];
  sum_splits<VEC>(ws, split_elems, S, i, v, [&] { load_bias<VEC>(bias, bias_dtype, n, bv); });
  if (bias) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] += bv[e];
  }
  if constexpr (VEC == 4) {
    if (y_dtype == DT_F32) {
      *(float4*)((float*)y + i) = make_float4(v[0], v[1], v[2], v[3]);
      return;
    }
    const uint32_t lo = y_dtype == DT_BF16 ? pack_bf16x2(v[0], v[1]) : pack2<X_F16>(v[0], v[1]);
    const uint32_t hi = y_dtype == DT_BF16 ? pack_bf16x2(v[2], v[3]) : pack2<X_F16>(v[2], v[3]);
    *(uint2*)((uint16_t*)y + i) = make_uint2(lo, hi);
  } else {
    store_scalar(y, y_dtype, i, v[0]);
  }
}

// Grouped split-K: the partial planes hold the launch's weights side by side (rows of
// ws_ld = total N); element (m, c) goes to the weight whose column range holds c.
struct ReduceGroups {
  void* y[MAX_TG];
  const void* bias[MAX_TG];
  int col0[MAX_TG], N[MAX_TG], y_dtype[MAX_TG], bias_dtype[MAX_TG];
  int ngroups;
};
// VEC = 4 (every group's N a multiple of 4): four consecutive columns of one group per thread.
template <int VEC>
__global__ __launch_bounds__(256) void splitk_reduce_grouped_kernel(const float* __restrict__ ws, size_t split_elems,
                                                                    int S, int ws_ld, size_t total, ReduceGroups rg) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (i >= total) return;
  const int m = (int)(i / (size_t)ws_ld), c = (int)(i - (size_t)m * ws_ld);
  int g = 0;
#pragma unroll
  for (int k = 1; k < MAX_TG; ++k)
    if (k < rg.ngroups && c >= rg.col0[k]) g = k;
  const int n = c - rg.col0[g];
  float bv[VEC], v[VEC];
  sum_splits<VEC>(ws, split_elems, S, i, v, [&] { load_bias<VEC>(rg.bias[g], rg.bias_dtype[g], n, bv); });
  if (rg.bias[g]) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] += bv[e];
  }
  const size_t o = (size_t)m * rg.N[g] + n;
  if constexpr (VEC == 4) {
    const int yd = rg.y_dtype[g];
    if (yd == DT_F32) {
      *(float4*)((float*)rg.y[g] + o) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      const uint32_t lo = yd == DT_BF16 ? pack_bf16x2(v[0], v[1]) : pack2<X_F16>(v[0], v[1]);
      const uint32_t hi = yd == DT_BF16 ? pack_bf16x2(v[2], v[3]) : pack2<X_F16>(v[2], v[3]);
      *(uint2*)((uint16_t*)rg.y[g] + o) = make_uint2(lo, hi);
    }
  } else {
    store_scalar(rg.y[g], rg.y_dtype[g], o, v[0]);
  }
}

// SwiGLU split-K: the partial planes hold gate (columns 0 .. N-1) and up (N .. 2N-1) side
// by side; h[m][n] = swish(sum gate + bias_g) * (sum up + bias_u), sums in split order.
__global__ __launch_bounds__(256) void splitk_reduce_swiglu_kernel(const float* __restrict__ ws, size_t split_elems,
                                                                   int S, int N, size_t total, const void* bias_g,
                                                                   const void* bias_u, int bias_dtype, void* y,
                                                                   int y_dtype) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const size_t m = i / (size_t)N, n = i - m * (size_t)N;
  const size_t gi = m * 2 * (size_t)N + n, ui = gi + (size_t)N;
  float bg, bu, g, u;
  sum_splits<1>(ws, split_elems, S, gi, &g, [&] { load_bias<1>(bias_g, bias_dtype, (int)n, &bg); });
  sum_splits<1>(ws, split_elems, S, ui, &u, [&] { load_bias<1>(bias_u, bias_dtype, (int)n, &bu); });
  if (bias_g) g += bg;
  if (bias_u) u += bu;
  store_scalar(y, y_dtype, i, swiglu1(g, u));
}

hipError_t launch_chunk(const TileParams& tp, int bm, int S, int qtype, bool f16, hipStream_t s) {
  switch (qtype) {
    case QT_Q4_K: return launch_tile_q4k(tp, bm, S, f16, s);
    case QT_Q6_K: return launch_tile_q6k(tp, bm, S, f16, s);
    case QT_Q5_K: return launch_tile_q5k(tp, bm, S, f16, s);
    case QT_Q4_0: return launch_tile_q40(tp, bm, S, f16, s);
    case QT_Q4_1: return launch_tile_q41(tp, bm, S, f16, s);
    default: return launch_tile_q80(tp, bm, S, f16, s);
  }
}

size_t dtype_bytes(int dt) { return dt == DT_F32 ? 4 : 2; }

}  // namespace

// Kernels address operands with 32-bit buffer offsets; problems whose activations or
// weight planes reach 2 GiB run as several launches over M and N chunks (plane bytes are
// a whole number per weight row, so an N chunk is a row range of every plane).
hipError_t launch_mfma(const RunArgs& a, hipStream_t s) {
  const int M = a.M, N = a.L.N, K = a.L.K;
  const size_t lim = operand_limit();
  size_t prb[4] = {0, 0, 0, 0};
  size_t max_prb = 1;
  for (int i = 0; i < a.L.nplanes; ++i) {
    prb[i] = a.L.size[i] / (size_t)N;
    max_prb = std::max(max_prb, prb[i]);
  }
  const int Mc = (int)std::max<size_t>(256, ((lim - 1) / ((size_t)K * 2)) / 256 * 256);
  const int Nc = (int)std::max<size_t>(TN, ((lim - 1) / max_prb) / TN * TN);
  const PlanePtrs P = plane_ptrs(a.L, a.packed);
  const size_t ye = dtype_bytes(a.y_dtype), be = dtype_bytes(a.bias_dtype);
  // split-K (single-chunk problems with a large enough workspace only)
  // the plan for an unlimited workspace, used only if the caller's workspace holds it
  // (so a given shape either takes that plan or the unsplit one, never a third)
  SplitPlan sp{0, 0, 1, 0};
  if (a.ws && M <= Mc && N <= Nc) {
    sp = plan_split(M, N, K, ~(size_t)0);
    if (sp.S > 1 && (size_t)sp.S * (size_t)M * (size_t)N * 4u > a.ws_bytes) sp.S = 1;
  }
  if (sp.S > 1) {
    TileParams tp;
    tp.swiglu = 0;
    tp.M = M;
    tp.K = K;
    tp.x = a.x;
    tp.nib = 0x0F0F0F0Fu;
    tp.kps = sp.kps;
    tp.ws = (float*)a.ws;
    tp.ws_split = (size_t)M * (size_t)N;
    tp.ws_ld = N;
    tp.ngroups = 1;
    TileGroup& g = tp.g[0];
    for (int i = 0; i < 4; ++i) {
      g.P[i] = P.p[i];
      g.psize[i] = i < a.L.nplanes ? (uint32_t)a.L.size[i] : 0u;
    }
    g.y = a.y;
    g.bias = nullptr;
    g.N = N;
    g.ldy = N;
    g.tn0 = 0;
    g.col0 = 0;
    g.bias_dtype = a.bias_dtype;
    g.y_dtype = DT_F32;
    tp.tiles_n = (N + TN - 1) / TN;
    hipError_t e = launch_chunk(tp, sp.bm, sp.S, a.L.qtype, a.x_dtype == DT_F16, s);
    if (e != hipSuccess) return e;
    return launch_splitk_reduce((const float*)a.ws, tp.ws_split, sp.S, a.bias, a.bias_dtype, a.y, a.y_dtype, M, N,
                                s);
  }
  for (int mc = 0; mc < M; mc += Mc) {
    for (int nc = 0; nc < N; nc += Nc) {
      TileParams tp;
      tp.swiglu = 0;
      tp.M = std::min(Mc, M - mc);
      tp.K = K;
      tp.x = (const uint8_t*)a.x + (size_t)mc * K * 2;
      tp.nib = 0x0F0F0F0Fu;
      tp.kps = (K + TK - 1) / TK;
      tp.ws = nullptr;
      tp.ws_split = 0;
      tp.ws_ld = 0;
      tp.ngroups = 1;
      TileGroup& g = tp.g[0];
      g.N = std::min(Nc, N - nc);
      for (int i = 0; i < 4; ++i) {
        g.P[i] = P.p[i] ? P.p[i] + (size_t)nc * prb[i] : nullptr;
        g.psize[i] = i < a.L.nplanes ? (uint32_t)((size_t)g.N * prb[i]) : 0u;
      }
      g.y = (uint8_t*)a.y + ((size_t)mc * N + nc) * ye;
      g.bias = a.bias ? (const uint8_t*)a.bias + (size_t)nc * be : nullptr;
      g.ldy = N;
      g.tn0 = 0;
      g.col0 = 0;
      g.bias_dtype = a.bias_dtype;
      g.y_dtype = a.y_dtype;
      tp.tiles_n = (g.N + TN - 1) / TN;
      const int bm = plan_split(tp.M, g.N, K, 0).bm;
      const hipError_t e = launch_chunk(tp, bm, 1, a.L.qtype, a.x_dtype == DT_F16, s);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Grouped launch: up to MAX_TG weights of one quant type and K that share x, as one grid
// whose tile columns run over the weights in turn; the split plan is that of the
// concatenated N.  Requires every operand below 2 GiB (mfma_groupable).
bool mfma_groupable(const RunArgs& a) {
  const size_t lim = operand_limit();
  if ((size_t)a.M * (size_t)a.L.K * 2u >= lim) return false;
  for (int i = 0; i < a.L.nplanes; ++i)
    if (a.L.size[i] >= lim) return false;
  return true;
}

static int grouped_cols(const RunArgs* const* items, int n, int* ntiles) {
  int cols = 0, t = 0;
  for (int i = 0; i < n; ++i) {
    cols += items[i]->L.N;
    t += (items[i]->L.N + TN - 1) / TN;
  }
  if (ntiles) *ntiles = t;
  return cols;
}

size_t mfma_grouped_workspace_bytes(const RunArgs* const* items, int n) {
  int nt = 0;
  const int cols = grouped_cols(items, n, &nt);
  const RunArgs& a = *items[0];
  if (!mfma_groupable(a)) return 0;
  const SplitPlan sp = plan_split(a.M, nt * TN, a.L.K, ~(size_t)0);
  return sp.S > 1 ? (size_t)sp.S * (size_t)a.M * (size_t)cols * 4u : 0;
}

hipError_t launch_mfma_grouped(const RunArgs* const* items, int n, void* ws, size_t ws_bytes, hipStream_t s) {
  const RunArgs& a = *items[0];
  const int M = a.M, K = a.L.K;
  int nt = 0;
  const int cols = grouped_cols(items, n, &nt);
  SplitPlan sp = plan_split(M, nt * TN, K, ~(size_t)0);
  if (sp.S > 1 && (!ws || (size_t)sp.S * (size_t)M * (size_t)cols * 4u > ws_bytes)) sp = plan_split(M, nt * TN, K, 0);
  TileParams tp;
  tp.swiglu = 0;
  tp.M = M;
  tp.K = K;
  tp.x = a.x;
  tp.nib = 0x0F0F0F0Fu;
  tp.kps = sp.S > 1 ? sp.kps : (K + TK - 1) / TK;
  tp.ws = sp.S > 1 ? (float*)ws : nullptr;
  tp.ws_split = (size_t)M * (size_t)cols;
  tp.ws_ld = cols;
  tp.ngroups = n;
  tp.tiles_n = nt;
  ReduceGroups rg;
  rg.ngroups = n;
  int tn0 = 0, col0 = 0;
  for (int i = 0; i < MAX_TG; ++i) {
    TileGroup& g = tp.g[i];
    if (i >= n) {  // unused entries: never selected (ngroups), kept defined
      g = tp.g[0];
      continue;
    }
    const RunArgs& b = *items[i];
    const PlanePtrs P = plane_ptrs(b.L, b.packed);
    for (int k = 0; k < 4; ++k) {
      g.P[k] = P.p[k];
      g.psize[k] = k < b.L.nplanes ? (uint32_t)b.L.size[k] : 0u;
    }
    g.y = b.y;
    g.bias = sp.S > 1 ? nullptr : b.bias;
    g.N = b.L.N;
    g.ldy = b.L.N;
    g.tn0 = tn0;
    g.col0 = col0;
    g.bias_dtype = b.bias_dtype;
    g.y_dtype = b.y_dtype;
    rg.y[i] = b.y;
    rg.bias[i] = b.bias;
    rg.col0[i] = col0;
    rg.N[i] = b.L.N;
    rg.y_dtype[i] = b.y_dtype;
    rg.bias_dtype[i] = b.bias_dtype;
    tn0 += (b.L.N + TN - 1) / TN;
    col0 += b.L.N;
  }
  hipError_t e = launch_chunk(tp, sp.bm, sp.S > 1 ? sp.S : 1, a.L.qtype, a.x_dtype == DT_F16, s);
  if (e != hipSuccess || sp.S <= 1) return e;
  const size_t total = (size_t)M * (size_t)cols;
  bool vec4 = true;
  for (int i = 0; i < n; ++i) vec4 = vec4 && (items[i]->L.N & 3) == 0;
  if (vec4)
    splitk_reduce_grouped_kernel<4><<<dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, s>>>(
        (const float*)ws, tp.ws_split, sp.S, cols, total, rg);
  else
    splitk_reduce_grouped_kernel<1><<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(
        (const float*)ws, tp.ws_split, sp.S, cols, total, rg);
  return hipGetLastError();
}

// SwiGLU: gate and up (same type and [N, K]) in one tiled launch, 128 columns of each per
// tile; the split plan is that of a 2N-column problem.
size_t mfma_swiglu_workspace_bytes(int M, int N, int K) {
  if ((size_t)M * (size_t)K * 2u >= ((size_t)1 << 31)) return 0;
  const SplitPlan sp = plan_split(M, 2 * ((N + TN / 2 - 1) / (TN / 2)) * (TN / 2), K, ~(size_t)0);
  return sp.S > 1 ? (size_t)sp.S * (size_t)M * (size_t)N * 8u : 0;
}

hipError_t launch_mfma_swiglu(const RunArgs& gate, const RunArgs& up, void* ws, size_t ws_bytes, hipStream_t s) {
  if (gate.bias || up.bias) return hipErrorInvalidValue;  // the tiled SwiGLU epilogue adds no bias
  const int M = gate.M, N = gate.L.N, K = gate.L.K;
  const int tiles_n = (N + TN / 2 - 1) / (TN / 2);
  SplitPlan sp = plan_split(M, 2 * tiles_n * (TN / 2), K, ~(size_t)0);
  if (sp.S > 1 && (!ws || (size_t)sp.S * (size_t)M * (size_t)N * 8u > ws_bytes))
    sp = plan_split(M, 2 * tiles_n * (TN / 2), K, 0);
  const bool split = sp.S > 1;
  TileParams tp;
  tp.swiglu = 1;
  tp.M = M;
  tp.K = K;
  tp.x = gate.x;
  tp.nib = 0x0F0F0F0Fu;
  tp.kps = split ? sp.kps : (K + TK - 1) / TK;
  tp.ws = split ? (float*)ws : nullptr;
  tp.ws_split = (size_t)M * (size_t)N * 2u;
  tp.ws_ld = 2 * N;
  tp.ngroups = 2;
  tp.tiles_n = tiles_n;
  const RunArgs* ab[2] = {&gate, &up};
  for (int i = 0; i < MAX_TG; ++i) {
    TileGroup& g = tp.g[i];
    const RunArgs& b = *ab[i < 2 ? i : 0];
    const PlanePtrs P = plane_ptrs(b.L, b.packed);
    for (int k = 0; k < 4; ++k) {
      g.P[k] = P.p[k];
      g.psize[k] = k < b.L.nplanes ? (uint32_t)b.L.size[k] : 0u;
    }
    g.y = gate.y;
    g.bias = nullptr;
    g.N = N;
    g.ldy = N;
    g.tn0 = 0;
    g.col0 = i == 1 ? N : 0;
    g.bias_dtype = b.bias_dtype;
    g.y_dtype = gate.y_dtype;
  }
  hipError_t e = launch_chunk(tp, sp.bm, split ? sp.S : 1, gate.L.qtype, gate.x_dtype == DT_F16, s);
  if (e != hipSuccess || !split) return e;
  return launch_splitk_reduce_swiglu((const float*)ws, tp.ws_split, sp.S, gate.bias, up.bias, gate.bias_dtype, gate.y,
                                     gate.y_dtype, M, N, s);
}

hipError_t launch_splitk_reduce_swiglu(const float* ws, size_t split_elems, int S, const void* bias_g,
                                       const void* bias_u, int bias_dtype, void* y, int y_dtype, int M, int N,
                                       hipStream_t s) {
  const size_t total = (size_t)M * (size_t)N;
  splitk_reduce_swiglu_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(
      ws, split_elems, S, N, total, bias_g, bias_u, bias_dtype, y, y_dtype);
  return hipGetLastError();
}

double mfma_est_us(int M, int N, int K, int qtype, size_t ws_bytes) {
  const SplitPlan sp = plan_split(M, N, K, ws_bytes);
  const int nkt = (K + TK - 1) / TK;
  const long rounds = ((long)sp.tiles * sp.S + device_cu_count() - 1) / device_cu_count();
  // Q6_K steps dequantize more per weight: measured on MI355X (Llama-3-70B v, 1024x8192,
  // M = 256) 40.6 us against 24.8 us for the Q4_K weight of the same shape
  const double qf = qtype == QT_Q6_K ? 1.6 : 1.0;
  double t = (double)rounds * (sp.kps * step_cost(sp.bm) * qf + 0.8);
  if (sp.S > 1) t += (3.0 + (double)sp.S * M * N * 8.0 / 5e6) / 1.86;
  // launches of one ring per workgroup take about 4.5 us more than the model says
  // (measured on MI355X, Llama-3-8B q/k shapes at M = 64-512)
  return t * 1.86 + (sp.kps <= 8 && nkt > 8 ? 4.5 : 0.0);
}

size_t mfma_workspace_bytes(int M, int N, int K) {
  if ((size_t)M * (size_t)K * 2u >= ((size_t)1 << 31)) return 0;
  const SplitPlan sp = plan_split(M, N, K, ~(size_t)0);
  return sp.S > 1 ? (size_t)sp.S * (size_t)M * (size_t)N * 4u : 0;
}

hipError_t launch_splitk_reduce(const float* ws, size_t split_elems, int S, const void* bias, int bias_dtype, void* y,
                                int y_dtype, int M, int N, hipStream_t s) {
  const size_t total = (size_t)M * (size_t)N;
  if ((N & 3) == 0) {
    const size_t threads = total / 4;
    splitk_reduce_kernel<4><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(
        ws, split_elems, S, bias, bias_dtype, y, y_dtype, N, total);
  } else {
    splitk_reduce_kernel<1><<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s>>>(
        ws, split_elems, S, bias, bias_dtype, y, y_dtype, N, total);
  }
  return hipGetLastError();
}

}  // namespace mlxr
