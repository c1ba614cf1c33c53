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
#include <stdlib.h>

#include <algorithm>
#include <atomic>

#include "qgemm_gemv_common.h"

namespace mlxr {

namespace {

struct GemvParams {
  PlanePtrs P;
  const void* x;
  const void* bias;
  void* y;
  int M, N, K;
  int bias_dtype, y_dtype;
};

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

// SW (SwiGLU): the launch has two weights of the same shape, gate (group 0) and up (group
// 1); a wavefront walks its gate rows, then the same up rows, and stores swish(gate) * up
// for those rows into group 0's output.
template <int QT, int XT, int MT, int D, bool LIN, bool SW, bool NT>
__global__ __launch_bounds__(256) void qgemv_lds_kernel(LdsParams lp) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps the loop scalar
  const int K = lp.K, M = lp.M;
  const int nsub = K >> 5, nsb = K >> 8;
  const int nseg = (nsub + 63) >> 6;
  // which weight of the launch this wavefront works on (scalar search)
  const int gw = blockIdx.x * 4 + wave;
  int gi = 0;
#pragma unroll
  for (int g = 1; g < MAX_GROUPS; ++g)
    if (g < lp.ngroups && gw >= lp.g[g].wave_start) gi = g;
  // select the group's fields with static kernarg offsets, so every parameter load is
  // issued at once instead of after the (scalar) search
  LdsGroup G = lp.g[0];
#pragma unroll
  for (int g = 1; g < MAX_GROUPS; ++g) {
    const LdsGroup& H = lp.g[g];
    const bool t = g == gi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      G.P.p[i] = t ? H.P.p[i] : G.P.p[i];
      G.psize[i] = t ? H.psize[i] : G.psize[i];
    }
    G.y = t ? H.y : G.y;
    G.bias = t ? H.bias : G.bias;
    G.N = t ? H.N : G.N;
    G.rows_per_wave = t ? H.rows_per_wave : G.rows_per_wave;
    G.wave_start = t ? H.wave_start : G.wave_start;
    G.y_dtype = t ? H.y_dtype : G.y_dtype;
    G.bias_dtype = t ? H.bias_dtype : G.bias_dtype;
  }
  const int N = G.N;
  const int rpw = G.rows_per_wave;
  const int r0 = (gw - G.wave_start) * rpw;
  const int r1 = min(r0 + rpw, N);
  constexpr int NW = SW ? 2 : 1;  // weights walked per row
  const int C = r1 > r0 ? (r1 - r0) * nseg * NW : 0;
  uint4* xs = (uint4*)smem;                                          // [MT][nseg][4][64]
  float2* Xs = (float2*)(smem + (size_t)MT * nseg * 4096);           // [MT][nseg][64]

  rsrc_t R[4], RU[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) R[i] = make_rsrc(G.P.p[i] ? G.P.p[i] : (const uint8_t*)lp.x, G.psize[i]);
  if constexpr (SW) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      RU[i] = make_rsrc(lp.g[1].P.p[i] ? lp.g[1].P.p[i] : (const uint8_t*)lp.x, lp.g[1].psize[i]);
  }

  // Activation loads go out first (two padded tasks per thread; padding reads zeros),
  // then the weight prefetch, so the in-order memory counter never makes the LDS staging
  // wait for HBM.
  const rsrc_t RX = make_rsrc(lp.x, (uint32_t)M * (uint32_t)K * 2u);
  const int T = MT * nseg * 64;
  auto xoff = [&](int t) -> uint32_t {
    const int m = t / (nseg * 64), sbp = t - m * nseg * 64;
    return (t < T && m < M && sbp < nsub) ? ((uint32_t)m * K + (uint32_t)sbp * 32u) * 2u : OOB;
  };
  auto xload = [&](int t, uint4* v) {
    const uint32_t o = xoff(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(RX, o + 16 * i, 0, 0);
      v[i] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  };
  uint4 xa[4], xc[4];
  xload(threadIdx.x, xa);
  if (T > 256) xload(threadIdx.x + 256, xc);

  CLoad<QT> buf[D];
  // SW: a wavefront walks all its gate rows, then the same up rows (chunk c < CG: gate)
  const int CG = SW ? C / 2 : C;
  auto issue = [&](int c, CLoad<QT>& b) {
    int cc = max(min(c, C - 1), 0);
    if constexpr (SW) {
      const bool up = cc >= CG;
      cc = up ? cc - CG : cc;
      rsrc_t Rs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) Rs[i] = up ? RU[i] : R[i];
      if constexpr (LIN) {
        load_chunk<QT, NT ? POL_NT : POL_DEFAULT>(Rs, r0, cc, nsub, nsb, lane, true, b);
      } else {
        const int rl = cc / nseg, seg = cc - rl * nseg;
        load_chunk<QT, NT ? POL_NT : POL_DEFAULT>(Rs, min(r0 + rl, N - 1), seg, nsub, nsb, lane, seg * 64 + lane < nsub, b);
      }
    } else if constexpr (LIN) {
      // every row is exactly nseg full segments: chunk cc starts at sub-block r0*nsub + 64*cc
      load_chunk<QT, NT ? POL_NT : POL_DEFAULT>(R, r0, cc, nsub, nsb, lane, true, b);
    } else {
      const int rl = cc / nseg, seg = cc - rl * nseg;
      const int row = min(r0 + rl, N - 1);
      load_chunk<QT, NT ? POL_NT : POL_DEFAULT>(R, row, seg, nsub, nsb, lane, seg * 64 + lane < nsub, b);
    }
  };
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, buf[d]);

  auto stage = [&](int t, const uint4* v) {
    const int m = t / (nseg * 64), sbp = t - m * nseg * 64;
    const int seg = sbp >> 6, l = sbp & 63;
    uint32_t xv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xs[((m * nseg + seg) * 4 + i) * 64 + l] = v[i];
      xv[4 * i + 0] = v[i].x;
      xv[4 * i + 1] = v[i].y;
      xv[4 * i + 2] = v[i].z;
      xv[4 * i + 3] = v[i].w;
    }
    float2 X;
    X.x = sum_range<XT, 0, 8>(xv);
    X.y = sum_range<XT, 8, 16>(xv);
    Xs[(m * nseg + seg) * 64 + l] = X;
  };
  if ((int)threadIdx.x < T) stage(threadIdx.x, xa);
  if ((int)threadIdx.x + 256 < T) stage(threadIdx.x + 256, xc);
  for (int t = threadIdx.x + 512; t < T; t += 256) {
    uint4 v[4];
    xload(t, v);
    stage(t, v);
  }
  __syncthreads();
  if (C == 0) return;

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;
  float res = 0.f, res_up = 0.f;
  const uint32_t MASK = lp.cmask, MAGIC = lp.cmagic;

  auto compute = [&](const CLoad<QT>& b, const int rl, const int seg, const bool up) {
    WDec wd;
    decode_chunk<QT, XT>(b, lane & 7, MASK, MAGIC, wd);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) {
        const uint4* xp = xs + (m * nseg + seg) * 256 + lane;
        uint32_t xv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 v = xp[64 * i];
          xv[4 * i + 0] = v.x;
          xv[4 * i + 1] = v.y;
          xv[4 * i + 2] = v.z;
          xv[4 * i + 3] = v.w;
        }
        const float2 X = Xs[(m * nseg + seg) * 64 + lane];
        acc[m] += contrib<QT, XT>(xv, wd, X.x, X.y);
      }
    }
    if (seg == nseg - 1) {
      // Row finished: its total goes to lane (row_local * MT + m); stored after the loop.
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < M) {
          const float tot = wave_total(acc[m]);
          if (SW && up) res_up = (lane == rl * MT + m) ? tot : res_up;
          else res = (lane == rl * MT + m) ? tot : res;
        }
        acc[m] = 0.f;
      }
    }
  };

  // Steady state: D chunks per trip, every load and compute unconditional.
  // (row_local, segment) of the chunk being reduced: uniform loop state.
  // (SW: which weight of the row pair, also uniform)
  int c = 0, rl = 0, seg = 0;
  bool up = false;
  auto advance = [&]() {
    if (++seg == nseg) {
      seg = 0;
      ++rl;
      if (SW && !up && rl == r1 - r0) {
        rl = 0;
        up = true;
      }
    }
  };
  for (; c + D <= C; c += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(c + d + D - 1, buf[(d + D - 1) % D]);
      compute(buf[d], rl, seg, up);
      advance();
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    if (c + d < C) {
      compute(buf[d], rl, seg, up);
      advance();
    }
  }

  // Lane (row_local * MT + m) holds y[m, r0 + row_local].
  const int orl = lane / MT, om = lane - orl * MT;
  if (orl < r1 - r0 && om < M) {
    float v = res;
    if (G.bias) v += load_scalar(G.bias, G.bias_dtype, (size_t)(r0 + orl));
    if constexpr (SW) {
      float u = res_up;
      if (lp.g[1].bias) u += load_scalar(lp.g[1].bias, lp.g[1].bias_dtype, (size_t)(r0 + orl));
      v = swiglu1(v, u);
    }
    store_scalar(G.y, G.y_dtype, (size_t)om * N + r0 + orl, v);
  }
}


size_t lds_bytes(int MT, int K) { return (size_t)MT * (size_t)(((K >> 5) + 63) >> 6) * 64 * 72; }

// gfx950 gives a workgroup up to 160 KiB of LDS (above 64 KiB once the kernel's limit
// is raised); device_lds_limit() is that figure as the device reports it.

// Wavefronts per CU the row split aims for.  Every workgroup stages all of X in LDS, so
// for long rows (K >= 8192: down-projection shapes) fewer, longer-lived wavefronts win:
// the X staging traffic halves (measured on MI355X: Llama-3-8B down 10.6 -> 9.9 us at
// M = 1).
int waves_per_cu_target(int K) { return K >= 8192 ? 8 : 16; }

// Weight loads of a launch streaming at least this many bytes are non-temporal: measured
// on MI355X (Llama-3-8B, M = 1) gate_up 15.1 -> 14.1 us and down 9.9 -> 9.6 us, while
// the small launches (o, k/v, 2-9 MB) lose 2-5% with them.
constexpr size_t kNtMinBytes = (size_t)16 << 20;

// Raises the kernel's dynamic LDS limit on the current device (once per device).
template <typename KernelPtr>
hipError_t allow_lds(KernelPtr k, size_t bytes, std::atomic<uint64_t>& done) {
  if (bytes <= 65536) return hipSuccess;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  const hipError_t e =
      hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)device_lds_limit());
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return e;
}

template <int QT, int XT, int MT, int D, bool LIN, bool SW, bool NT>
hipError_t launch_lds_k(const LdsParams& lp, unsigned grid, hipStream_t s) {
  static std::atomic<uint64_t> attr{0};
  const size_t lb = lds_bytes(MT, lp.K);
  const hipError_t e = allow_lds(qgemv_lds_kernel<QT, XT, MT, D, LIN, SW, NT>, lb, attr);
  if (e != hipSuccess) return e;
  qgemv_lds_kernel<QT, XT, MT, D, LIN, SW, NT><<<dim3(grid), dim3(256), lb, s>>>(lp);
  return hipGetLastError();
}

// LIN: every row is a whole number of 64-sub-block segments.  NT (M = 1 only, where
// launches stream the most bytes per activation): non-temporal weight loads.
template <int QT, int XT, int MT, int D, bool SW = false>
hipError_t launch_lds_t(const LdsParams& lp, unsigned grid, bool nt, hipStream_t s) {
  const bool lin = ((lp.K >> 5) & 63) == 0;
  if constexpr (MT == 1) {
    if (nt) return lin ? launch_lds_k<QT, XT, MT, D, true, SW, true>(lp, grid, s)
                       : launch_lds_k<QT, XT, MT, D, false, SW, true>(lp, grid, s);
  }
  return lin ? launch_lds_k<QT, XT, MT, D, true, SW, false>(lp, grid, s)
             : launch_lds_k<QT, XT, MT, D, false, SW, false>(lp, grid, s);
}

// Planes addressed with 32-bit buffer offsets: every plane (and x) must stay below 2 GiB.
bool lds_fits(int M, int K, const PackedLayout& L, int MT) {
  const size_t lim = operand_limit();
  for (int i = 0; i < L.nplanes; ++i)
    if (L.size[i] >= lim) return false;
  if ((size_t)M * K * 2 >= lim) return false;
  return lds_bytes(MT, K) <= device_lds_limit();
}

int mt_for(int M) { return M == 1 ? 1 : M <= 2 ? 2 : 4; }

// Fills the launch parameters for `n` weights sharing x; returns the grid size.  *bytes:
// the launch's weight bytes.
unsigned lds_setup(const RunArgs* const* items, int n, LdsParams& lp, size_t* bytes) {
  const RunArgs& a0 = *items[0];
  const int MT = mt_for(a0.M);
  lp.x = a0.x;
  lp.M = a0.M;
  lp.K = a0.L.K;
  lp.ngroups = n;
  lp.cmask = 0x000F000Fu;
  lp.cmagic = a0.x_dtype == DT_F16 ? 0x64006400u : 0x43004300u;
  long total_rows = 0;
  for (int i = 0; i < n; ++i) total_rows += items[i]->L.N;
  // rows per wavefront: as few as keep ~waves_per_cu wavefronts per CU busy
  const long target = (long)device_cu_count() * waves_per_cu_target(a0.L.K);
  int rpw = (int)min((total_rows + target - 1) / target, (long)(64 / MT));  // row results: one per lane
  if (rpw < 1) rpw = 1;
  int ws = 0;
  *bytes = 0;
  for (int i = 0; i < n; ++i) {
    const RunArgs& a = *items[i];
    LdsGroup& G = lp.g[i];
    G.P = plane_ptrs(a.L, a.packed);
    for (int k = 0; k < 4; ++k) G.psize[k] = k < a.L.nplanes ? (uint32_t)a.L.size[k] : 0u;
    G.y = a.y;
    G.bias = a.bias;
    G.N = a.L.N;
    G.rows_per_wave = rpw;
    G.wave_start = ws;
    G.y_dtype = a.y_dtype;
    G.bias_dtype = a.bias_dtype;
    ws += (a.L.N + rpw - 1) / rpw;
    *bytes += a.L.total;
  }
  return (unsigned)((ws + 3) / 4);
}

template <int QT, int XT>
hipError_t launch_lds(const RunArgs* const* items, int n, hipStream_t s) {
  LdsParams lp;
  size_t bytes = 0;
  const unsigned grid = lds_setup(items, n, lp, &bytes);
  const int M = lp.M;
  if (M == 1) return launch_lds_t<QT, XT, 1, 3>(lp, grid, bytes >= kNtMinBytes, s);
  if (M == 2) return launch_lds_t<QT, XT, 2, 3>(lp, grid, false, s);
  return launch_lds_t<QT, XT, 4, 3>(lp, grid, false, s);
}

template <int QT, int XT, int MT, int R>
hipError_t launch_t(const GemvParams& p, hipStream_t s) {
  const int rows_per_block = 4 * R;
  const dim3 grid((unsigned)((p.N + rows_per_block - 1) / rows_per_block));
  qgemv_kernel<QT, XT, MT, R><<<grid, dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

template <int QT, int XT>
hipError_t launch_x(const GemvParams& p, const RunArgs& a, int R, hipStream_t s) {
  const int M = p.M;
  if (M <= 4 && lds_fits(M, p.K, a.L, mt_for(M))) {
    const RunArgs* items[1] = {&a};
    return launch_lds<QT, XT>(items, 1, s);
  }
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

// Rows per wavefront at M = 1 in the register-staged kernel.
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
    case QT_Q4_K: return f16 ? launch_x<QT_Q4_K, X_F16>(p, a, R, s) : launch_x<QT_Q4_K, X_BF16>(p, a, R, s);
    case QT_Q6_K: return f16 ? launch_x<QT_Q6_K, X_F16>(p, a, R, s) : launch_x<QT_Q6_K, X_BF16>(p, a, R, s);
    case QT_Q5_K: return f16 ? launch_x<QT_Q5_K, X_F16>(p, a, R, s) : launch_x<QT_Q5_K, X_BF16>(p, a, R, s);
    case QT_Q4_0: return f16 ? launch_x<QT_Q4_0, X_F16>(p, a, R, s) : launch_x<QT_Q4_0, X_BF16>(p, a, R, s);
    case QT_Q4_1: return f16 ? launch_x<QT_Q4_1, X_F16>(p, a, R, s) : launch_x<QT_Q4_1, X_BF16>(p, a, R, s);
    default: return f16 ? launch_x<QT_Q8_0, X_F16>(p, a, R, s) : launch_x<QT_Q8_0, X_BF16>(p, a, R, s);
  }
}

bool gemv_groupable(const RunArgs& a) { return a.M <= 4 && lds_fits(a.M, a.L.K, a.L, mt_for(a.M)); }

template <int QT, int XT>
hipError_t launch_lds_swiglu(const RunArgs& gate, const RunArgs& up, hipStream_t s) {
  const RunArgs* items[2] = {&gate, &up};
  LdsParams lp;
  size_t bytes = 0;
  lds_setup(items, 2, lp, &bytes);
  // every wavefront works on gate rows (and the same up rows): group 1 owns no wavefronts;
  // as many wavefronts as a grouped launch of the two weights would have
  const long target = (long)device_cu_count() * waves_per_cu_target(gate.L.K);
  lp.g[0].rows_per_wave = lp.g[1].rows_per_wave =
      (int)std::min<long>(64 / mt_for(gate.M), std::max<long>(1, (gate.L.N + target - 1) / target));
  lp.g[1].wave_start = 0x7fffffff;
  const int waves = (gate.L.N + lp.g[0].rows_per_wave - 1) / lp.g[0].rows_per_wave;
  const unsigned grid = (unsigned)((waves + 3) / 4);
  const int M = lp.M;
  if (M == 1) return launch_lds_t<QT, XT, 1, 3, true>(lp, grid, bytes >= kNtMinBytes, s);
  if (M == 2) return launch_lds_t<QT, XT, 2, 3, true>(lp, grid, false, s);
  return launch_lds_t<QT, XT, 4, 3, true>(lp, grid, false, s);
}

hipError_t launch_gemv_grouped(const RunArgs* const* items, int n, hipStream_t s) {
  const RunArgs& a = *items[0];
  const bool f16 = a.x_dtype == DT_F16;
  switch (a.L.qtype) {
    case QT_Q4_K: return f16 ? launch_lds<QT_Q4_K, X_F16>(items, n, s) : launch_lds<QT_Q4_K, X_BF16>(items, n, s);
    case QT_Q6_K: return f16 ? launch_lds<QT_Q6_K, X_F16>(items, n, s) : launch_lds<QT_Q6_K, X_BF16>(items, n, s);
    case QT_Q5_K: return f16 ? launch_lds<QT_Q5_K, X_F16>(items, n, s) : launch_lds<QT_Q5_K, X_BF16>(items, n, s);
    case QT_Q4_0: return f16 ? launch_lds<QT_Q4_0, X_F16>(items, n, s) : launch_lds<QT_Q4_0, X_BF16>(items, n, s);
    case QT_Q4_1: return f16 ? launch_lds<QT_Q4_1, X_F16>(items, n, s) : launch_lds<QT_Q4_1, X_BF16>(items, n, s);
    default: return f16 ? launch_lds<QT_Q8_0, X_F16>(items, n, s) : launch_lds<QT_Q8_0, X_BF16>(items, n, s);
  }
}

hipError_t launch_gemv_swiglu(const RunArgs& gate, const RunArgs& up, hipStream_t s) {
  const bool f16 = gate.x_dtype == DT_F16;
  switch (gate.L.qtype) {
    case QT_Q4_K: return f16 ? launch_lds_swiglu<QT_Q4_K, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q4_K, X_BF16>(gate, up, s);
    case QT_Q6_K: return f16 ? launch_lds_swiglu<QT_Q6_K, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q6_K, X_BF16>(gate, up, s);
    case QT_Q5_K: return f16 ? launch_lds_swiglu<QT_Q5_K, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q5_K, X_BF16>(gate, up, s);
    case QT_Q4_0: return f16 ? launch_lds_swiglu<QT_Q4_0, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q4_0, X_BF16>(gate, up, s);
    case QT_Q4_1: return f16 ? launch_lds_swiglu<QT_Q4_1, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q4_1, X_BF16>(gate, up, s);
    default: return f16 ? launch_lds_swiglu<QT_Q8_0, X_F16>(gate, up, s) : launch_lds_swiglu<QT_Q8_0, X_BF16>(gate, up, s);
  }
}

}  // namespace mlxr
