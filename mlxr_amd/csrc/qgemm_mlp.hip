// Fused SwiGLU MLP for decode (M = 1): y = down( swish(x . Wg^T) * (x . Wu^T) ) in ONE launch.
//
// The reference fuses the whole MLP into one kernel (core/kernels/metal/swiglu_mlp_fused.metal:
// 110-131: gate, up, gating and the down projection).  Here the launch has two roles that
// run at the same time, pipelined over the segments of h (2048 values, the K extent of
// one GEMV chunk of the down projection):
//   - workgroups [0, G1) ("gate/up"): wavefront w of workgroup b computes, in iteration k,
//     row 4(b + G1 k) + w of gate and of up (each walked segment by segment against x in
//     LDS, exactly as qgemv_lds_kernel<SW> walks a row) and stores h = swish(gate) * up in
//     the activation type.  Iteration k of all workgroups covers rows [4 G1 k, 4 G1 (k+1)),
//     so h fills up in row order and its segments complete one after another.  Each
//     workgroup counts itself in at the segment its rows belong to; the last one in raises
//     that segment's go flag.
//   - workgroups [G1, G1 + G2) ("down"): each wavefront owns rpw_b rows of the down
//     projection and walks them segment-major: wait for segment s's go flag, stage that
//     segment of h in LDS, add segment s of every row.  Its weight loads run ahead of the
//     waits (they do not depend on h).
// The down projection therefore streams while gate/up is still producing later segments,
// and the MLP is one launch instead of two.  Every row is summed in the same order as the
// two-launch chain (mlxr_qgemm_swiglu, then the down GEMV), so the results equal it bit for
// bit.
//
// Synchronisation without cache maintenance: h is written with device-scope stores
// (through the XCD's L2) and read with device-scope loads, and the counters are
// device-scope atomics, so no L2 write-back or invalidation is issued (a release and an
// acquire fence per workgroup cost about 0.15 ms per launch on MI355X).  A workgroup
// counts in an iteration only once its h stores are complete: the vector-memory counter
// retires in order on gfx9, and by the end of iteration k+delta every wavefront has waited
// for weight loads it issued after its iteration-k store (delta = 1, or 2 when a row has a
// single segment and the loads in flight reach past one iteration).  Counters that
// hundreds of workgroups hit are two-level trees of counters 256 bytes apart (device-scope
// atomics on one address serialise at the memory side), and each go flag is polled in
// several copies.
//
// Forward progress does not depend on residency: every down workgroup has a higher id than
// every gate/up workgroup and workgroups are dispatched in id order, and gate/up
// workgroups never wait.  The waits are bounded all the same: past `spin_limit` ticks of
// the 100 MHz real-time counter a down workgroup records an error flag in the workspace
// and stops waiting (its output is then wrong, the launch still ends);
// mlxr_qgemm_mlp_status reports the flag and re-initialises the sync region.
//
// The sync region resets itself: the last member of each counter returns it to zero, and
// the last down workgroup past its final wait lowers every go flag, so a replayed graph
// finds it zeroed.  It must be zero before the first use (mlxr_qgemm_mlp_workspace_init);
// calls sharing a workspace must not overlap.  Every wavefront of a workgroup runs the same
// number of chunks (rows past the end are masked), so the workgroup barriers inside the
// walks always pair up.
#include <algorithm>
#include <atomic>

#include "../../include/mlxr_qgemm.h"
#include "qgemm_gemv_common.h"

namespace mlxr {

namespace {

// Cache policy of device-scope loads (sc1): served from the coherent memory side, not from
// an XCD's L2 that may hold a stale copy.
constexpr int POL_DEVICE = 16;

struct MlpRole {
  PlanePtrs P;
  uint32_t psize[4];
};

struct MlpParams {
  const void* x;   // [1, H] activations
  void* h;         // [1, I] gated intermediate, activation type (workspace)
  void* y;         // [1, H] output
  unsigned* sync;  // sync region (kMlpSyncWords words)
  int H, I, y_dtype;
  uint32_t cmask, cmagic;
  MlpRole gate, up, down;
  int G1, KA, delta;  // gate/up workgroups, iterations, arrival delay (iterations)
  int rpw_b, G2;      // down: rows per wavefront, workgroups
  uint32_t spin_limit;
};

// VMEM instructions load_chunk issues per chunk.
template <int QT>
constexpr int chunk_loads() {
  return QT == QT_Q6_K ? 4 : (QT == QT_Q5_K || QT == QT_Q8_0) ? 3 : 2;
}

// Plane bases and sizes of up to two weights; the buffer descriptors are built per chunk
// from the selected plane (scalar selects): an array of descriptors indexed by a uniform
// loop state is demoted to scratch by the compiler.
template <int NW>
struct Planes {
  const uint8_t* base[NW][4];
  uint32_t size[NW][4];
  __device__ __forceinline__ void set(int w, const MlpRole& r, const void* fallback) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      base[w][i] = r.P.p[i] ? r.P.p[i] : (const uint8_t*)fallback;
      size[w][i] = r.psize[i];
    }
  }
  __device__ __forceinline__ void rsrc(bool second, rsrc_t* R) const {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      R[i] = make_rsrc((NW > 1 && second) ? base[NW - 1][i] : base[0][i],
                       (NW > 1 && second) ? size[NW - 1][i] : size[0][i]);
  }
};

__device__ __forceinline__ unsigned* slot(unsigned* sync, int s) { return sync + kMlpSlotWords * s; }
__device__ __forceinline__ void sync_store(unsigned* sync, int s, unsigned v) {
  __hip_atomic_store(slot(sync, s), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts member `idx` of `total` in: a two-level tree, nsub first-level counters (idx %
// nsub) whose last member resets its counter and counts in at the top counter, whose last
// member resets it.  Returns true for exactly one caller, the last of all.
__device__ __forceinline__ bool count_in(unsigned* sync, int sub_slot, int nsub, int top_slot, int idx, int total) {
  const int j = idx % nsub;
  const unsigned members = (unsigned)((total - j + nsub - 1) / nsub);
  unsigned* c = slot(sync, sub_slot + j);
  if (__hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != members - 1) return false;
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned groups = (unsigned)min(total, nsub);
  unsigned* t = slot(sync, top_slot);
  if (__hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != groups - 1) return false;
  __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Go-flag copies in use: each has a down workgroup polling it, so the last one past its
// final wait has seen every copy raised before it lowers them.
__device__ __forceinline__ int go_copies(const MlpParams& p) { return min(p.G2, kMlpGoCopies); }

// Segment s of h has received every gate/up row (called by one thread of the last
// workgroup to count in).
__device__ __forceinline__ void arrive(const MlpParams& p, int group) {
  const int s = group / 512;  // 4-row groups per 2048-value segment
  const int E = min(512, p.I / 4 - 512 * s);
  if (count_in(p.sync, kMlpSegSlots * s, kMlpSegSub, kMlpSegSlots * s + kMlpSegSub, group - 512 * s, E)) {
#pragma unroll 1
    for (int i = 0; i < go_copies(p); ++i) sync_store(p.sync, kMlpSegSlots * s + kMlpSegSub + 1 + i, 1u);
  }
}

template <int XT, int POL = POL_DEFAULT>
struct ActStage {
  rsrc_t RX;
  int nsub, T;
  uint4 va[4], vb[4];

  __device__ __forceinline__ void ld(int t, uint4* v) const {
    const uint32_t o = t < nsub ? (uint32_t)t * 64u : OOB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(RX, o + 16 * i, 0, POL);
      v[i] = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
  __device__ __forceinline__ void st(int t, const uint4* v, uint4* xs, float2* Xs) const {
    uint32_t xv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xs[((t >> 6) * 4 + i) * 64 + (t & 63)] = v[i];
      xv[4 * i + 0] = v[i].x;
      xv[4 * i + 1] = v[i].y;
      xv[4 * i + 2] = v[i].z;
      xv[4 * i + 3] = v[i].w;
    }
    float2 X;
    X.x = sum_range<XT, 0, 8>(xv);
    X.y = sum_range<XT, 8, 16>(xv);
    Xs[t] = X;
  }
  __device__ __forceinline__ void load(const void* a, int K) {
    nsub = K >> 5;
    T = ((nsub + 63) >> 6) * 64;
    RX = make_rsrc(a, (uint32_t)K * 2u);
    const int t = threadIdx.x;
    ld(t, va);
    if (T > 256) ld(t + 256, vb);
  }
  __device__ __forceinline__ void store(uint4* xs, float2* Xs) {
    const int t = threadIdx.x;
    if (t < T) st(t, va, xs, Xs);
    if (t + 256 < T) st(t + 256, vb, xs, Xs);
    for (int u = t + 512; u < T; u += 256) {
      uint4 v[4];
      ld(u, v);
      st(u, v, xs, Xs);
    }
  }
};

// Segment s of h (64 sub-blocks of 32 values) staged in LDS buffer xs/Xs with device-scope
// loads, by the first wavefront of the workgroup.
template <int XT>
__device__ __forceinline__ void stage_h_segment(const void* h, int I, int s, uint4* xs, float2* Xs) {
  const int t = threadIdx.x;
  if (t >= 64) return;
  const rsrc_t RH = make_rsrc(h, (uint32_t)I * 2u);
  const int sb = s * 64 + t;
  const uint32_t o = sb < (I >> 5) ? (uint32_t)sb * 64u : OOB;
  uint32_t xv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(RH, o + 16 * i, 0, POL_DEVICE);
    const uint4 v = make_uint4(q[0], q[1], q[2], q[3]);
    xs[i * 64 + t] = v;
    xv[4 * i + 0] = v.x;
    xv[4 * i + 1] = v.y;
    xv[4 * i + 2] = v.z;
    xv[4 * i + 3] = v.w;
  }
  float2 X;
  X.x = sum_range<XT, 0, 8>(xv);
  X.y = sum_range<XT, 8, 16>(xv);
  Xs[t] = X;
}

// Contribution of one chunk against one staged activation segment.
template <int QT, int XT>
__device__ __forceinline__ float chunk_dot(const CLoad<QT>& b, int lane, const uint4* xs, const float2* Xs,
                                           uint32_t MASK, uint32_t MAGIC) {
  WDec wd;
  decode_chunk<QT, XT>(b, lane & 7, MASK, MAGIC, wd);
  const uint4* xp = xs + lane;
  uint32_t xv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = xp[64 * i];
    xv[4 * i + 0] = v.x;
    xv[4 * i + 1] = v.y;
    xv[4 * i + 2] = v.z;
    xv[4 * i + 3] = v.w;
  }
  const float2 X = Xs[lane];
  return contrib<QT, XT>(xv, wd, X.x, X.y);
}

// ---- gate/up role: KA iterations of one row of gate and up per wavefront
template <int QT, int XT, int D>
__device__ __forceinline__ void role_gate_up(const MlpParams& p, uint8_t* smem, int lane, int wave, int bid) {
  const int K = p.H;
  const int nsub = K >> 5, nsb = K >> 8, nseg = (nsub + 63) >> 6;
  uint4* xs = (uint4*)smem;
  float2* Xs = (float2*)(smem + (size_t)nseg * 4096);
  Planes<2> W;
  W.set(0, p.gate, p.x);
  W.set(1, p.up, p.x);
  const int per = 2 * nseg;       // chunks per iteration: gate segments, then up segments
  const int C = p.KA * per;       // the same for every wavefront of the workgroup
  const int hdt = XT == X_BF16 ? DT_BF16 : DT_F16;
  auto row_of = [&](int k) { return 4 * (bid + p.G1 * k) + wave; };

  // issue cursor
  int ik = 0, ij = 0;
  auto issue = [&](CLoad<QT>& b) {
    const bool live = ik < p.KA;
    const int row = row_of(ik);
    const bool up = ij >= nseg;
    const int seg = up ? ij - nseg : ij;
    // row and segment are uniform (they set the scalar offset; selecting them with a
    // per-lane condition would make the compiler loop over lanes); the lane mask only
    // moves a lane's offset out of range
    const bool rok = live && row < p.I;
    const bool ok = rok && seg * 64 + lane < nsub;
    rsrc_t R[4];
    W.rsrc(up, R);
    load_chunk<QT, POL_NT>(R, rok ? row : 0, rok ? seg : 0, nsub, nsb, lane, ok, b);
    if (++ij == per) {
      ij = 0;
      ++ik;
    }
  };

  ActStage<XT> st;
  st.load(p.x, K);
  CLoad<QT> buf[D];
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(buf[d]);
  st.store(xs, Xs);
  __syncthreads();

  // consume cursor
  int k = 0, j = 0;
  float acc = 0.f, g = 0.f;
  auto consume = [&](const CLoad<QT>& b) {
    const int seg = j >= nseg ? j - nseg : j;
    acc += chunk_dot<QT, XT>(b, lane, xs + seg * 256, Xs + seg * 64, p.cmask, p.cmagic);
    if (j == nseg - 1) {
      g = wave_total(acc);
      acc = 0.f;
    }
    if (++j == per) {
      const float u = wave_total(acc);
      acc = 0.f;
      const int row = row_of(k);
      if (lane == 0 && row < p.I) {
        const float v = swiglu1(g, u);
        const uint16_t hb = hdt == DT_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        __hip_atomic_store((uint16_t*)p.h + row, hb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // iteration k - delta's stores are complete in every wavefront: count it in
      __syncthreads();
      if (threadIdx.x == 0 && k >= p.delta && 4 * (bid + p.G1 * (k - p.delta)) < p.I)
        arrive(p, bid + p.G1 * (k - p.delta));
      j = 0;
      ++k;
    }
  };
  int c = 0;
  for (; c + D <= C; c += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(buf[(d + D - 1) % D]);
      consume(buf[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (c + d < C) consume(buf[d]);
  // the last delta iterations: wait for every store, then count them in
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    for (int kk = max(0, p.KA - p.delta); kk < p.KA; ++kk)
      if (4 * (bid + p.G1 * kk) < p.I) arrive(p, bid + p.G1 * kk);
}

// ---- down role: rpw_b rows per wavefront, walked segment-major over h
template <int QT, int XT, int D, int RB>
__device__ __forceinline__ void role_down(const MlpParams& p, uint8_t* smem, int lane, int wave, int bid) {
  const int K = p.I;
  const int nsub = K >> 5, nsb = K >> 8, nseg = (nsub + 63) >> 6;
  const int b2 = bid - p.G1;
  const int rpw = p.rpw_b;  // <= RB
  const int r0 = (b2 * 4 + wave) * rpw;
  const int C = nseg * rpw;  // the same for every wavefront of the workgroup
  // two staging buffers of one segment each (4 KiB words + 512 B sums)
  uint4* xs0 = (uint4*)smem;
  Planes<1> W;
  W.set(0, p.down, p.x);
  rsrc_t R[4];
  W.rsrc(false, R);

  int is = 0, ir = 0;
  auto issue = [&](CLoad<QT>& b) {
    const int row = r0 + ir;
    const bool rok = is < nseg && ir < rpw && row < p.H;  // uniform (see role_gate_up)
    const bool ok = rok && is * 64 + lane < nsub;
    load_chunk<QT, POL_NT>(R, rok ? row : 0, rok ? is : 0, nsub, nsb, lane, ok, b);
    if (++ir == rpw) {
      ir = 0;
      ++is;
    }
  };
  CLoad<QT> buf[D];
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(buf[d]);

  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool gave_up = false;  // thread 0 only
  const int copy = b2 % go_copies(p);
  int s = 0, r = 0;
  float acc[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) acc[i] = 0.f;
  float res = 0.f;
  auto consume = [&](const CLoad<QT>& b) {
    uint4* xs = xs0 + (s & 1) * 288;  // 4608 bytes per buffer
    float2* Xs = (float2*)(xs + 256);
    if (r == 0) {
      // segment s: wait for its go flag, stage it
      if (threadIdx.x == 0 && !gave_up) {
        const unsigned* go = slot(p.sync, kMlpSegSlots * s + kMlpSegSub + 1 + copy);
        while (__hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
          __builtin_amdgcn_s_sleep(4);
          if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)p.spin_limit) {
            sync_store(p.sync, kMlpErr, 1u);
            gave_up = true;
            break;
          }
        }
        if (s == nseg - 1 && count_in(p.sync, kMlpDepartSub, kMlpDepartN, kMlpDepartTop, b2, p.G2)) {
          // every down workgroup is past every wait: lower the go flags for the next launch
#pragma unroll 1
          for (int ss = 0; ss < nseg; ++ss)
#pragma unroll 1
            for (int i = 0; i < go_copies(p); ++i) sync_store(p.sync, kMlpSegSlots * ss + kMlpSegSub + 1 + i, 0u);
        }
      }
      __syncthreads();
      stage_h_segment<XT>(p.h, K, s, xs, Xs);
      __syncthreads();
    }
    const float v = chunk_dot<QT, XT>(b, lane, xs, Xs, p.cmask, p.cmagic);
#pragma unroll
    for (int i = 0; i < RB; ++i)
      if (i == r) acc[i] += v;
    if (s == nseg - 1) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < RB; ++i)
        if (i == r) a = acc[i];
      const float tot = wave_total(a);
      res = lane == r ? tot : res;
    }
    if (++r == rpw) {
      r = 0;
      ++s;
    }
  };
  int c = 0;
  for (; c + D <= C; c += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(buf[(d + D - 1) % D]);
      consume(buf[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (c + d < C) consume(buf[d]);
  if (lane < rpw && r0 + lane < p.H) store_scalar(p.y, p.y_dtype, (size_t)(r0 + lane), res);
}

template <int QTG, int QTD, int XT, int DA, int DB, int RB>
__global__ __launch_bounds__(256) void qmlp_gemv_kernel(MlpParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bid = blockIdx.x;
  if (bid < p.G1) role_gate_up<QTG, XT, DA>(p, smem, lane, wave, bid);
  else role_down<QTD, XT, DB, RB>(p, smem, lane, wave, bid);
}

__global__ void mlp_sync_zero_kernel(unsigned* sync) {
  for (int i = threadIdx.x; i < kMlpSyncWords; i += blockDim.x) sync[i] = 0u;
}

size_t act_lds_bytes(int K) { return (size_t)(((K >> 5) + 63) >> 6) * 64 * 72; }

std::atomic<uint32_t> g_spin_limit{20000000u};  // 0.2 s of the 100 MHz counter

MlpRole role_of(const PackedLayout& L, const void* packed) {
  MlpRole r;
  r.P = plane_ptrs(L, (const uint8_t*)packed);
  for (int k = 0; k < 4; ++k) r.psize[k] = k < L.nplanes ? (uint32_t)L.size[k] : 0u;
  return r;
}

constexpr int kDA = 3, kDB = 3, kRB = 4;  // loads in flight (chunks) per role; down rows per wavefront

template <int QTG, int QTD, int XT>
hipError_t launch_t(const MlpParams& p, unsigned grid, size_t lds, hipStream_t s) {
  auto k = qmlp_gemv_kernel<QTG, QTD, XT, kDA, kDB, kRB>;
  static std::atomic<uint64_t> attr{0};
  if (lds > 65536) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(attr.load(std::memory_order_acquire) & bit)) {
      const hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)device_lds_limit());
      if (e != hipSuccess) return e;
      attr.fetch_or(bit, std::memory_order_release);
    }
  }
  k<<<dim3(grid), dim3(256), lds, s>>>(p);
  return hipGetLastError();
}

template <int QTG, int XT>
hipError_t launch_qtd(const MlpParams& p, int qtd, unsigned grid, size_t lds, hipStream_t s) {
  if (qtd == QTG) return launch_t<QTG, QTG, XT>(p, grid, lds, s);
  if constexpr (QTG != QT_Q6_K) {
    if (qtd == QT_Q6_K) return launch_t<QTG, QT_Q6_K, XT>(p, grid, lds, s);
  }
  return hipErrorInvalidValue;
}

template <int XT>
hipError_t launch_x(const MlpParams& p, int qtg, int qtd, unsigned grid, size_t lds, hipStream_t s) {
  switch (qtg) {
    case QT_Q4_K: return launch_qtd<QT_Q4_K, XT>(p, qtd, grid, lds, s);
    case QT_Q6_K: return launch_qtd<QT_Q6_K, XT>(p, qtd, grid, lds, s);
    case QT_Q5_K: return launch_qtd<QT_Q5_K, XT>(p, qtd, grid, lds, s);
    case QT_Q4_0: return launch_qtd<QT_Q4_0, XT>(p, qtd, grid, lds, s);
    case QT_Q4_1: return launch_qtd<QT_Q4_1, XT>(p, qtd, grid, lds, s);
    default: return launch_qtd<QT_Q8_0, XT>(p, qtd, grid, lds, s);
  }
}

}  // namespace

bool mlp_fused_ok(const MlpArgs& a) {
  if (a.M != 1) return false;
  if (a.qtd != a.gate.qtype && a.qtd != QT_Q6_K) return false;
  if ((((a.I >> 5) + 63) >> 6) > kMlpMaxSeg || (a.I & 3)) return false;
  const size_t lim = operand_limit();
  for (const PackedLayout* L : {&a.gate, &a.up, &a.down})
    for (int i = 0; i < L->nplanes; ++i)
      if (L->size[i] >= lim) return false;
  return act_lds_bytes(a.H) <= device_lds_limit() && (size_t)a.H * 2 < lim && (size_t)a.I * 2 < lim;
}

hipError_t launch_mlp_fused(const MlpArgs& a, hipStream_t s) {
  MlpParams p;
  p.x = a.x;
  p.h = a.h;
  p.y = a.y;
  p.sync = a.sync;
  p.H = a.H;
  p.I = a.I;
  p.y_dtype = a.y_dtype;
  p.cmask = 0x000F000Fu;
  p.cmagic = a.x_dtype == DT_F16 ? 0x64006400u : 0x43004300u;
  p.gate = role_of(a.gate, a.gate_packed);
  p.up = role_of(a.up, a.up_packed);
  p.down = role_of(a.down, a.down_packed);
  const long cus = device_cu_count();
  // gate/up: about 16 wavefronts per CU, one row of gate and up each per iteration, the
  // iteration count chosen so the last iteration is (nearly) full
  const long target_a = cus * 16;
  p.KA = (int)std::max<long>(1, (a.I + target_a - 1) / target_a);
  const long rows_per_iter = (a.I + p.KA - 1) / p.KA;
  p.G1 = (int)((rows_per_iter + 3) / 4);
  const int nseg_h = ((a.H >> 5) + 63) >> 6;
  p.delta = (kDA + 2 * nseg_h - 1) / (2 * nseg_h);
  // down: about 8 wavefronts per CU, at most kRB rows each
  const long target_b = cus * 8;
  p.rpw_b = (int)std::min<long>(kRB, std::max<long>(1, (a.H + target_b - 1) / target_b));
  p.G2 = (int)(((a.H + p.rpw_b - 1) / p.rpw_b + 3) / 4);
  p.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  const size_t lds = std::max(act_lds_bytes(a.H), (size_t)2 * 4608);
  const unsigned grid = (unsigned)(p.G1 + p.G2);
  return a.x_dtype == DT_F16 ? launch_x<X_F16>(p, a.gate.qtype, a.qtd, grid, lds, s)
                             : launch_x<X_BF16>(p, a.gate.qtype, a.qtd, grid, lds, s);
}

hipError_t launch_mlp_sync_zero(unsigned* sync, hipStream_t s) {
  mlp_sync_zero_kernel<<<dim3(1), dim3(256), 0, s>>>(sync);
  return hipGetLastError();
}

void set_mlp_spin_limit(uint32_t ticks) { g_spin_limit.store(ticks, std::memory_order_relaxed); }

}  // namespace mlxr
