// Internal launcher interface between the C ABI (qgemm_api.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>

#include "qgemm_layout.h"

namespace mlxr {

struct PlanePtrs {
  const uint8_t* p[4];
};

inline PlanePtrs plane_ptrs(const PackedLayout& L, const uint8_t* base) {
  PlanePtrs P;
  for (int i = 0; i < 4; ++i) P.p[i] = (i < L.nplanes) ? base + L.off[i] : nullptr;
  return P;
}

// Arguments of one Y = X . W^T (+ bias) call, validated by the caller.
struct RunArgs {
  PackedLayout L;
  const uint8_t* packed;
  const void* x;
  int x_dtype;
  const void* bias;  // may be null
  int bias_dtype;
  void* y;
  int y_dtype;
  int M;
  void* ws = nullptr;    // caller's device workspace for split-K partials (may be null)
  size_t ws_bytes = 0;
};

// Sets the calling thread's mlxr_qgemm_last_error message; returns code.
int set_error(int code, const char* fmt, ...);

hipError_t launch_pack(const PackedLayout& L, const uint8_t* gguf_dev, uint8_t* packed_dev,
                       hipStream_t s);
hipError_t launch_dequant(const PackedLayout& L, const uint8_t* packed_dev, void* out,
                          int out_dtype, hipStream_t s);

// Wavefront-reduction GEMV / skinny GEMM, no MFMA.  Requires 1 <= M <= 64.
hipError_t launch_gemv(const RunArgs& a, hipStream_t s);

// Several weights that share K, quant type, activations and M (<= 4) in one launch;
// gemv_groupable() tells whether an item qualifies.  n <= 4.
bool gemv_groupable(const RunArgs& a);
hipError_t launch_gemv_grouped(const RunArgs* const* items, int n, hipStream_t s);
// gate and up (same type and shape, both groupable) in one launch storing
// swish(x.gate^T) * (x.up^T) into gate.y.
hipError_t launch_gemv_swiglu(const RunArgs& gate, const RunArgs& up, hipStream_t s);

// MFMA GEMM (qgemm_tile.hip).  Any M >= 1 (rows beyond M are masked).  With a.ws, shapes
// with too few tiles for the device split K over workgroups (fp32 partials in a.ws).
hipError_t launch_mfma(const RunArgs& a, hipStream_t s);
// Workspace bytes launch_mfma would use for an [M, N, K] problem (0: no split).
size_t mfma_workspace_bytes(int M, int N, int K);
// Up to 4 weights of one quant type and K sharing x and M in one tiled launch (their tile
// columns side by side; split-K over the concatenated N when ws holds the partials).
// mfma_groupable() tells whether an item qualifies (every operand below 2 GiB).
bool mfma_groupable(const RunArgs& a);
hipError_t launch_mfma_grouped(const RunArgs* const* items, int n, void* ws, size_t ws_bytes, hipStream_t s);
size_t mfma_grouped_workspace_bytes(const RunArgs* const* items, int n);

// Largest operand (activations, weight plane) the 32-bit-offset kernels address in one
// launch: 2 GiB.  Test hook: mlxr_qgemm_test_set_operand_limit lowers it (an atomic), so the
// tests reach the chunked and fallback launches at small sizes.
size_t operand_limit();
// Compute units of the current device, queried once per device.
int device_cu_count();
// LDS a workgroup may use on the current device once a kernel's limit is raised: the
// device's opt-in maximum, at most 160 KiB (gfx950), queried once per device.
size_t device_lds_limit();

// Skinny MFMA GEMM for M <= 64 (qgemm_skinny.hip), weights streamed once.  With a.ws,
// shapes with fewer 32-row slabs than CUs also split K over workgroups.
hipError_t launch_skinny(const RunArgs& a, hipStream_t s);
// Whether the narrow skinny kernel stages its activations in LDS where they fit (default 1;
// test hook mlxr_qgemm_test_skinny_stage).
extern std::atomic<int> g_skinny_stage;
// Whether every operand of a is below operand_limit() (else: launch_mfma, which chunks).
bool skinny_fits(const RunArgs& a);
// Workspace bytes launch_skinny would use (0: no split).
size_t skinny_workspace_bytes(int M, int N, int K, int qtype);
// Estimated time of launch_skinny for M > 32 (64-row blocks of M over a second grid
// dimension) and of launch_mfma with a workspace of ws_bytes, in microseconds.
double skinny_mb_est_us(int M, int N, int K);
double mfma_est_us(int M, int N, int K, int qtype, size_t ws_bytes);
// SwiGLU, h = swish(x.gate^T + bias_g) * (x.up^T + bias_u) into gate.y, with gate and up
// of one type and shape; gate.ws / ws (may be null) holds split-K partials.
// Narrow skinny kernel (M <= 32, skinny_swiglu_ok) and tiled kernel (any M; operands
// below 2 GiB, mfma_groupable; no biases).
bool skinny_swiglu_ok(int M);
hipError_t launch_skinny_swiglu(const RunArgs& gate, const RunArgs& up, hipStream_t s);
size_t skinny_swiglu_workspace_bytes(int M, int N, int K);
hipError_t launch_mfma_swiglu(const RunArgs& gate, const RunArgs& up, void* ws, size_t ws_bytes, hipStream_t s);
size_t mfma_swiglu_workspace_bytes(int M, int N, int K);
// h[m][n] = swish(sum gate + bias_g) * (sum up + bias_u) over S partial planes whose rows
// hold gate (columns 0 .. N-1) then up (N .. 2N-1) (qgemm_tile.hip).
hipError_t launch_splitk_reduce_swiglu(const float* ws, size_t split_elems, int S, const void* bias_g,
                                       const void* bias_u, int bias_dtype, void* y, int y_dtype, int M, int N,
                                       hipStream_t s);
// y = sum of S fp32 partial planes (split order) + bias, converted (qgemm_tile.hip).
hipError_t launch_splitk_reduce(const float* ws, size_t split_elems, int S, const void* bias, int bias_dtype, void* y,
                                int y_dtype, int M, int N, hipStream_t s);

// Fused SwiGLU MLP (qgemm_mlp.hip): y = down(swish(x . gate^T) * (x . up^T)).
// Sync region at the start of its workspace, one word per 256-byte slot: for each of up
// to kMlpMaxSeg segments of h, kMlpSegSub arrival counters, their top counter and
// kMlpGoCopies go flags; then kMlpDepartN departure counters, their top counter and the
// error flag.
constexpr int kMlpSlotWords = 64;
constexpr int kMlpMaxSeg = 32, kMlpSegSub = 8, kMlpGoCopies = 8;
constexpr int kMlpSegSlots = kMlpSegSub + 1 + kMlpGoCopies;
constexpr int kMlpDepartSub = kMlpMaxSeg * kMlpSegSlots, kMlpDepartN = 32;
constexpr int kMlpDepartTop = kMlpDepartSub + kMlpDepartN, kMlpErr = kMlpDepartTop + 1;
constexpr int kMlpSlots = 640;  // kMlpErr + 1 rounded up
static_assert(kMlpErr < kMlpSlots, "sync region");
constexpr int kMlpSyncWords = kMlpSlots * kMlpSlotWords;  // 160 KiB
struct MlpArgs {
  PackedLayout gate, up, down;  // gate/up [I, H], down [H, I]
  int qtd;                      // down's quant type (gate's, or Q6_K)
  const void *gate_packed, *up_packed, *down_packed;
  const void* x;  // [M, H]
  int x_dtype;
  void* h;  // [M, I] in the activation type (workspace)
  void* y;  // [M, H]
  int y_dtype;
  unsigned* sync;  // kMlpSyncWords words, zero between calls
  int M, H, I;
};
// Whether the one-launch kernel serves the call (M = 1, down of gate's type or Q6_K,
// operands below 2 GiB, activations fit LDS, at most kMlpMaxSeg segments of h).
bool mlp_fused_ok(const MlpArgs& a);
hipError_t launch_mlp_fused(const MlpArgs& a, hipStream_t s);
// Zeroes the sync words with a kernel (no memset node in a captured graph).
hipError_t launch_mlp_sync_zero(unsigned* sync, hipStream_t s);
// Bound of the down workgroups' wait, in ticks of the 100 MHz real-time counter.
void set_mlp_spin_limit(uint32_t ticks);

}  // namespace mlxr
