// extern "C" boundary of libmlxr_qgemm.so (declared in include/mlxr_qgemm.h).
//
// Validation and error behaviour follow the reference operator
// (core/kernels/primitives/q_gemm_dequant_primitive.mm:478-522 shape checks,
// :76/:133/:340 unsupported types) but as status codes plus a thread-local message:
// no exception crosses the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <vector>

#include "../../include/mlxr_qgemm.h"
#include "qgemm_internal.h"

namespace {

// Largest M the automatic path sends to the GEMV kernel.
constexpr int kGemvMaxM = 4;
// Whether the automatic path runs a call with M <= kGemvMaxM on the GEMV kernel.  The GEMV
// stages all M rows of X per workgroup (M = 3, 4 as four rows), so long rows cost it LDS
// and occupancy; the skinny MFMA kernel's time hardly depends on M.  Measured on MI355X
// (µs, GEMV / skinny MFMA without a K split): Llama-3-8B down (4096 x 14336) at M = 3 and
// 4: 22.1 / 21.3 and 24.9 / 21.8 (the skinny one splits K with a workspace: about 17.5);
// gate (14336 x 4096) at M = 4 16.5 / 15.1 and at M = 3 14.5 / 14.9; Llama-3-70B down (8192
// x 28672) at M = 2 51.2 / 38.9; 4096 x 4096 at M = 4 7.4 / 9.8; the Q6_K lm_head (128256 x
// 4096) at M = 4 116 / 146.
bool gemv_auto(int M, const mlxr::PackedLayout& L) {
  if (M <= 1) return true;
  if (M > kGemvMaxM) return false;
  if (M >= 3 && L.K >= 8192) return false;
  if (M == 2 && L.K >= 16384) return false;
  if (M == 4 && (long)L.N * (long)L.K >= (48L << 20) && L.qtype != mlxr::QT_Q6_K) return false;
  return true;
}
// Up to this M the skinny kernel serves every MFMA call (measured on MI355X, Llama-3-8B
// FFN shapes: at M = 32 its 16x16x32 variant is ahead of the tiled GEMM with 64-row tiles
// and split-K, gate 26.9 vs 29.0 us and down 26.7 vs 29.7 us; at M = 64 the tiled one,
// gate 28.3 vs 42.7 us).
constexpr int kSkinnyOnlyMaxM = 32;
int skinny_only_max_m() { return kSkinnyOnlyMaxM; }
// Up to this M a single call chooses between the skinny kernel (in 64-row blocks of M)
// and the tiled one by their estimated times: on MI355X the skinny one wins for narrow
// weights, e.g. Llama-3-8B k/v at M = 128: 12.3 against 18.6 us.
constexpr int kSkinnyMaxM = 256;

// For skinny_only_max_m() < M <= kSkinnyMaxM: whether the skinny kernel serves a call that
// has the workspace the library asks for (ws) or none.  Without one the skinny kernel
// takes M <= 64 and the tiled one (unsplit) larger M.
bool skinny_mid(int M, const mlxr::PackedLayout& L, bool ws) {
  if (!ws) return M <= 64;
  return mlxr::skinny_mb_est_us(M, L.N, L.K) < mlxr::mfma_est_us(M, L.N, L.K, L.qtype, ~(size_t)0);
}
// The workspace size for those M: that of the kernel skinny_mid picks with one.
void mid_workspace(int M, const mlxr::PackedLayout& L, size_t* bytes) {
  *bytes = skinny_mid(M, L, true) ? mlxr::skinny_workspace_bytes(M, L.N, L.K, L.qtype)
                                  : mlxr::mfma_workspace_bytes(M, L.N, L.K);
}
std::atomic<int> g_force_skinny{0};

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace

namespace mlxr {

namespace {
// 2 GiB unless a test lowered it (mlxr_qgemm_test_set_operand_limit)
std::atomic<size_t> g_operand_limit{(size_t)1 << 31};
}  // namespace

size_t operand_limit() { return g_operand_limit.load(std::memory_order_relaxed); }

int device_cu_count() {
  constexpr int kDev = 64;
  static std::atomic<int> cache[kDev];  // 0: not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDev) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

size_t device_lds_limit() {
  constexpr int kDev = 64;
  static std::atomic<uint32_t> cache[kDev];  // 0: not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDev) return 64 * 1024;
  uint32_t v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int a = 0;
    if (hipDeviceGetAttribute(&a, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess || a <= 0)
      a = 64 * 1024;
    v = (uint32_t)std::min(a, 160 * 1024);
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace mlxr

namespace {

int hip_fail(hipError_t e, const char* where) {
  return fail(MLXR_E_HIP, "%s: HIP error %d (%s)", where, (int)e, hipGetErrorString(e));
}

bool implemented(int qtype) {
  return qtype == MLXR_Q4_0 || qtype == MLXR_Q4_1 || qtype == MLXR_Q8_0 || qtype == MLXR_Q4_K || qtype == MLXR_Q5_K ||
         qtype == MLXR_Q6_K;
}

int check_type_shape(int qtype, int N, int K, mlxr::PackedLayout* L) {
  if (qtype < 0 || qtype > MLXR_IQ3_S) return fail(MLXR_E_INVALID, "invalid quant type %d", qtype);
  if (!implemented(qtype))
    return fail(MLXR_E_UNSUPPORTED, "Unsupported quantization type %s", mlxr_qgemm_type_name(qtype));
  if (N <= 0 || K <= 0) return fail(MLXR_E_INVALID, "N and K must be positive (N=%d, K=%d)", N, K);
  const int g = mlxr::gguf_block_elems(qtype);
  if (K % g != 0)
    return fail(MLXR_E_SHAPE, "K=%d is not a multiple of the %s block size %d", K,
                mlxr_qgemm_type_name(qtype), g);
  if (!mlxr::make_layout(qtype, N, K, L)) return fail(MLXR_E_SHAPE, "cannot lay out %dx%d", N, K);
  return MLXR_OK;
}

bool valid_dtype(int dt) { return dt == MLXR_F32 || dt == MLXR_F16 || dt == MLXR_BF16; }

}  // namespace

extern "C" {

int mlxr_qgemm_version(void) { return 10000; }

const char* mlxr_qgemm_last_error(void) { return g_err.c_str(); }

const char* mlxr_qgemm_type_name(int qtype) {
  static const char* names[] = {"Q4_0", "Q4_1", "Q8_0",    "Q4_K",   "Q6_K",    "Q5_0",
                                "Q5_1", "Q8_1", "Q2_K",    "Q3_K",   "Q5_K",    "Q8_K",
                                "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ3_S"};
  if (qtype < 0 || qtype > 15) return "Unknown";
  return names[qtype];
}

int mlxr_qgemm_group_size(int qtype) {
  // reference get_default_group_size (.mm:80-92): 256 for Q4_K/Q6_K, 32 otherwise.  Q5_K,
  // which the reference never runs (its default would be 32), takes its GGUF super-block.
  return (qtype == MLXR_Q4_K || qtype == MLXR_Q5_K || qtype == MLXR_Q6_K) ? 256 : 32;
}

int mlxr_qgemm_gguf_size(int qtype, int N, int K, size_t* bytes) {
  if (!bytes) return fail(MLXR_E_INVALID, "bytes is null");
  if (N <= 0 || K <= 0) return fail(MLXR_E_INVALID, "N and K must be positive (N=%d, K=%d)", N, K);
  const int g = mlxr::gguf_block_elems(qtype), bb = mlxr::gguf_block_bytes(qtype);
  if (g == 0) return fail(MLXR_E_UNSUPPORTED, "Unsupported quantization type %s", mlxr_qgemm_type_name(qtype));
  *bytes = (size_t)N * (size_t)((K + g - 1) / g) * (size_t)bb;
  return MLXR_OK;
}

int mlxr_qgemm_packed_size(int qtype, int N, int K, size_t* bytes) {
  if (!bytes) return fail(MLXR_E_INVALID, "bytes is null");
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  *bytes = L.total;
  return MLXR_OK;
}

int mlxr_qgemm_pack_device(int qtype, int N, int K, const void* gguf_dev, void* packed_dev,
                           void* stream) {
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!gguf_dev || !packed_dev) return fail(MLXR_E_INVALID, "null buffer");
  const hipError_t e = mlxr::launch_pack(L, (const uint8_t*)gguf_dev, (uint8_t*)packed_dev, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "pack launch");
  return MLXR_OK;
}

int mlxr_qgemm_pack(int qtype, int N, int K, const void* gguf_host, void* packed_dev, void* stream) {
  mlxr::PackedLayout L;
  int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!gguf_host || !packed_dev) return fail(MLXR_E_INVALID, "null buffer");
  size_t bytes = 0;
  mlxr_qgemm_gguf_size(qtype, N, K, &bytes);
  hipStream_t s = (hipStream_t)stream;
  void* staging = nullptr;
  hipError_t e = hipMalloc(&staging, bytes);
  if (e != hipSuccess) return fail(MLXR_E_NOMEM, "staging allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
  e = hipMemcpyAsync(staging, gguf_host, bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = mlxr::launch_pack(L, (const uint8_t*)staging, (uint8_t*)packed_dev, s);
  const hipError_t es = hipStreamSynchronize(s);
  (void)hipFree(staging);
  if (e != hipSuccess) return hip_fail(e, "pack");
  if (es != hipSuccess) return hip_fail(es, "pack sync");
  return MLXR_OK;
}

int mlxr_qgemm_dequant(int qtype, int N, int K, const void* packed_dev, void* out_dev, int out_dtype,
                       void* stream) {
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!packed_dev || !out_dev) return fail(MLXR_E_INVALID, "null buffer");
  if (out_dtype != MLXR_F32 && out_dtype != MLXR_BF16)
    return fail(MLXR_E_INVALID, "dequant output dtype must be F32 or BF16 (got %d)", out_dtype);
  const hipError_t e = mlxr::launch_dequant(L, (const uint8_t*)packed_dev, out_dev, out_dtype, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dequant launch");
  return MLXR_OK;
}

int mlxr_qgemm_workspace_size(int qtype, int N, int K, int M, size_t* bytes) {
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!bytes) return fail(MLXR_E_INVALID, "null output pointer");
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  if (M > skinny_only_max_m() && M <= kSkinnyMaxM)
    mid_workspace(M, L, bytes);
  else
    *bytes = M > skinny_only_max_m() ? mlxr::mfma_workspace_bytes(M, N, K)
             : !gemv_auto(M, L)      ? mlxr::skinny_workspace_bytes(M, N, K, qtype)
                                     : 0;
  return MLXR_OK;
}

int mlxr_qgemm_auto_path(int qtype, int N, int K, int M, int* path) {
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!path) return fail(MLXR_E_INVALID, "null output pointer");
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  *path = gemv_auto(M, L) ? MLXR_PATH_GEMV : MLXR_PATH_MFMA;
  return MLXR_OK;
}

int mlxr_qgemm_run_ex(int qtype, int N, int K, int group_size, const void* packed_dev, const void* x_dev,
                      int x_dtype, const void* bias_dev, int bias_dtype, void* y_dev, int y_dtype, int M,
                      int path, void* stream) {
  return mlxr_qgemm_run_ws(qtype, N, K, group_size, packed_dev, x_dev, x_dtype, bias_dev, bias_dtype, y_dev, y_dtype,
                           M, path, nullptr, 0, stream);
}

int mlxr_qgemm_run_ws(int qtype, int N, int K, int group_size, const void* packed_dev, const void* x_dev,
                      int x_dtype, const void* bias_dev, int bias_dtype, void* y_dev, int y_dtype, int M,
                      int path, void* workspace_dev, size_t workspace_bytes, void* stream) {
  mlxr::RunArgs a;
  int rc = check_type_shape(qtype, N, K, &a.L);
  if (rc) return rc;
  if (group_size != 0 && group_size != mlxr_qgemm_group_size(qtype))
    return fail(MLXR_E_SHAPE, "group_size %d does not match %s (block of %d)", group_size,
                mlxr_qgemm_type_name(qtype), mlxr_qgemm_group_size(qtype));
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  if (x_dtype != MLXR_BF16 && x_dtype != MLXR_F16)
    return fail(MLXR_E_INVALID, "activation dtype must be BF16 or F16 (got %d)", x_dtype);
  if (!valid_dtype(y_dtype)) return fail(MLXR_E_INVALID, "invalid output dtype %d", y_dtype);
  if (bias_dev && !valid_dtype(bias_dtype)) return fail(MLXR_E_INVALID, "invalid bias dtype %d", bias_dtype);
  if (path < MLXR_PATH_AUTO || path > MLXR_PATH_MFMA) return fail(MLXR_E_INVALID, "invalid path %d", path);
  if (M == 0) return MLXR_OK;
  if (!packed_dev || !x_dev || !y_dev) return fail(MLXR_E_INVALID, "null buffer");
  if (path == MLXR_PATH_GEMV && M > 64)
    return fail(MLXR_E_INVALID, "the GEMV path takes M <= 64 (M=%d)", M);
  a.packed = (const uint8_t*)packed_dev;
  a.x = x_dev;
  a.x_dtype = x_dtype;
  a.bias = bias_dev;
  a.bias_dtype = bias_dtype;
  a.y = y_dev;
  a.y_dtype = y_dtype;
  a.M = M;
  a.ws = workspace_dev;
  a.ws_bytes = workspace_dev ? workspace_bytes : 0;
  // GEMV (no MFMA) for decode (gemv_auto); MFMA kernels otherwise: the skinny one up to
  // M = 32, then up to M = 256 the skinny or the tiled one (skinny_mid), the tiled one above
  // (MLXR_PATH_GEMV / MLXR_PATH_MFMA force the family)
  const bool gemv = path == MLXR_PATH_GEMV || (path == MLXR_PATH_AUTO && gemv_auto(M, a.L));
  // the skinny kernels address operands with 32-bit offsets; the tiled launcher splits
  // larger problems into chunks
  bool skinny = false;
  if (!gemv && g_force_skinny.load(std::memory_order_relaxed)) {
    skinny = mlxr::skinny_fits(a);
  } else if (!gemv && M <= skinny_only_max_m()) {
    skinny = mlxr::skinny_fits(a);
  } else if (!gemv && M <= kSkinnyMaxM) {
    // a workspace below the size mlxr_qgemm_workspace_size asks for is not used; a call
    // whose size is 0 has what it asks for, with or without one
    size_t need = 0;
    mid_workspace(M, a.L, &need);
    const bool ws_ok = need == 0 || (a.ws && a.ws_bytes >= need);
    if (!ws_ok) {
      a.ws = nullptr;
      a.ws_bytes = 0;
    }
    skinny = mlxr::skinny_fits(a) && skinny_mid(M, a.L, ws_ok);
  }
  hipError_t e;
  if (gemv) e = mlxr::launch_gemv(a, (hipStream_t)stream);
  else if (skinny) e = mlxr::launch_skinny(a, (hipStream_t)stream);
  else e = mlxr::launch_mfma(a, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, gemv ? "gemv launch" : "mfma launch");
  return MLXR_OK;
}

}  // extern "C"

namespace {

// Whether a grouped call at M <= kGemvMaxM keeps an item in a grouped GEMV launch: where the
// automatic path would run it on the GEMV, and also where it would not unless the weight is
// very large (N*K >= 128 Mi): sharing one launch beats a skinny launch of its own for the
// others (measured on MI355X, µs, grouped GEMV / items the automatic path gives the skinny
// kernel on it: Llama-3-70B q,k at M = 3 20.3 / 23.0, with v 26.5 / 23.9; gate/up at M = 3 /
// 4 94.4 / 105.7 grouped, 90.1 / 91.3 each on the skinny kernel).
bool grouped_gemv(int M, const mlxr::RunArgs& a) {
  return mlxr::gemv_groupable(a) && (gemv_auto(M, a.L) || (long)a.L.N * (long)a.L.K < (128L << 20));
}

// How a grouped call runs its items: launches of several items (GEMV at M <= 4, tiled MFMA
// where the tiled kernel serves the call) and single calls for the rest.
struct Batch {
  int kind;  // 0 single call, 1 grouped GEMV, 2 grouped tiled MFMA
  int idx[4];
  int n;
};
std::vector<Batch> plan_batches(const std::vector<mlxr::RunArgs>& a, int M, bool with_ws) {
  const int count = (int)a.size();
  const bool tiled = M > 64 || (M > skinny_only_max_m() && with_ws);
  std::vector<bool> done((size_t)count, false);
  std::vector<Batch> out;
  for (int i = 0; i < count; ++i) {
    if (done[i]) continue;
    const int kind = (M <= kGemvMaxM && grouped_gemv(M, a[i])) ? 1 : (tiled && mlxr::mfma_groupable(a[i])) ? 2 : 0;
    Batch bt{kind, {i, 0, 0, 0}, 1};
    done[i] = true;
    if (kind != 0) {
      for (int j = i + 1; j < count && bt.n < 4; ++j) {
        if (done[j] || a[j].L.qtype != a[i].L.qtype) continue;
        if (kind == 1 ? !grouped_gemv(M, a[j]) : !mlxr::mfma_groupable(a[j])) continue;
        bt.idx[bt.n++] = j;
        done[j] = true;
      }
    }
    out.push_back(bt);
  }
  return out;
}

// Validates the items (each exactly as a single call) and fills their run arguments.
int grouped_args(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M, bool need_ptrs,
                 void* stream, std::vector<mlxr::RunArgs>& a) {
  if (count < 0 || (count > 0 && !items)) return fail(MLXR_E_INVALID, "invalid item list");
  a.resize((size_t)count);
  if (count == 0) return MLXR_OK;
  const int K = items[0].K;
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  for (int i = 0; i < count; ++i) {
    const mlxr_qgemm_item& it = items[i];
    if (it.K != K) return fail(MLXR_E_SHAPE, "grouped items must share K (item %d has K=%d, item 0 K=%d)", i, it.K, K);
    if (need_ptrs) {
      // full validation of each item, exactly as a single call would do it
      int rc = mlxr_qgemm_run_ex(it.qtype, it.N, it.K, it.group_size, it.packed_dev, x_dev, x_dtype, it.bias_dev,
                                 it.bias_dtype, it.y_dev, it.y_dtype, 0, MLXR_PATH_AUTO, stream);
      if (rc) return rc;
      if (M > 0 && (!it.packed_dev || !x_dev || !it.y_dev)) return fail(MLXR_E_INVALID, "null buffer (item %d)", i);
    } else {
      mlxr::PackedLayout L;
      int rc = check_type_shape(it.qtype, it.N, it.K, &L);
      if (rc) return rc;
    }
    mlxr::make_layout(it.qtype, it.N, it.K, &a[i].L);
    a[i].packed = (const uint8_t*)it.packed_dev;
    a[i].x = x_dev;
    a[i].x_dtype = x_dtype;
    a[i].bias = it.bias_dev;
    a[i].bias_dtype = it.bias_dtype;
    a[i].y = it.y_dev;
    a[i].y_dtype = it.y_dtype;
    a[i].M = M;
  }
  return MLXR_OK;
}

int run_grouped(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M, void* ws,
                size_t ws_bytes, void* stream) {
  std::vector<mlxr::RunArgs> a;
  int rc = grouped_args(count, items, x_dev, x_dtype, M, true, stream, a);
  if (rc || count == 0 || M == 0) return rc;
  hipStream_t s = (hipStream_t)stream;
  for (const Batch& bt : plan_batches(a, M, ws != nullptr)) {
    const mlxr::RunArgs* batch[4];
    for (int k = 0; k < bt.n; ++k) batch[k] = &a[(size_t)bt.idx[k]];
    if (bt.kind == 1) {
      const hipError_t e = mlxr::launch_gemv_grouped(batch, bt.n, s);
      if (e != hipSuccess) return hip_fail(e, "grouped gemv launch");
    } else if (bt.kind == 2) {
      const hipError_t e = mlxr::launch_mfma_grouped(batch, bt.n, ws, ws ? ws_bytes : 0, s);
      if (e != hipSuccess) return hip_fail(e, "grouped mfma launch");
    } else {
      const mlxr_qgemm_item& it = items[bt.idx[0]];
      rc = mlxr_qgemm_run_ws(it.qtype, it.N, it.K, it.group_size, it.packed_dev, x_dev, x_dtype, it.bias_dev,
                             it.bias_dtype, it.y_dev, it.y_dtype, M, MLXR_PATH_AUTO, ws, ws ? ws_bytes : 0, stream);
      if (rc) return rc;
    }
  }
  return MLXR_OK;
}

}  // namespace

extern "C" {

int mlxr_qgemm_run_grouped(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M,
                           void* stream) {
  return run_grouped(count, items, x_dev, x_dtype, M, nullptr, 0, stream);
}

int mlxr_qgemm_run_grouped_ws(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M,
                              void* workspace_dev, size_t workspace_bytes, void* stream) {
  return run_grouped(count, items, x_dev, x_dtype, M, workspace_dev, workspace_dev ? workspace_bytes : 0, stream);
}

int mlxr_qgemm_grouped_workspace_size(int count, const mlxr_qgemm_item* items, int M, size_t* bytes) {
  if (!bytes) return fail(MLXR_E_INVALID, "null output pointer");
  std::vector<mlxr::RunArgs> a;
  int rc = grouped_args(count, items, nullptr, MLXR_BF16, M, false, nullptr, a);
  if (rc) return rc;
  size_t need = 0;
  if (count > 0 && M > 0) {
    for (const Batch& bt : plan_batches(a, M, true)) {
      const mlxr::RunArgs* batch[4];
      for (int k = 0; k < bt.n; ++k) batch[k] = &a[(size_t)bt.idx[k]];
      size_t b = 0;
      if (bt.kind == 2) {
        b = mlxr::mfma_grouped_workspace_bytes(batch, bt.n);
      } else if (bt.kind == 0) {
        const mlxr_qgemm_item& it = items[bt.idx[0]];
        rc = mlxr_qgemm_workspace_size(it.qtype, it.N, it.K, M, &b);
        if (rc) return rc;
      }
      need = std::max(need, b);
    }
  }
  *bytes = need;
  return MLXR_OK;
}

}  // extern "C"

namespace {
// How mlxr_qgemm_swiglu runs a shape: 0 GEMV launch (M <= 4), 1 narrow skinny kernel
// (M <= 32), 2 tiled kernel, 3 unfused (operands of 2 GiB or more: two projections, then
// mlxr_swiglu with up in the workspace).  Kinds 1 and 2 fuse the gating into the
// projection launch; their workspace only holds split-K partials.
int swiglu_kind(const mlxr::RunArgs& a) {
  if (a.M <= kGemvMaxM && gemv_auto(a.M, a.L) && mlxr::gemv_groupable(a)) return 0;
  if (!mlxr::mfma_groupable(a)) return 3;
  return mlxr::skinny_swiglu_ok(a.M) ? 1 : 2;
}
}  // namespace

extern "C" {

int mlxr_qgemm_swiglu_workspace_size(int qtype, int N, int K, int M, int h_dtype, size_t* bytes) {
  mlxr::PackedLayout L;
  const int rc = check_type_shape(qtype, N, K, &L);
  if (rc) return rc;
  if (!bytes) return fail(MLXR_E_INVALID, "null output pointer");
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  if (!valid_dtype(h_dtype)) return fail(MLXR_E_INVALID, "invalid output dtype %d", h_dtype);
  mlxr::RunArgs a;
  a.L = L;
  a.M = M;
  switch (M == 0 ? 0 : swiglu_kind(a)) {
    case 1: *bytes = mlxr::skinny_swiglu_workspace_bytes(M, N, K); break;
    case 2: *bytes = mlxr::mfma_swiglu_workspace_bytes(M, N, K); break;
    case 3: *bytes = (size_t)M * (size_t)N * (h_dtype == MLXR_F32 ? 4 : 2); break;
    default: *bytes = 0;
  }
  return MLXR_OK;
}

int mlxr_qgemm_swiglu(int qtype, int N, int K, const void* gate_packed, const void* up_packed, const void* x_dev,
                      int x_dtype, void* h_dev, int h_dtype, int M, void* workspace_dev, size_t workspace_bytes,
                      void* stream) {
  size_t need = 0;
  int rc = mlxr_qgemm_swiglu_workspace_size(qtype, N, K, M, h_dtype, &need);
  if (rc) return rc;
  if (x_dtype != MLXR_BF16 && x_dtype != MLXR_F16)
    return fail(MLXR_E_INVALID, "activation dtype must be BF16 or F16 (got %d)", x_dtype);
  if (M == 0) return MLXR_OK;
  if (!gate_packed || !up_packed || !x_dev || !h_dev) return fail(MLXR_E_INVALID, "null buffer");
  mlxr::RunArgs g, u;
  mlxr::make_layout(qtype, N, K, &g.L);
  u.L = g.L;
  g.packed = (const uint8_t*)gate_packed;
  u.packed = (const uint8_t*)up_packed;
  g.x = u.x = x_dev;
  g.x_dtype = u.x_dtype = x_dtype;
  g.bias = u.bias = nullptr;
  g.bias_dtype = u.bias_dtype = MLXR_F32;
  g.y = h_dev;
  u.y = nullptr;
  g.y_dtype = u.y_dtype = h_dtype;
  g.M = u.M = M;
  const int kind = swiglu_kind(g);
  hipStream_t s = (hipStream_t)stream;
  if (kind == 0) {
    const hipError_t e = mlxr::launch_gemv_swiglu(g, u, s);
    return e != hipSuccess ? hip_fail(e, "swiglu gemv launch") : MLXR_OK;
  }
  if (kind == 1 || kind == 2) {
    // a workspace smaller than the split plan's runs the launch unsplit
    void* ws = workspace_dev && workspace_bytes >= need ? workspace_dev : nullptr;
    g.ws = ws;
    g.ws_bytes = ws ? workspace_bytes : 0;
    const hipError_t e =
        kind == 1 ? mlxr::launch_skinny_swiglu(g, u, s) : mlxr::launch_mfma_swiglu(g, u, ws, g.ws_bytes, s);
    return e != hipSuccess ? hip_fail(e, "swiglu launch") : MLXR_OK;
  }
  // operands of 2 GiB or more: gate into h, up into the workspace, then the gating in place
  if (!workspace_dev || workspace_bytes < need)
    return fail(MLXR_E_INVALID, "swiglu at M=%d needs a workspace of %zu bytes (got %zu)", M, need,
                workspace_bytes);
  rc = mlxr_qgemm_run_ex(qtype, N, K, 0, gate_packed, x_dev, x_dtype, nullptr, MLXR_F32, h_dev, h_dtype, M,
                         MLXR_PATH_AUTO, stream);
  if (rc) return rc;
  rc = mlxr_qgemm_run_ex(qtype, N, K, 0, up_packed, x_dev, x_dtype, nullptr, MLXR_F32, workspace_dev, h_dtype, M,
                         MLXR_PATH_AUTO, stream);
  if (rc) return rc;
  return mlxr_swiglu(h_dev, workspace_dev, h_dev, (size_t)M * (size_t)N, h_dtype, stream);
}

int mlxr_qgemm_run(int qtype, int N, int K, int group_size, const void* packed_dev, const void* x_dev,
                   int x_dtype, const void* bias_dev, int bias_dtype, void* y_dev, int y_dtype, int M,
                   void* stream) {
  return mlxr_qgemm_run_ex(qtype, N, K, group_size, packed_dev, x_dev, x_dtype, bias_dev, bias_dtype, y_dev,
                           y_dtype, M, MLXR_PATH_AUTO, stream);
}

}  // extern "C"

// ------------------------------------------------------------------ fused SwiGLU MLP

namespace {

constexpr size_t kMlpSyncBytes = (size_t)mlxr::kMlpSyncWords * 4;
static_assert(kMlpSyncBytes == MLXR_MLP_H_OFFSET, "h follows the sync region");

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Validates the MLP's shapes; fills the layouts.
int mlp_shapes(int qgu, int qd, int H, int I, int M, mlxr::MlpArgs* a) {
  int rc = check_type_shape(qgu, I, H, &a->gate);
  if (rc) return rc;
  rc = check_type_shape(qd, H, I, &a->down);
  if (rc) return rc;
  if (M < 0) return fail(MLXR_E_INVALID, "Input shape must be [M, K] (M=%d)", M);
  a->up = a->gate;
  a->qtd = qd;
  a->M = M;
  a->H = H;
  a->I = I;
  return MLXR_OK;
}

// Workspace past the sync words and h: split-K partials of the unfused launches.
int mlp_rest_bytes(int qgu, int qd, int H, int I, int M, size_t* bytes) {
  size_t a = 0, b = 0;
  int rc = mlxr_qgemm_swiglu_workspace_size(qgu, I, H, M, MLXR_BF16, &a);
  if (rc) return rc;
  rc = mlxr_qgemm_workspace_size(qd, H, I, M, &b);
  if (rc) return rc;
  *bytes = std::max(a, b);
  return MLXR_OK;
}

}  // namespace

extern "C" {

int mlxr_qgemm_mlp_workspace_size(int qtype_gu, int qtype_down, int hidden, int inter, int M, size_t* bytes) {
  mlxr::MlpArgs a;
  int rc = mlp_shapes(qtype_gu, qtype_down, hidden, inter, M, &a);
  if (rc) return rc;
  if (!bytes) return fail(MLXR_E_INVALID, "null output pointer");
  size_t rest = 0;
  rc = mlp_rest_bytes(qtype_gu, qtype_down, hidden, inter, M, &rest);
  if (rc) return rc;
  *bytes = kMlpSyncBytes + align256((size_t)M * (size_t)inter * 2) + rest;
  return MLXR_OK;
}

int mlxr_qgemm_mlp_workspace_init(void* workspace_dev, size_t workspace_bytes, void* stream) {
  if (!workspace_dev || workspace_bytes < kMlpSyncBytes)
    return fail(MLXR_E_INVALID, "MLP workspace must be at least %zu bytes (got %zu)", kMlpSyncBytes,
                workspace_dev ? workspace_bytes : (size_t)0);
  const hipError_t e = mlxr::launch_mlp_sync_zero((unsigned*)workspace_dev, (hipStream_t)stream);
  return e != hipSuccess ? hip_fail(e, "mlp workspace init") : MLXR_OK;
}

int mlxr_qgemm_mlp(int qtype_gu, int qtype_down, int hidden, int inter, const void* gate_packed,
                   const void* up_packed, const void* down_packed, const void* x_dev, int x_dtype, void* y_dev,
                   int y_dtype, int M, void* workspace_dev, size_t workspace_bytes, void* stream) {
  return mlxr_qgemm_mlp_ex(qtype_gu, qtype_down, hidden, inter, gate_packed, up_packed, down_packed, x_dev, x_dtype,
                           y_dev, y_dtype, M, MLXR_MLP_AUTO, workspace_dev, workspace_bytes, stream);
}

int mlxr_qgemm_mlp_ex(int qtype_gu, int qtype_down, int hidden, int inter, const void* gate_packed,
                      const void* up_packed, const void* down_packed, const void* x_dev, int x_dtype, void* y_dev,
                      int y_dtype, int M, int mode, void* workspace_dev, size_t workspace_bytes, void* stream) {
  if (mode != MLXR_MLP_AUTO && mode != MLXR_MLP_CHAIN && mode != MLXR_MLP_ONE_LAUNCH)
    return fail(MLXR_E_INVALID, "invalid MLP mode %d", mode);
  mlxr::MlpArgs a;
  int rc = mlp_shapes(qtype_gu, qtype_down, hidden, inter, M, &a);
  if (rc) return rc;
  if (x_dtype != MLXR_BF16 && x_dtype != MLXR_F16)
    return fail(MLXR_E_INVALID, "activation dtype must be BF16 or F16 (got %d)", x_dtype);
  if (!valid_dtype(y_dtype)) return fail(MLXR_E_INVALID, "invalid output dtype %d", y_dtype);
  if (M == 0) return MLXR_OK;
  if (!gate_packed || !up_packed || !down_packed || !x_dev || !y_dev)
    return fail(MLXR_E_INVALID, "null buffer");
  size_t need = 0;
  rc = mlxr_qgemm_mlp_workspace_size(qtype_gu, qtype_down, hidden, inter, M, &need);
  if (rc) return rc;
  if (!workspace_dev || workspace_bytes < need)
    return fail(MLXR_E_INVALID, "the MLP at M=%d needs a workspace of %zu bytes (got %zu)", M, need,
                workspace_dev ? workspace_bytes : (size_t)0);
  uint8_t* ws = (uint8_t*)workspace_dev;
  a.gate_packed = gate_packed;
  a.up_packed = up_packed;
  a.down_packed = down_packed;
  a.x = x_dev;
  a.x_dtype = x_dtype;
  a.sync = (unsigned*)ws;
  a.h = ws + kMlpSyncBytes;
  a.y = y_dev;
  a.y_dtype = y_dtype;
  hipStream_t s = (hipStream_t)stream;
  // the one-launch kernel only when asked for: on MI355X it is slower than the two launches
  // (Llama-3-8B at M = 1: 28 us against 22 us)
  if (mode == MLXR_MLP_ONE_LAUNCH && mlxr::mlp_fused_ok(a)) {
    const hipError_t e = mlxr::launch_mlp_fused(a, s);
    return e != hipSuccess ? hip_fail(e, "mlp launch") : MLXR_OK;
  }
  // two launches: gate/up with the gating, then down over h
  const size_t hb = align256((size_t)M * (size_t)inter * 2);
  void* rest = ws + kMlpSyncBytes + hb;
  const size_t rest_bytes = workspace_bytes - kMlpSyncBytes - hb;
  rc = mlxr_qgemm_swiglu(qtype_gu, inter, hidden, gate_packed, up_packed, x_dev, x_dtype, a.h, x_dtype, M, rest,
                         rest_bytes, stream);
  if (rc) return rc;
  return mlxr_qgemm_run_ws(qtype_down, hidden, inter, 0, down_packed, a.h, x_dtype, nullptr, MLXR_F32, y_dev,
                           y_dtype, M, MLXR_PATH_AUTO, rest, rest_bytes, stream);
}

int mlxr_qgemm_mlp_status(void* workspace_dev, void* stream) {
  if (!workspace_dev) return fail(MLXR_E_INVALID, "null workspace");
  unsigned flag = 0;
  unsigned* f = (unsigned*)workspace_dev + mlxr::kMlpSlotWords * mlxr::kMlpErr;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(&flag, f, sizeof(flag), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  // after a timeout the counters may be left mid-count: the whole sync region is zeroed
  if (e == hipSuccess && flag) e = mlxr::launch_mlp_sync_zero((unsigned*)workspace_dev, s);
  if (e == hipSuccess && flag) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "mlp status");
  if (flag)
    return fail(MLXR_E_TIMEOUT,
                "a fused MLP launch on this workspace gave up waiting for its gate/up workgroups; its output is "
                "invalid");
  return MLXR_OK;
}

int mlxr_qgemm_test_set_mlp_spin_limit(unsigned ticks) {
  mlxr::set_mlp_spin_limit(ticks ? ticks : 20000000u);
  return MLXR_OK;
}

int mlxr_qgemm_test_skinny_stage(int on) {
  mlxr::g_skinny_stage.store(on <= 0 ? 0 : on >= 2 ? 2 : 1, std::memory_order_relaxed);
  return MLXR_OK;
}

int mlxr_qgemm_test_force_skinny(int on) {
  g_force_skinny.store(on ? 1 : 0, std::memory_order_relaxed);
  return MLXR_OK;
}

int mlxr_qgemm_test_set_operand_limit(size_t bytes) {
  const size_t full = (size_t)1 << 31;
  mlxr::g_operand_limit.store(bytes ? std::min(bytes, full) : full, std::memory_order_relaxed);
  return MLXR_OK;
}

}  // extern "C"
