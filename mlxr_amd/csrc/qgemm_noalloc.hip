// mlxr_qgemm_run_noalloc: mlxr_qgemm_run_ws without a caller workspace, for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The split-K partials live in a fixed device array of
// this library, one per GPU, held until the process ends.
//
// In host code the name `scratch` is a host-side stand-in, not a device address: every
// kernel argument and copy uses the per-device address hipGetSymbolAddress returns,
// looked up once per device (with that device current) on the first call there.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/mlxr_qgemm.h"
#include "qgemm_internal.h"

static __device__ __align__(256) uint8_t scratch[MLXR_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // per-device address of `scratch`

// Address of this device's scratch array (looked up on the first call on the device).
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mlxr::set_error(MLXR_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return mlxr::set_error(MLXR_E_INVALID, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return mlxr::set_error(MLXR_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MLXR_OK;
}

}  // namespace

extern "C" {

int mlxr_qgemm_run_noalloc(int qtype, int N, int K, int group_size, const void* packed_dev, const void* x_dev,
                           int x_dtype, const void* bias_dev, int bias_dtype, void* y_dev, int y_dtype, int M,
                           int path, void* stream) {
  // the workspace the call's plan would use; the array must hold it
  size_t need = 0;
  int rc = mlxr_qgemm_workspace_size(qtype, N, K, M < 0 ? 0 : M, &need);
  if (rc) return rc;
  if (need > (size_t)MLXR_NOALLOC_SCRATCH_BYTES)
    return mlxr::set_error(MLXR_E_INVALID,
                           "mlxr_qgemm_run_noalloc: M=%d N=%d K=%d needs %zu bytes of split-K scratch, more than "
                           "the %zu the library holds; use mlxr_qgemm_run_ws with a workspace",
                           M, N, K, need, (size_t)MLXR_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_ptr(&ws);
    if (rc) return rc;
  }
  return mlxr_qgemm_run_ws(qtype, N, K, group_size, packed_dev, x_dev, x_dtype, bias_dev, bias_dtype, y_dev, y_dtype,
                           M, path, ws, ws ? (size_t)MLXR_NOALLOC_SCRATCH_BYTES : 0, stream);
}

}  // extern "C"
