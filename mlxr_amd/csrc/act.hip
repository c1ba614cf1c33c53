// SwiGLU gating of the MLP (reference core/graph/layers.cpp:391-414, MLP::forward:
// swish(gate) * up with swish(x) = x * sigmoid(x)), as one elementwise kernel between the
// gate/up projections and the down projection.
#include <hip/hip_runtime.h>

#include "../../include/mlxr_qgemm.h"
#include "qgemm_device.h"
#include "qgemm_internal.h"

namespace mlxr {

namespace {

// swiglu1 (qgemm_device.h): silu(g) * u in fp32, silu(g) = g / (1 + exp(-g)) (exp
// saturates to inf for g < -88, giving -0 or 0 as the limit requires).

template <int DT>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ gate, const void* __restrict__ up,
                                                     void* __restrict__ out, size_t n) {
  // four elements per thread: 8-byte (16-bit types) or 16-byte (fp32) accesses
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    float g[4], u[4];
    if constexpr (DT == DT_F32) {
      const float4 a = *(const float4*)((const float*)gate + i), b = *(const float4*)((const float*)up + i);
      g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
      u[0] = b.x; u[1] = b.y; u[2] = b.z; u[3] = b.w;
      *(float4*)((float*)out + i) = make_float4(swiglu1(g[0], u[0]), swiglu1(g[1], u[1]), swiglu1(g[2], u[2]),
                                                swiglu1(g[3], u[3]));
    } else {
      const uint2 a = *(const uint2*)((const uint16_t*)gate + i), b = *(const uint2*)((const uint16_t*)up + i);
      const uint32_t aw[2] = {a.x, a.y}, bw[2] = {b.x, b.y};
      uint32_t o[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float r[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t gb = (aw[k] >> (16 * h)) & 0xffffu, ub = (bw[k] >> (16 * h)) & 0xffffu;
          const float gv = DT == DT_BF16 ? bf16_bits_to_f32(gb) : f16_bits_to_f32(gb);
          const float uv = DT == DT_BF16 ? bf16_bits_to_f32(ub) : f16_bits_to_f32(ub);
          r[h] = swiglu1(gv, uv);
        }
        o[k] = DT == DT_BF16 ? pack_bf16x2(r[0], r[1]) : (f32_to_f16_bits(r[0]) | (f32_to_f16_bits(r[1]) << 16));
      }
      *(uint2*)((uint16_t*)out + i) = make_uint2(o[0], o[1]);
    }
    return;
  }
  for (size_t j = i; j < n; ++j) store_scalar(out, DT, j, swiglu1(load_scalar(gate, DT, j), load_scalar(up, DT, j)));
}

}  // namespace

}  // namespace mlxr

extern "C" int mlxr_swiglu(const void* gate_dev, const void* up_dev, void* out_dev, size_t n, int dtype,
                           void* stream) {
  if (n == 0) return MLXR_OK;
  if (!gate_dev || !up_dev || !out_dev) return mlxr::set_error(MLXR_E_INVALID, "null buffer");
  if (dtype != MLXR_F32 && dtype != MLXR_F16 && dtype != MLXR_BF16)
    return mlxr::set_error(MLXR_E_INVALID, "invalid dtype %d", dtype);
  const size_t threads = (n + 3) / 4;
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == MLXR_F32) mlxr::swiglu_kernel<mlxr::DT_F32><<<grid, block, 0, s>>>(gate_dev, up_dev, out_dev, n);
  else if (dtype == MLXR_F16) mlxr::swiglu_kernel<mlxr::DT_F16><<<grid, block, 0, s>>>(gate_dev, up_dev, out_dev, n);
  else mlxr::swiglu_kernel<mlxr::DT_BF16><<<grid, block, 0, s>>>(gate_dev, up_dev, out_dev, n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mlxr::set_error(MLXR_E_HIP, "swiglu launch: %s", hipGetErrorString(e));
  return MLXR_OK;
}
