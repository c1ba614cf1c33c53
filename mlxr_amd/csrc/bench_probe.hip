// Measurement kernels for the benchmark, built into their own library (libmlxr_bench.so),
// not into the matmul library: nothing on the matmul path calls them.
//  - stream_read_kernel: a pure streaming read of up to four device buffers in one launch,
//    the bytes a grouped GEMV launch reads, with nothing computed on them.  bench.py runs
//    it over the headline step's packed weights in the step's launch structure (one launch
//    per grouped projection, one graph) to give the HBM ceiling that structure allows.
//  - mfma_peak_kernel: back-to-back independent bf16 MFMAs (32x32x16, sixteen
//    accumulators per wavefront, one wavefront per SIMD), nothing loaded: the matrix-core
//    rate the chip sustains under full load, clock throttling included, as the ceiling of
//    the prefill GEMMs.
#include <hip/hip_runtime.h>
#include <stdint.h>


// Exported (bench.py binds them with ctypes; return 0, -1 for invalid arguments, -4 for a
// HIP launch error):
//   int mlxr_bench_stream_read(int nbuf, const void* const* bufs, const size_t* bytes,
//                              void* sink_dev, int grid, void* stream);
//     one launch of `grid` workgroups that only reads bytes[i] (multiples of 16) of each
//     of the nbuf (1-4) buffers with non-temporal loads; sink_dev: 4 KiB it could write.
//   int mlxr_bench_mfma_peak(int grid, int iters, void* out_dev, void* stream);
//     grid workgroups of four wavefronts, each iters x 16 independent bf16 32x32x16 MFMAs
//     (flops = grid * 4 * iters * 16 * 32768); writes grid * 256 floats to out_dev.

namespace mlxr {
namespace {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

struct ReadParams {
  const uint8_t* p[4];
  size_t n16[4];   // 16-byte units of each buffer
  size_t start[4];  // first unit of buffer i in the launch's concatenated range
  size_t total;
  int nbuf;
  uint32_t* sink;
};

// Threads take 16-byte units of the concatenated range in a grid-stride loop, four loads
// in flight each; the XOR of the data goes to sink only if it equals a value no input
// here produces, so the loads cannot be dropped and nothing is written.
__global__ __launch_bounds__(256) void stream_read_kernel(ReadParams rp) {
  const size_t stride = (size_t)gridDim.x * 256;
  uint32_t acc = 0;
  for (size_t base = (size_t)blockIdx.x * 256 + threadIdx.x; base < rp.total; base += 4 * stride) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t i = base + u * stride;
      v[u] = u32x4_t{0, 0, 0, 0};
      if (i < rp.total) {
        int b = 0;
#pragma unroll
        for (int k = 1; k < 4; ++k)
          if (k < rp.nbuf && i >= rp.start[k]) b = k;
        const u32x4_t* q = (const u32x4_t*)rp.p[b] + (i - rp.start[b]);
        v[u] = __builtin_nontemporal_load(q);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9E3779B9u && threadIdx.x == 0) rp.sink[blockIdx.x & 1023] = acc;
}

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Each wavefront: iters x 16 MFMAs on sixteen independent accumulators; operands from
// registers (small values, so nothing overflows); the sums go to out (one float per
// thread) so nothing is dropped.
__global__ __launch_bounds__(256, 1) void mfma_peak_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  const uint32_t va = 0x3c003c00u ^ (uint32_t)(lane * 0x00010001u), vb = va ^ 0x00400040u;
  const u32x4_t a = {va, va ^ 0x10001u, va ^ 0x20002u, va ^ 0x30003u};
  const u32x4_t b = {vb, vb ^ 0x10001u, vb ^ 0x20002u, vb ^ 0x30003u};
  f32x16_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[i][v];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// Does nothing: a graph of these measures what a launch costs before any work.
__global__ __launch_bounds__(256) void empty_kernel(uint32_t* sink) {
  if (sink && blockIdx.x == 0x7fffffffu) sink[0] = 1u;  // never true: keeps the argument live
}

}  // namespace
}  // namespace mlxr

// One launch of an empty kernel of `grid` workgroups of 256 threads.
extern "C" int mlxr_bench_empty(int grid, void* sink_dev, void* stream) {
  if (grid < 1) return -1;
  mlxr::empty_kernel<<<dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream>>>((uint32_t*)sink_dev);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -4;
}

extern "C" int mlxr_bench_mfma_peak(int grid, int iters, void* out_dev, void* stream) {
  if (grid < 1 || iters < 1 || !out_dev) return -1;
  mlxr::mfma_peak_kernel<<<dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream>>>((float*)out_dev, iters);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -4;
}

extern "C" int mlxr_bench_stream_read(int nbuf, const void* const* bufs, const size_t* bytes, void* sink_dev,
                                      int grid, void* stream) {
  if (nbuf < 1 || nbuf > 4 || !bufs || !bytes || !sink_dev || grid < 1) return -1;
  mlxr::ReadParams rp;
  rp.total = 0;
  rp.nbuf = nbuf;
  rp.sink = (uint32_t*)sink_dev;
  for (int i = 0; i < 4; ++i) {
    const int k = i < nbuf ? i : 0;
    if (!bufs[k] || (bytes[k] & 15)) return -1;
    rp.p[i] = (const uint8_t*)bufs[k];
    rp.n16[i] = i < nbuf ? bytes[k] / 16 : 0;
    rp.start[i] = rp.total;
    rp.total += rp.n16[i];
  }
  mlxr::stream_read_kernel<<<dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream>>>(rp);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -4;
}
