// Buffer loads and wait helpers shared by the MFMA kernels (qgemm_tile_kernel.h,
// qgemm_skinny.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qgemm_wdequant.h"

namespace mlxr {

typedef __attribute__((ext_vector_type(4))) int i32x4_t;

constexpr uint32_t OOB = 0x80000000u;  // voffset beyond every buffer: loads return 0

// Raw buffer resource in SGPRs (wave-uniform base and size).
__device__ __forceinline__ i32x4_t make_srsrc(const void* ptr, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)ptr;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// Weight loads are compiler-visible buffer loads (the compiler then never reads a
// register before its data has arrived, even where it copies loop-carried values);
// out-of-range offsets replace branches.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* ptr, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t bload16(rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// VMEM instructions of load_raw / load_hdr (one weight row).
template <int QT>
constexpr int raw_loads() { return QT == QT_Q4_K ? 1 : QT == QT_Q6_K ? 2 : QT == QT_Q8_0 ? 3 : 2; }  // Q5_K, Q4_0/1: 2
template <int QT>
constexpr int hdr_loads() { return (QT == QT_Q4_K || QT == QT_Q5_K) ? 1 : QT == QT_Q6_K ? 2 : 0; }  // K-quants only

template <int QT>
__device__ __forceinline__ void load_raw(const rsrc_t* R, uint32_t row_sub, int sb, bool ok, Raw<QT>& r) {
  // row_sub = row * nsub (sub-block index of the row start); sb = sub-block within the row
  const uint32_t s = row_sub + (uint32_t)sb;
  if constexpr (QT == QT_Q4_K) {
    r.q = bload16(R[0], ok ? s * 16u : OOB);
  } else if constexpr (QT == QT_Q6_K) {
    r.ql = bload16(R[0], ok ? s * 16u : OOB);
    r.qh = __builtin_amdgcn_raw_buffer_load_b64(R[1], ok ? s * 8u : OOB, 0, 0);
  } else if constexpr (QT == QT_Q5_K) {
    r.q = bload16(R[0], ok ? s * 16u : OOB);
    r.qh = __builtin_amdgcn_raw_buffer_load_b32(R[1], ok ? s * 4u : OOB, 0, 0);
  } else if constexpr (QT == QT_Q4_0) {
    r.q = bload16(R[0], ok ? s * 16u : OOB);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? s * 2u : OOB, 0, 0);
  } else if constexpr (QT == QT_Q4_1) {
    r.q = bload16(R[0], ok ? s * 16u : OOB);
    r.d = __builtin_amdgcn_raw_buffer_load_b32(R[1], ok ? s * 4u : OOB, 0, 0);
  } else {
    const uint32_t o = ok ? s * 32u : OOB;
    r.a = bload16(R[0], o);
    r.b = bload16(R[0], o, 16u);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(R[1], ok ? s * 2u : OOB, 0, 0);
  }
}

template <int QT>
__device__ __forceinline__ void load_hdr(const rsrc_t* R, uint32_t row_sb, int g, bool ok, Hdr<QT>& h) {
  // row_sb = row * nsb; g = super-block within the row
  const uint32_t s = row_sb + (uint32_t)g;
  if constexpr (QT == QT_Q4_K) {
    h.h = bload16(R[1], ok ? s * 16u : OOB);
  } else if constexpr (QT == QT_Q5_K) {
    h.h = bload16(R[2], ok ? s * 16u : OOB);
  } else if constexpr (QT == QT_Q6_K) {
    h.h = bload16(R[2], ok ? s * 16u : OOB);
    h.d = __builtin_amdgcn_raw_buffer_load_b16(R[3], ok ? s * 2u : OOB, 0, 0);
  }
}

// Wait until at most N vector memory instructions of this wavefront are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace mlxr
