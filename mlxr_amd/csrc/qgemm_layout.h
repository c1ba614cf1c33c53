// Packed HBM layout of a quantized [N, K] weight, shared by host and device code.
//
// GGUF stores a weight as N rows of K/B blocks (B = 32 for Q4_0/Q4_1/Q8_0, 256 for the
// K-quants), each block an array-of-structs record (block_q4_0 = 18 B, block_q4_1 = 20 B,
// block_q8_0 = 34 B, block_q4_K = 144 B, block_q6_K = 210 B).  The packed form splits every record into planes so that a
// 64-lane wavefront reading one plane touches whole, contiguous 128-byte lines, and it
// reorders nibbles inside 32-bit words so the GEMV can turn two 4-bit weights into a
// bf16/fp16 pair with a single mask-and-or.  It holds exactly the GGUF bytes (no
// padding except that each plane starts on a 256-byte boundary).
//
// Sub-block: 32 consecutive weights of one row along K.  Row n has nsub = K/32 of them.
// "Pair-interleaved" 32-bit word: holds the 4-bit fields of 8 consecutive weights
// e = 0..7 with weight e at nibble position (e/2) + 4*(e%2); so
// (word >> 4s) & 0x000F000F puts weight 2s in bits 0..3 and weight 2s+1 in bits 16..19.
//
//   Q4_K  plane 0  qs   [N][nsub][16 B]  sub-block = 4 pair-interleaved words (q 0..15)
//         plane 1  hdr  [N][K/256][8 x u16] lane-sliced header: u16 j (one per sub-block)
//                                        = sc_j | m_j << 6 | nibble j of (d | dmin << 16) << 12,
//                                        so the lane that owns sub-block j loads 2 bytes and
//                                        rebuilds d, dmin with an OR across the 8 lanes
//   Q5_K  plane 0  qs   [N][nsub][16 B]  low 4 bits, as Q4_K
//         plane 1  qh   [N][nsub][4 B]   fifth bits: weight e = 8t + f of the sub-block at
//                                        bit 2t + ((f>>1)&1) + 8(((f>>2)&1) + 2(f&1)), so one
//                                        shift lines them up with a word's nibble bytes
//         plane 2  hdr  [N][K/256][16 B] lane-sliced header, as Q4_K
//   Q6_K  plane 0  ql   [N][nsub][16 B]  low 4 bits, 4 pair-interleaved words
//         plane 1  qh   [N][nsub][8 B]   high 2 bits; for word t (weights 8t..8t+7) of
//                                        the sub-block: u32 index t/2, weight 8t+2s at
//                                        bit 2s + 8(t&1), weight 8t+2s+1 at 16 + 2s + 8(t&1)
//         plane 2  sc   [N][K/256][16 B] int8 scales, GGUF order (scale of weight e is e/16)
//         plane 3  d    [N][K/256][2 B]  fp16 d
//   Q8_0  plane 0  qs   [N][K/32][32 B]  int8, natural order
//         plane 1  d    [N][K/32][2 B]   fp16 d
//   Q4_0  plane 0  qs   [N][K/32][16 B]  block = 4 pair-interleaved words (q 0..15), as a
//                                        Q4_K sub-block
//         plane 1  d    [N][K/32][2 B]   fp16 d
//   Q4_1  plane 0  qs   [N][K/32][16 B]  as Q4_0
//         plane 1  dm   [N][K/32][4 B]   fp16 d | fp16 m << 16
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __HIPCC__
#define MLXR_HD __host__ __device__
#else
#define MLXR_HD
#endif

namespace mlxr {

// Same numeric values as mlxr::kernels::QuantType (core/kernels/primitives/
// q_gemm_dequant_primitive.h:18-35 in the reference).
enum QType : int { QT_Q4_0 = 0, QT_Q4_1 = 1, QT_Q8_0 = 2, QT_Q4_K = 3, QT_Q6_K = 4, QT_Q5_K = 10 };

struct PackedLayout {
  int qtype, N, K;
  int nplanes;
  size_t off[4];   // byte offset of each plane from the packed base
  size_t size[4];  // bytes in each plane
  size_t total;    // bytes of the whole packed buffer
};

MLXR_HD inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// K-quants carry a per-super-block header (scales of eight sub-blocks); the 32-weight
// block types carry their scale with every block.
MLXR_HD constexpr bool is_kquant(int qtype) { return qtype == QT_Q4_K || qtype == QT_Q5_K || qtype == QT_Q6_K; }

// Fills L; returns false if the type is not one the kernels implement or K does not
// split into whole blocks.
MLXR_HD inline bool make_layout(int qtype, int N, int K, PackedLayout* L) {
  L->qtype = qtype; L->N = N; L->K = K; L->nplanes = 0; L->total = 0;
  for (int i = 0; i < 4; ++i) { L->off[i] = 0; L->size[i] = 0; }
  if (N <= 0 || K <= 0) return false;
  const size_t n = (size_t)N;
  if (qtype == QT_Q4_K) {
    if (K % 256) return false;
    const size_t nsb = (size_t)(K / 256);
    L->nplanes = 2; L->size[0] = n * nsb * 128; L->size[1] = n * nsb * 16;
  } else if (qtype == QT_Q5_K) {
    if (K % 256) return false;
    const size_t nsb = (size_t)(K / 256);
    L->nplanes = 3; L->size[0] = n * nsb * 128; L->size[1] = n * nsb * 32; L->size[2] = n * nsb * 16;
  } else if (qtype == QT_Q6_K) {
    if (K % 256) return false;
    const size_t nsb = (size_t)(K / 256);
    L->nplanes = 4; L->size[0] = n * nsb * 128; L->size[1] = n * nsb * 64;
    L->size[2] = n * nsb * 16; L->size[3] = n * nsb * 2;
  } else if (qtype == QT_Q8_0) {
    if (K % 32) return false;
    const size_t nb = (size_t)(K / 32);
    L->nplanes = 2; L->size[0] = n * nb * 32; L->size[1] = n * nb * 2;
  } else if (qtype == QT_Q4_0 || qtype == QT_Q4_1) {
    if (K % 32) return false;
    const size_t nb = (size_t)(K / 32);
    L->nplanes = 2; L->size[0] = n * nb * 16; L->size[1] = n * nb * (qtype == QT_Q4_1 ? 4 : 2);
  } else {
    return false;
  }
  size_t o = 0;
  for (int i = 0; i < L->nplanes; ++i) { L->off[i] = o; o = align256(o + L->size[i]); }
  L->total = o;
  return true;
}

// GGUF block geometry (elements, bytes) -- daemon/registry/gguf_parser.cpp:103-132 and
// :179-241 in the reference, with the correct Q6_K record size of 210 bytes.
MLXR_HD inline int gguf_block_elems(int qtype) {
  switch (qtype) {
    case QT_Q4_0: case QT_Q4_1: case QT_Q8_0: return 32;
    case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: return 256;
    default: return 0;
  }
}
MLXR_HD inline int gguf_block_bytes(int qtype) {
  switch (qtype) {
    case QT_Q4_0: return 18;
    case QT_Q4_1: return 20;
    case QT_Q8_0: return 34;
    case QT_Q4_K: return 144;
    case QT_Q6_K: return 210;
    case QT_Q5_K: return 176;
    default: return 0;
  }
}

}  // namespace mlxr
