/*
 * mlxr_qgemm.h -- C ABI of the MI355X (gfx950) quantized-matmul library
 * (libmlxr_qgemm.so).
 *
 * It replaces the device side of MLXR's q_gemm_dequant operator:
 *   reference  core/kernels/primitives/q_gemm_dequant_primitive.h:211-215
 *              (mlxr::kernels::q_gemm_dequant, Y[M,N] = X[M,K] . W[N,K]^T + bias)
 *              core/kernels/primitives/q_gemm_dequant_primitive.mm:367-450 (eval_gpu)
 *              core/kernels/metal/q_gemm_dequant.metal:292-312,338-486 (QGemmArgs + kernel)
 * and the weight upload the reference leaves unimplemented
 *   reference  daemon/server/model_loader.cpp:236-245 (quantized tensors skipped)
 *              core/runtime/mmap_loader.h:51-61 (WeightTensor host bytes)
 *
 * Conventions
 *   - Every pointer named *_dev is device memory on the current HIP device; *_host is
 *     host memory.  `stream` is a hipStream_t passed as void* (NULL = default stream).
 *   - All work is stream-ordered and asynchronous; no entry point synchronises the
 *     device except mlxr_qgemm_pack (host source; it waits for its own copy).
 *   - Return value 0 = success, negative = error (MLXR_E_*); the message of the last
 *     error on the calling thread is returned by mlxr_qgemm_last_error().  No C++
 *     exception crosses this boundary.
 *   - Thread-safe: the library's only mutable global state is the thread-local error
 *     string and the two test hooks' atomics.
 *   - Dequantized weights follow the GGUF block_q4_0 / block_q4_1 / block_q8_0 /
 *     block_q4_K / block_q5_K / block_q6_K definitions exactly (fp32 results are bit-exact to those
 *     formulas).
 */
#ifndef MLXR_QGEMM_H
#define MLXR_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantization types: same numeric values as mlxr::kernels::QuantType
 * (reference q_gemm_dequant_primitive.h:18-35).  Implemented: Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K.
 * Q4_0/Q4_1 follow GGUF block_q4_0/block_q4_1 (byte j holds elements j and j+16); the
 * reference's CPU routines (.mm:189-216) read them interleaved (elements 2j, 2j+1). */
enum {
  MLXR_Q4_0 = 0, MLXR_Q4_1 = 1, MLXR_Q8_0 = 2, MLXR_Q4_K = 3, MLXR_Q6_K = 4,
  MLXR_Q5_0 = 5, MLXR_Q5_1 = 6, MLXR_Q8_1 = 7, MLXR_Q2_K = 8, MLXR_Q3_K = 9,
  MLXR_Q5_K = 10, MLXR_Q8_K = 11, MLXR_IQ2_XXS = 12, MLXR_IQ2_XS = 13,
  MLXR_IQ3_XXS = 14, MLXR_IQ3_S = 15
};

/* Element types of activations, bias and outputs. */
enum { MLXR_F32 = 0, MLXR_F16 = 1, MLXR_BF16 = 2 };

/* Status codes. */
enum {
  MLXR_OK = 0,
  MLXR_E_INVALID = -1,     /* null pointer, bad dtype, non-positive size */
  MLXR_E_UNSUPPORTED = -2, /* quant type not implemented (reference: .mm:76,133,340) */
  MLXR_E_SHAPE = -3,       /* K not a multiple of the block size, group_size mismatch */
  MLXR_E_HIP = -4,         /* HIP runtime error (message has the HIP error string) */
  MLXR_E_NOMEM = -5,       /* device allocation failed (mlxr_qgemm_pack only) */
  MLXR_E_TIMEOUT = -6      /* a fused MLP launch gave up its bounded wait (mlxr_qgemm_mlp_status) */
};

/* Execution path selector for mlxr_qgemm_run_ex. */
enum {
  MLXR_PATH_AUTO = 0, /* GEMV (no MFMA) for M = 1 and, depending on the shape
                         (mlxr_qgemm_auto_path), M <= 4; MFMA kernels above: skinny
                         (weights streamed once) for M <= 64, tiled GEMM beyond.  When
                         mlxr_qgemm_run_ws is given the workspace it asks for, calls with
                         32 < M <= 256 take whichever of the two is estimated faster for
                         the shape (the skinny one for narrow weights) */
  MLXR_PATH_GEMV = 1, /* force the wavefront-reduction GEMV kernel (any M <= 64) */
  MLXR_PATH_MFMA = 2  /* force the MFMA kernels (chosen as for MLXR_PATH_AUTO) */
};

/* Library version (major*10000 + minor*100 + patch). */
int mlxr_qgemm_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mlxr_qgemm_last_error(void);

/* Bytes of the raw GGUF tensor: N * ceil(K/group) * sizeof(block).
 * Replaces compute_quantized_weight_size (reference .mm:116-135) and
 * calculate_tensor_size (daemon/registry/gguf_parser.cpp:179-241, Q6_K = 210 B). */
int mlxr_qgemm_gguf_size(int qtype, int N, int K, size_t* bytes);

/* Elements per quantization group: Q4_0/Q4_1/Q8_0 -> 32, Q4_K/Q5_K/Q6_K -> 256
 * (reference get_default_group_size, .mm:80-92; it has no Q5_K). */
int mlxr_qgemm_group_size(int qtype);

/* Name of a quant type ("Q4_K", ...; "Unknown" otherwise) (reference .mm:94-114). */
const char* mlxr_qgemm_type_name(int qtype);

/* Bytes of the packed device buffer for an [N, K] weight of type qtype. */
int mlxr_qgemm_packed_size(int qtype, int N, int K, size_t* bytes);

/* One-time upload: repack GGUF blocks (host memory, N rows of K/group blocks, as stored
 * in the file) into packed_dev (mlxr_qgemm_packed_size bytes).  Allocates a temporary
 * device staging buffer, copies, repacks on the device, frees the staging buffer, and
 * synchronises `stream` before returning. */
int mlxr_qgemm_pack(int qtype, int N, int K, const void* gguf_host, void* packed_dev,
                    void* stream);

/* Same, from GGUF bytes already on the device.  Asynchronous, allocates nothing. */
int mlxr_qgemm_pack_device(int qtype, int N, int K, const void* gguf_dev, void* packed_dev,
                           void* stream);

/* Dequantize a packed weight into out_dev [N, K] (row-major), out_dtype MLXR_F32
 * (bit-exact GGUF formulas) or MLXR_BF16 (round-to-nearest-even of those fp32 values,
 * produced by the same routine the MFMA GEMM uses to fill its LDS tiles). */
int mlxr_qgemm_dequant(int qtype, int N, int K, const void* packed_dev, void* out_dev,
                       int out_dtype, void* stream);

/* Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]), fp32 accumulation.
 *   x_dev    [M, K] row-major, x_dtype MLXR_BF16 or MLXR_F16
 *   bias_dev [N] or NULL, bias_dtype MLXR_F32 / MLXR_F16 / MLXR_BF16 (ignored if NULL)
 *   y_dev    [M, N] row-major, y_dtype MLXR_F32 / MLXR_F16 / MLXR_BF16
 *   group_size must be 0 (use the type's default) or equal to mlxr_qgemm_group_size.
 * Arguments mirror q_gemm_dequant(input, weights, M, N, K, quant_type, group_size, bias)
 * (reference q_gemm_dequant_primitive.h:211-215) with the weights already packed. */
int mlxr_qgemm_run(int qtype, int N, int K, int group_size, const void* packed_dev,
                   const void* x_dev, int x_dtype, const void* bias_dev, int bias_dtype,
                   void* y_dev, int y_dtype, int M, void* stream);

/* mlxr_qgemm_run with an explicit path (MLXR_PATH_*). */
int mlxr_qgemm_run_ex(int qtype, int N, int K, int group_size, const void* packed_dev,
                      const void* x_dev, int x_dtype, const void* bias_dev, int bias_dtype,
                      void* y_dev, int y_dtype, int M, int path, void* stream);

/* Device workspace bytes mlxr_qgemm_run_ws can use for an [M, N, K] problem; 0 when the
 * problem would not use one.  MFMA GEMMs whose workgroups would be too few to fill the
 * device (tiled ones, M > 32, and skinny ones with few 32-row slabs) split K over several
 * workgroups and add the fp32 partials in a second kernel; the workspace holds those
 * partials (splits x M x N x 4 bytes).  For 32 < M <= 256 the size is that of the kernel
 * the call would choose with it; mlxr_qgemm_run_ws ignores a smaller workspace (the call
 * then runs as mlxr_qgemm_run_ex: skinny kernel for M <= 64, tiled one above, unsplit).
 * When the size is 0 the call makes the same choice with or without a workspace.
 * No counterpart in the reference (its kernel has no K split, q_gemm_dequant.metal:374-464). */
int mlxr_qgemm_workspace_size(int qtype, int N, int K, int M, size_t* bytes);

/* The kernel family MLXR_PATH_AUTO runs an [M, N, K] call on: MLXR_PATH_GEMV or
 * MLXR_PATH_MFMA in *path.  M = 1 is always the GEMV; 2 <= M <= 4 the GEMV unless the rows
 * are long (K >= 8192 at M >= 3, K >= 16384 at M = 2) or, at M = 4, the weight is large (N*K
 * >= 48 Mi elements, not Q6_K), where the skinny MFMA kernel is faster; M > 4 the MFMA
 * kernels.  No counterpart in the reference (its operator has one kernel). */
int mlxr_qgemm_auto_path(int qtype, int N, int K, int M, int* path);

/* mlxr_qgemm_run_ex with a caller-owned device workspace (workspace_bytes bytes; NULL or
 * too small = the kernel and result of mlxr_qgemm_run_ex).  The workspace must not be
 * in use by other work while this call's kernels run on `stream`.  The two choices differ
 * only in fp32 summation order; a given (shape, workspace size) always
 * takes the same choice, so repeated calls are bit-identical. */
int mlxr_qgemm_run_ws(int qtype, int N, int K, int group_size, const void* packed_dev,
                      const void* x_dev, int x_dtype, const void* bias_dev, int bias_dtype,
                      void* y_dev, int y_dtype, int M, int path, void* workspace_dev,
                      size_t workspace_bytes, void* stream);

/* Bytes of the split-K scratch array mlxr_qgemm_run_noalloc keeps on each GPU. */
#define MLXR_NOALLOC_SCRATCH_BYTES (32u << 20)

/* mlxr_qgemm_run_ws without a workspace argument and without any allocation: split-K
 * partials go to a fixed device array of MLXR_NOALLOC_SCRATCH_BYTES per GPU that the
 * library holds until the process ends.  Same arguments, kernels and results as
 * mlxr_qgemm_run_ws with a workspace of that size.  Calls whose plan needs more scratch
 * (mlxr_qgemm_workspace_size above MLXR_NOALLOC_SCRATCH_BYTES) fail with MLXR_E_INVALID.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU (concurrent
 * streams or threads) race on it; serialize them.  The array keeps the last call's
 * partials (every element a call reads it has written first).
 * No counterpart in the reference: it exists for callers that cannot allocate device
 * memory (HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int mlxr_qgemm_run_noalloc(int qtype, int N, int K, int group_size, const void* packed_dev,
                           const void* x_dev, int x_dtype, const void* bias_dev, int bias_dtype,
                           void* y_dev, int y_dtype, int M, int path, void* stream);

/* One weight of a grouped call (see mlxr_qgemm_run_grouped). */
typedef struct mlxr_qgemm_item {
  int qtype, N, K, group_size; /* as in mlxr_qgemm_run */
  const void* packed_dev;      /* packed weight [N, K] */
  const void* bias_dev;        /* [N] or NULL */
  int bias_dtype;
  void* y_dev;                 /* [M, N] */
  int y_dtype;
} mlxr_qgemm_item;

/* y_i[M, N_i] = X[M, K] . W_i[N_i, K]^T (+ bias_i) for `count` weights that read the same
 * activations -- the projections of one input, e.g. q/k/v or gate/up of a decoder layer.
 * Every item must have the same K.  Items of one quant type run up to four per launch
 * where the kernel allows it: the GEMV at M <= 4 (X staged once) and the tiled MFMA GEMM
 * at M > 64 (tile columns of the weights side by side); other items run as
 * mlxr_qgemm_run(..., MLXR_PATH_AUTO).  Results equal count separate mlxr_qgemm_run calls
 * bit for bit, with one exception at M <= 4: an item whose single call the automatic path
 * gives the skinny MFMA kernel (mlxr_qgemm_auto_path) stays in the GEMV launch unless its
 * weight is very large (N*K >= 128 Mi elements), and then equals its single call with
 * MLXR_PATH_GEMV.  No counterpart in the reference (its Linear layers call q_gemm_dequant one
 * projection at a time, core/graph/layers.cpp:86-99); it exists to cut kernel launches
 * and, for prefill, to fill the device with the small projections' tiles. */
int mlxr_qgemm_run_grouped(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M,
                           void* stream);
/* mlxr_qgemm_run_grouped with a caller-owned device workspace (NULL or too small = as
 * mlxr_qgemm_run_grouped).  With it the tiled launches also serve 32 < M <= 64 and split K
 * over the concatenated N of their weights when their tiles cannot fill the device, and
 * single items run as mlxr_qgemm_run_ws.  Results then differ from separate calls only in
 * fp32 summation order (within the matmul tolerance) and are deterministic for a given
 * (items, M, workspace size).  Same workspace rules as mlxr_qgemm_run_ws. */
int mlxr_qgemm_run_grouped_ws(int count, const mlxr_qgemm_item* items, const void* x_dev, int x_dtype, int M,
                              void* workspace_dev, size_t workspace_bytes, void* stream);
/* Workspace bytes mlxr_qgemm_run_grouped_ws can use for these items at this M (only the
 * items' qtype, N and K are read). */
int mlxr_qgemm_grouped_workspace_size(int count, const mlxr_qgemm_item* items, int M, size_t* bytes);

/* h[M, N] = swish(X . Wg^T) * (X . Wu^T): the gate/up half of a SwiGLU MLP
 * (reference core/graph/layers.cpp:391-414; swiglu_mlp_fused.metal:131-345 plans the
 * fusion).  gate_packed and up_packed are packed weights of the same type and [N, K].
 * At M <= 4 one launch computes both projections and the gating (no gate/up outputs ever
 * reach memory) and needs no workspace; above, it runs the two projections and
 * mlxr_swiglu, and the up projection goes to the caller's workspace of
 * mlxr_qgemm_swiglu_workspace_size bytes.  No counterpart in the reference's operator. */
int mlxr_qgemm_swiglu_workspace_size(int qtype, int N, int K, int M, int h_dtype, size_t* bytes);
int mlxr_qgemm_swiglu(int qtype, int N, int K, const void* gate_packed, const void* up_packed,
                      const void* x_dev, int x_dtype, void* h_dev, int h_dtype, int M,
                      void* workspace_dev, size_t workspace_bytes, void* stream);

/* out[i] = swish(gate[i]) * up[i], swish(g) = g / (1 + exp(-g)), computed in fp32 and
 * rounded to dtype (MLXR_F32 / MLXR_F16 / MLXR_BF16); out may alias gate or up.  The
 * gating of the SwiGLU MLP between its gate/up and down projections (reference
 * core/graph/layers.cpp:391-414, MLP::forward). */
int mlxr_swiglu(const void* gate_dev, const void* up_dev, void* out_dev, size_t n, int dtype, void* stream);

/* SwiGLU MLP, y[M, hidden] = down( swish(x . gate^T) * (x . up^T) ), the whole MLP block
 * of a decoder layer (reference core/graph/layers.cpp:391-414, MLP::forward;
 * core/kernels/metal/swiglu_mlp_fused.metal:110-131 computes the same chain in one
 * kernel).  gate and up are packed [inter, hidden] weights of qtype_gu, down a packed
 * [hidden, inter] weight of qtype_down; x is [M, hidden] (BF16/F16), y [M, hidden].
 * The gated intermediate h is kept in the activation type in the workspace.
 *   MLXR_MLP_CHAIN (and MLXR_MLP_AUTO): mlxr_qgemm_swiglu into the workspace (one launch
 *     for gate, up and the gating at every M), then the down projection.
 *   MLXR_MLP_ONE_LAUNCH (M = 1, qtype_down == qtype_gu or MLXR_Q6_K; other calls run the
 *     chain): one launch whose gate/up workgroups write h segment by segment and whose
 *     down workgroups consume each segment once a device-scope counter says it is
 *     complete (bounded waits).  Results equal the chain bit for bit.  Measured on
 *     MI355X it is slower than the chain (Llama-3-8B: 28 us against 22 us), so AUTO does
 *     not take it.
 * The workspace (mlxr_qgemm_mlp_workspace_size bytes) starts with a 160 KiB sync region
 * whose words must be zero before its first use: call mlxr_qgemm_mlp_workspace_init once
 * after allocating it (a kernel, so it may also be captured).  Each launch leaves them
 * zero again.  Calls that share a workspace must not overlap (same stream, or ordered
 * streams).
 * mlxr_qgemm_mlp_status synchronises `stream` and returns MLXR_E_TIMEOUT if a one-launch
 * call on this workspace gave up its wait since the last status call (its y is invalid;
 * only possible when the down workgroups wait 0.2 s, e.g. on a device shared with a
 * kernel that never yields); it then re-initialises the sync region, so the next launch is
 * exact.  No counterpart in the reference's operator. */
enum { MLXR_MLP_AUTO = 0, MLXR_MLP_CHAIN = 1, MLXR_MLP_ONE_LAUNCH = 2 };
#define MLXR_MLP_H_OFFSET 163840 /* byte offset of h ([M, inter], activation type) in the workspace */
int mlxr_qgemm_mlp_workspace_size(int qtype_gu, int qtype_down, int hidden, int inter, int M, size_t* bytes);
int mlxr_qgemm_mlp_workspace_init(void* workspace_dev, size_t workspace_bytes, void* stream);
int mlxr_qgemm_mlp(int qtype_gu, int qtype_down, int hidden, int inter, const void* gate_packed,
                   const void* up_packed, const void* down_packed, const void* x_dev, int x_dtype, void* y_dev,
                   int y_dtype, int M, void* workspace_dev, size_t workspace_bytes, void* stream);
int mlxr_qgemm_mlp_ex(int qtype_gu, int qtype_down, int hidden, int inter, const void* gate_packed,
                      const void* up_packed, const void* down_packed, const void* x_dev, int x_dtype, void* y_dev,
                      int y_dtype, int M, int mode, void* workspace_dev, size_t workspace_bytes, void* stream);
int mlxr_qgemm_mlp_status(void* workspace_dev, void* stream);

/* Test hooks (no counterpart in the reference; not for production callers).
 * mlxr_qgemm_test_set_operand_limit: the largest operand the 32-bit-offset kernels take in
 * one launch (default 2 GiB; 0 restores it), lowered by tests so small shapes reach the
 * chunked and fallback launches.  mlxr_qgemm_test_set_mlp_spin_limit: the fused MLP's wait
 * bound in ticks of the 100 MHz real-time counter (default 0.2 s; 0 restores it), lowered
 * by tests to exercise the timeout path.  mlxr_qgemm_test_force_skinny(1): every call of the
 * MFMA family (M > 4, or MLXR_PATH_MFMA) runs the skinny kernel, at any M, until called
 * with 0; tests use it to reach the skinny kernel's 64-row M blocks at shapes the automatic
 * choice gives to the tiled kernel.  mlxr_qgemm_test_skinny_stage(0): the narrow skinny
 * kernel reads its activations from global memory at every step instead of staging them in
 * LDS once (its mode at M <= 16 when the stages fit; 1 restores it; 2 prefers the mode where
 * two slabs share their stages wherever it fits); tests use it to check every mode against
 * the oracle.  All are process-wide (atomics). */
int mlxr_qgemm_test_set_operand_limit(size_t bytes);
int mlxr_qgemm_test_set_mlp_spin_limit(unsigned ticks);
int mlxr_qgemm_test_force_skinny(int on);
int mlxr_qgemm_test_skinny_stage(int on);

/* Deterministic synthetic inputs with the shapes/distributions of the benchmark
 * configurations (host memory).  Generator: SplitMix64 from `seed`; normals by
 * Box-Muller in double precision.
 *   Q8_0: d = RNE_fp16(|N(0,1)| * 0.02/127), qs uniform in [-127, 127]
 *   Q4_K: d, dmin = RNE_fp16(|N(0,1)| * 1e-3), 12 scale bytes and 128 qs bytes uniform
 *   Q6_K: ql, qh bytes uniform, scales uniform in [-32, 31], d = RNE_fp16(|N(0,1)|*1e-3)
 *   Q4_0: d = RNE_fp16(|N(0,1)| * 2e-3), 16 qs bytes uniform
 *   Q4_1: d = RNE_fp16(|N(0,1)| * 2e-3), m = RNE_fp16(N(0,1) * 8e-3), 16 qs bytes uniform
 *   Q5_K: as Q4_K, plus 32 uniform qh bytes
 * out_host must hold mlxr_qgemm_gguf_size bytes. */
int mlxr_synth_gguf(int qtype, int N, int K, uint64_t seed, void* out_host);

/* count values of N(0,1) rounded (RNE) to dtype MLXR_BF16 / MLXR_F16 / MLXR_F32. */
int mlxr_synth_act(size_t count, int dtype, uint64_t seed, void* out_host);

#ifdef __cplusplus
}
#endif

#endif /* MLXR_QGEMM_H */
