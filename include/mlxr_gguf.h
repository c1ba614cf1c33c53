/*
 * mlxr_gguf.h -- C ABI of the GGUF reader in libmlxr_qgemm.so: locate the quantized
 * weights of a .gguf file in a read-only memory map and upload them into the packed
 * device layout of mlxr_qgemm.h.
 *
 * It replaces, for the quantized-matmul path:
 *   reference  daemon/registry/gguf_parser.h:16-69, 122-219 (GGUFFile, header, metadata,
 *              tensor infos, GGUFTensorType ids)
 *              daemon/registry/gguf_parser.cpp:103-132 (gguf_block_size),
 *              179-241 (calculate_tensor_size), 278-316 (parse / data offset),
 *              448-491 (read_tensor_infos)
 *              core/runtime/mmap_loader.h:51-61, mmap_loader.cpp:102-199 (WeightTensor,
 *              map_tensor / map_region: zero-copy view of the tensor bytes)
 *              daemon/server/model_loader.cpp:65-110 (tensor registration) and 236-245
 *              (quantized tensors, which the reference skips; here they are uploaded)
 * Differences from the reference, on purpose:
 *   - block sizes follow the GGUF/ggml definitions: Q6_K 210 B (reference: 208),
 *     Q2_K 84 B (80), Q3_K 110 B (108);
 *   - the data section starts at the header end rounded up to general.alignment
 *     (default 32; the reference always uses 32);
 *   - the reader is bounds-checked: a truncated or malformed header is an error instead
 *     of a read past the end.  Tensor data ranges are checked when a tensor's bytes are
 *     requested (a header may describe tensors whose data is not in the file, as the
 *     reference's own parser test does).
 * Conventions as in mlxr_qgemm.h: 0 = success, negative MLXR_E_* codes, message in
 * mlxr_qgemm_last_error(); no exception crosses the boundary.  A handle may be read from
 * several threads at once; mlxr_gguf_close must not race with other calls on it.
 */
#ifndef MLXR_GGUF_H
#define MLXR_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (reference gguf_parser.h:40-69). */
enum {
  MLXR_GGML_F32 = 0, MLXR_GGML_F16 = 1, MLXR_GGML_Q4_0 = 2, MLXR_GGML_Q4_1 = 3,
  MLXR_GGML_Q5_0 = 6, MLXR_GGML_Q5_1 = 7, MLXR_GGML_Q8_0 = 8, MLXR_GGML_Q8_1 = 9,
  MLXR_GGML_Q2_K = 10, MLXR_GGML_Q3_K = 11, MLXR_GGML_Q4_K = 12, MLXR_GGML_Q5_K = 13,
  MLXR_GGML_Q6_K = 14, MLXR_GGML_Q8_K = 15, MLXR_GGML_I8 = 24, MLXR_GGML_I16 = 25,
  MLXR_GGML_I32 = 26, MLXR_GGML_I64 = 27, MLXR_GGML_F64 = 28, MLXR_GGML_BF16 = 30
};

/* Metadata value types (reference gguf_parser.h:23-37). */
enum {
  MLXR_GGUF_UINT8 = 0, MLXR_GGUF_INT8 = 1, MLXR_GGUF_UINT16 = 2, MLXR_GGUF_INT16 = 3,
  MLXR_GGUF_UINT32 = 4, MLXR_GGUF_INT32 = 5, MLXR_GGUF_FLOAT32 = 6, MLXR_GGUF_BOOL = 7,
  MLXR_GGUF_STRING = 8, MLXR_GGUF_ARRAY = 9, MLXR_GGUF_UINT64 = 10, MLXR_GGUF_INT64 = 11,
  MLXR_GGUF_FLOAT64 = 12
};

typedef struct mlxr_gguf mlxr_gguf; /* opaque handle: parsed header + read-only map */

typedef struct mlxr_gguf_header {
  uint32_t magic, version;
  uint64_t tensor_count, metadata_kv_count;
  uint64_t alignment;   /* general.alignment, or 32 */
  uint64_t data_offset; /* file offset of the data section */
  uint64_t file_size;
} mlxr_gguf_header;

typedef struct mlxr_gguf_tensor_info {
  const char* name;      /* NUL-terminated, owned by the handle */
  uint32_t n_dims;       /* 1..4 */
  uint64_t dims[4];      /* ggml order: dims[0] is the innermost (K of a weight) */
  uint32_t type;         /* MLXR_GGML_* */
  uint64_t offset;       /* from the data section start */
  uint64_t file_offset;  /* data_offset + offset */
  uint64_t size;         /* bytes (GGUF block sizes) */
  const void* data;      /* host pointer into the map, NULL if the range is not in the file */
} mlxr_gguf_tensor_info;

/* A metadata value.  Scalars in the union; strings as pointer + length into the map (not
 * NUL-terminated); arrays as element type + count, with `data` pointing at the packed
 * elements for arrays of fixed-size scalars (NULL for arrays of strings or arrays). */
typedef struct mlxr_gguf_value {
  uint32_t type; /* MLXR_GGUF_* */
  union {
    uint64_t u64;
    int64_t i64;
    double f64;
  } v;           /* integers widened (signed types sign-extended), floats as double,
                    bool as 0/1 */
  const char* str;
  uint64_t len;  /* string bytes, or array element count */
  uint32_t elem_type;
  const void* data;
} mlxr_gguf_value;

/* Parse a .gguf file (versions 1-3; v1 counts are 32-bit) and map it read-only. */
int mlxr_gguf_open(const char* path, mlxr_gguf** out);
/* Parse from memory the caller keeps alive for the life of the handle (nothing mapped). */
int mlxr_gguf_open_memory(const void* bytes, size_t size, mlxr_gguf** out);
void mlxr_gguf_close(mlxr_gguf* g);

int mlxr_gguf_get_header(const mlxr_gguf* g, mlxr_gguf_header* out);
/* Tensor i (0 <= i < tensor_count), in file order. */
int mlxr_gguf_get_tensor(const mlxr_gguf* g, uint64_t i, mlxr_gguf_tensor_info* out);
/* Index of the tensor called `name`, or -1 (reference find_tensor, gguf_parser.cpp). */
int64_t mlxr_gguf_find_tensor(const mlxr_gguf* g, const char* name);
/* Metadata key i in file order. */
int mlxr_gguf_get_key(const mlxr_gguf* g, uint64_t i, const char** key, mlxr_gguf_value* out);
/* Metadata by key: MLXR_OK, or MLXR_E_INVALID if absent. */
int mlxr_gguf_get_value(const mlxr_gguf* g, const char* key, mlxr_gguf_value* out);
/* Element j of an array value of strings: pointer + length. */
int mlxr_gguf_get_array_string(const mlxr_gguf* g, const char* key, uint64_t j, const char** s, uint64_t* len);

/* Bytes of n elements of a ggml type (GGUF block sizes; n must be a multiple of the
 * block), or MLXR_E_UNSUPPORTED for unknown types (reference calculate_tensor_size). */
int mlxr_gguf_type_bytes(uint32_t ggml_type, uint64_t n, uint64_t* bytes);
/* Elements per block: 32 for Q4_0..Q8_1, 256 for K-quants, 1 otherwise (gguf_block_size). */
int mlxr_gguf_block_size(uint32_t ggml_type);
/* "Q4_K", "F16", ... or "UNKNOWN" (reference gguf_type_name). */
const char* mlxr_gguf_type_name(uint32_t ggml_type);
/* The MLXR_Q* quant type of a ggml type the matmul implements, or MLXR_E_UNSUPPORTED. */
int mlxr_gguf_quant_type(uint32_t ggml_type);

/* Upload tensor i (a 2-D weight [N = dims[1], K = dims[0]] of a type the matmul
 * implements) into packed_dev (mlxr_qgemm_packed_size bytes), as mlxr_qgemm_pack does:
 * stages through a temporary device buffer and synchronises `stream`. */
int mlxr_gguf_upload(const mlxr_gguf* g, uint64_t i, void* packed_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLXR_GGUF_H */
