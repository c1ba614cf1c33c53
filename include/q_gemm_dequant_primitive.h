// C++ operator interface of the quantized matmul, mirroring the reference's
// core/kernels/primitives/q_gemm_dequant_primitive.h (namespace mlxr::kernels):
// same QuantType values (:18-35), same QGemmDequantPrimitive shape (:78-195), same
// q_gemm_dequant(...) signature (:211-215) and helpers (:225, :230).  MLX does not exist
// on ROCm, so `array` here is a minimal device tensor (HIP device pointer + shape + dtype,
// shared ownership) and `Stream` wraps a hipStream_t.  Everything runs through the C ABI
// of mlxr_qgemm.h; nonzero status codes become std::runtime_error, as the reference throws.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <utility>
#include <vector>

namespace mlxr {
namespace kernels {

enum class QuantType {
  Q4_0 = 0, Q4_1 = 1, Q8_0 = 2, Q4_K = 3, Q6_K = 4, Q5_0 = 5, Q5_1 = 6, Q8_1 = 7,
  Q2_K = 8, Q3_K = 9, Q5_K = 10, Q8_K = 11, IQ2_XXS = 12, IQ2_XS = 13, IQ3_XXS = 14, IQ3_S = 15,
};

enum class Dtype {
  float32 = 0,   // MLXR_F32
  float16 = 1,   // MLXR_F16
  bfloat16 = 2,  // MLXR_BF16
  uint8 = 3,     // raw bytes, e.g. GGUF blocks copied to the device
  packed = 4,    // a weight packed by pack_weights() (qtype/N/K carried by the array)
};

size_t dtype_size(Dtype d);

// Stand-in for mlx::core::StreamOrDevice: a HIP stream (nullptr = default stream).
struct Stream {
  void* hip_stream = nullptr;
};

// Minimal device array with shared ownership of a HIP allocation.
class array {
 public:
  array() = default;
  // Allocates nbytes(shape, dtype) of device memory (hipMalloc; freed with hipFree).
  array(std::vector<int> shape, Dtype dtype);
  // Stream-ordered allocation on s (hipMallocAsync; freed with hipFreeAsync on s when the
  // last owner lets go): no device synchronisation either way.  Use it on s only (other
  // streams must be ordered after s's work by the caller).
  array(std::vector<int> shape, Dtype dtype, Stream s);
  // Wraps memory the caller owns (not freed by the array).
  static array borrow(void* dev_ptr, std::vector<int> shape, Dtype dtype);

  const std::vector<int>& shape() const { return shape_; }
  int shape(int dim) const { return shape_.at(dim < 0 ? dim + (int)shape_.size() : dim); }
  int ndim() const { return (int)shape_.size(); }
  Dtype dtype() const { return dtype_; }
  size_t nbytes() const { return nbytes_; }
  size_t size() const;
  template <typename T>
  T* data() const { return static_cast<T*>(ptr_.get()); }

  // Set on packed weights.
  QuantType quant_type() const { return qtype_; }
  int packed_N() const { return pN_; }
  int packed_K() const { return pK_; }

 private:
  friend array pack_weights(const void*, int, int, QuantType, Stream);
  friend array pack_weights_device(const array&, int, int, QuantType, Stream, bool);
  std::shared_ptr<void> ptr_;
  std::vector<int> shape_;
  Dtype dtype_ = Dtype::uint8;
  size_t nbytes_ = 0;
  QuantType qtype_ = QuantType::Q4_0;
  int pN_ = 0, pK_ = 0;
};

class QGemmDequantPrimitive {
 public:
  QGemmDequantPrimitive(Stream stream, int M, int N, int K, QuantType quant_type, int group_size,
                        bool has_bias = false);
  ~QGemmDequantPrimitive() = default;

  // There is no CPU implementation in this library: throws std::runtime_error.
  void eval_cpu(const std::vector<array>& inputs, std::vector<array>& outputs);
  // inputs = {input [M,K] bf16/fp16, weights (packed, or raw GGUF uint8 on device), bias [N]?}
  // outputs = {out [M,N]} (allocated stream-ordered here if empty, dtype of the input; a
  // caller's output must hold M*N elements of its dtype).  Raw GGUF weights are packed
  // into a stream-ordered temporary for the call (no synchronisation); pass weights
  // packed once by pack_weights() to avoid that per-call pack.
  void eval_gpu(const std::vector<array>& inputs, std::vector<array>& outputs);

  std::vector<std::vector<int>> output_shapes(const std::vector<array>&) const { return {{M_, N_}}; }
  const char* name() const { return "q_gemm_dequant"; }
  bool is_equivalent(const QGemmDequantPrimitive& other) const;

  int M() const { return M_; }
  int N() const { return N_; }
  int K() const { return K_; }
  QuantType quant_type() const { return quant_type_; }
  int group_size() const { return group_size_; }
  bool has_bias() const { return has_bias_; }

  static float get_bytes_per_weight(QuantType type);
  static int get_default_group_size(QuantType type);

 private:
  Stream stream_;
  int M_, N_, K_;
  QuantType quant_type_;
  int group_size_;
  bool has_bias_;
};

// Y[M,N] = input[M,K] . W[N,K]^T (+ bias), fp32 accumulation, output in the input dtype.
array q_gemm_dequant(const array& input, const array& weights, int M, int N, int K, QuantType quant_type,
                     int group_size, const array* bias = nullptr, Stream s = {});

// One-time upload of GGUF blocks from host memory into the packed device layout.
array pack_weights(const void* gguf_host, int N, int K, QuantType quant_type, Stream s = {});
// Same, from GGUF bytes already on the device (Dtype::uint8 array); stream_ordered
// allocates the packed array on s (hipMallocAsync, see array).
array pack_weights_device(const array& gguf_dev, int N, int K, QuantType quant_type, Stream s = {},
                          bool stream_ordered = false);

size_t compute_quantized_weight_size(int N, int K, QuantType quant_type);
const char* quant_type_name(QuantType type);

}  // namespace kernels
}  // namespace mlxr
