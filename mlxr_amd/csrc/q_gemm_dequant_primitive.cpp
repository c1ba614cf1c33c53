// C++ operator layer over the C ABI (see include/q_gemm_dequant_primitive.h).
// Behaviour follows core/kernels/primitives/q_gemm_dequant_primitive.mm:
//   get_bytes_per_weight :63-78, get_default_group_size :80-92, quant_type_name :94-114,
//   compute_quantized_weight_size :116-135, is_equivalent :285-297,
//   q_gemm_dequant :478-522 (shape checks and messages :490-496).
#include "../../include/q_gemm_dequant_primitive.h"

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/mlxr_qgemm.h"

namespace mlxr {
namespace kernels {

namespace {

void check(int rc) {
  if (rc != MLXR_OK) throw std::runtime_error(mlxr_qgemm_last_error());
}

size_t elems(const std::vector<int>& shape) {
  size_t n = 1;
  for (int d : shape) n *= (size_t)(d < 0 ? 0 : d);
  return n;
}

}  // namespace

size_t dtype_size(Dtype d) {
  switch (d) {
    case Dtype::float32: return 4;
    case Dtype::float16: case Dtype::bfloat16: return 2;
    default: return 1;
  }
}

array::array(std::vector<int> shape, Dtype dtype) : shape_(std::move(shape)), dtype_(dtype) {
  nbytes_ = elems(shape_) * dtype_size(dtype_);
  void* p = nullptr;
  if (nbytes_) {
    const hipError_t e = hipMalloc(&p, nbytes_);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipMalloc failed: ") + hipGetErrorString(e));
  }
  ptr_ = std::shared_ptr<void>(p, [](void* q) {
    if (q) (void)hipFree(q);
  });
}

array::array(std::vector<int> shape, Dtype dtype, Stream s) : shape_(std::move(shape)), dtype_(dtype) {
  nbytes_ = elems(shape_) * dtype_size(dtype_);
  void* p = nullptr;
  hipStream_t hs = (hipStream_t)s.hip_stream;
  if (nbytes_) {
    const hipError_t e = hipMallocAsync(&p, nbytes_, hs);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipMallocAsync failed: ") + hipGetErrorString(e));
  }
  ptr_ = std::shared_ptr<void>(p, [hs](void* q) {
    if (q) (void)hipFreeAsync(q, hs);
  });
}

array array::borrow(void* dev_ptr, std::vector<int> shape, Dtype dtype) {
  array a;
  a.shape_ = std::move(shape);
  a.dtype_ = dtype;
  a.nbytes_ = elems(a.shape_) * dtype_size(dtype);
  a.ptr_ = std::shared_ptr<void>(dev_ptr, [](void*) {});
  return a;
}

size_t array::size() const { return elems(shape_); }

float QGemmDequantPrimitive::get_bytes_per_weight(QuantType type) {
  switch (type) {
    case QuantType::Q4_0: return 18 / 32.0f;
    case QuantType::Q4_1: return 20 / 32.0f;
    case QuantType::Q8_0: return 34 / 32.0f;
    case QuantType::Q4_K: return 144 / 256.0f;
    case QuantType::Q5_K: return 176 / 256.0f;
    case QuantType::Q6_K: return 210 / 256.0f;
    default: throw std::runtime_error("Unsupported quantization type");
  }
}

int QGemmDequantPrimitive::get_default_group_size(QuantType type) {
  return mlxr_qgemm_group_size((int)type);
}

const char* quant_type_name(QuantType type) { return mlxr_qgemm_type_name((int)type); }

size_t compute_quantized_weight_size(int N, int K, QuantType quant_type) {
  switch (quant_type) {
    case QuantType::Q4_0: case QuantType::Q4_1: case QuantType::Q8_0:
    case QuantType::Q4_K: case QuantType::Q5_K: case QuantType::Q6_K: break;
    default: throw std::runtime_error("Unsupported quantization type");
  }
  size_t bytes = 0;
  check(mlxr_qgemm_gguf_size((int)quant_type, N, K, &bytes));
  return bytes;
}

QGemmDequantPrimitive::QGemmDequantPrimitive(Stream stream, int M, int N, int K, QuantType quant_type,
                                             int group_size, bool has_bias)
    : stream_(stream), M_(M), N_(N), K_(K), quant_type_(quant_type), group_size_(group_size),
      has_bias_(has_bias) {}

bool QGemmDequantPrimitive::is_equivalent(const QGemmDequantPrimitive& o) const {
  return M_ == o.M_ && N_ == o.N_ && K_ == o.K_ && quant_type_ == o.quant_type_ &&
         group_size_ == o.group_size_ && has_bias_ == o.has_bias_;
}

void QGemmDequantPrimitive::eval_cpu(const std::vector<array>&, std::vector<array>&) {
  throw std::runtime_error("QGemmDequant: no CPU evaluation in the MI355X library; use a GPU stream");
}

void QGemmDequantPrimitive::eval_gpu(const std::vector<array>& inputs, std::vector<array>& outputs) {
  if (inputs.size() < 2 || (has_bias_ && inputs.size() < 3))
    throw std::runtime_error("QGemmDequant requires input, weights, and optional bias");
  const array& input = inputs[0];
  const array& weights = inputs[1];
  const array* bias = has_bias_ ? &inputs[2] : nullptr;
  int xdt;
  if (input.dtype() == Dtype::bfloat16) xdt = MLXR_BF16;
  else if (input.dtype() == Dtype::float16) xdt = MLXR_F16;
  else throw std::runtime_error("QGemmDequant input must be bfloat16 or float16");

  array packed;
  if (weights.dtype() == Dtype::packed) {
    if ((int)weights.quant_type() != (int)quant_type_ || weights.packed_N() != N_ || weights.packed_K() != K_)
      throw std::runtime_error("packed weights do not match (quant_type, N, K)");
    packed = weights;
  } else {
    // Raw GGUF blocks on the device, as the reference passes them: pack for this call into
    // a stream-ordered temporary, released (hipFreeAsync) after the GEMM in stream order.
    if (weights.nbytes() < compute_quantized_weight_size(N_, K_, quant_type_))
      throw std::runtime_error("weights buffer is smaller than N * K/group * sizeof(block)");
    packed = pack_weights_device(weights, N_, K_, quant_type_, stream_, true);
  }
  if (outputs.empty()) outputs.emplace_back();
  if (outputs[0].nbytes() == 0) outputs[0] = array({M_, N_}, input.dtype(), stream_);
  array& out = outputs[0];
  if (out.dtype() != Dtype::float32 && out.dtype() != Dtype::float16 && out.dtype() != Dtype::bfloat16)
    throw std::runtime_error("QGemmDequant output must be float32, float16 or bfloat16");
  if (out.nbytes() < (size_t)M_ * (size_t)N_ * dtype_size(out.dtype()))
    throw std::runtime_error("QGemmDequant output buffer is smaller than [M, N]");
  const int ydt = out.dtype() == Dtype::float32 ? MLXR_F32 : out.dtype() == Dtype::float16 ? MLXR_F16 : MLXR_BF16;
  int bdt = MLXR_F32;
  if (bias) bdt = bias->dtype() == Dtype::float32 ? MLXR_F32 : bias->dtype() == Dtype::float16 ? MLXR_F16 : MLXR_BF16;
  check(mlxr_qgemm_run((int)quant_type_, N_, K_, group_size_, packed.data<void>(), input.data<void>(), xdt,
                       bias ? bias->data<void>() : nullptr, bdt, out.data<void>(), ydt, M_, stream_.hip_stream));
}

namespace {
// Packed buffers are one-dimensional uint8 arrays: their byte count must fit the shape.
int packed_bytes(int N, int K, QuantType quant_type) {
  size_t bytes = 0;
  check(mlxr_qgemm_packed_size((int)quant_type, N, K, &bytes));
  if (bytes > 0x7fffffffu) throw std::runtime_error("packed weight of 2 GiB or more: split it by rows");
  return (int)bytes;
}
}  // namespace

array pack_weights(const void* gguf_host, int N, int K, QuantType quant_type, Stream s) {
  array a({packed_bytes(N, K, quant_type)}, Dtype::uint8);
  check(mlxr_qgemm_pack((int)quant_type, N, K, gguf_host, a.data<void>(), s.hip_stream));
  a.dtype_ = Dtype::packed;
  a.qtype_ = quant_type;
  a.pN_ = N;
  a.pK_ = K;
  return a;
}

array pack_weights_device(const array& gguf_dev, int N, int K, QuantType quant_type, Stream s, bool stream_ordered) {
  const int bytes = packed_bytes(N, K, quant_type);
  array a = stream_ordered ? array({bytes}, Dtype::uint8, s) : array({bytes}, Dtype::uint8);
  check(mlxr_qgemm_pack_device((int)quant_type, N, K, gguf_dev.data<void>(), a.data<void>(), s.hip_stream));
  a.dtype_ = Dtype::packed;
  a.qtype_ = quant_type;
  a.pN_ = N;
  a.pK_ = K;
  return a;
}

array q_gemm_dequant(const array& input, const array& weights, int M, int N, int K, QuantType quant_type,
                     int group_size, const array* bias, Stream s) {
  if (input.shape().size() != 2 || input.shape(0) != M || input.shape(1) != K)
    throw std::runtime_error("Input shape must be [M, K]");
  if (bias != nullptr && (bias->shape().size() != 1 || bias->shape(0) != N))
    throw std::runtime_error("Bias shape must be [N]");
  QGemmDequantPrimitive prim(s, M, N, K, quant_type, group_size, bias != nullptr);
  std::vector<array> inputs = {input, weights};
  if (bias) inputs.push_back(*bias);
  std::vector<array> outputs = {array({M, N}, input.dtype(), s)};
  prim.eval_gpu(inputs, outputs);
  return outputs[0];
}

}  // namespace kernels
}  // namespace mlxr
