// C++ operator-interface checks that need no GPU, in the style of the reference's
// GoogleTest units (tests/unit/gguf_parser_test.cpp:139-176 check block sizes and type
// names).  Built and run by tests/test_abi.py; prints "OK <n>" on success.
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>

#include "q_gemm_dequant_primitive.h"

using namespace mlxr::kernels;

static int checks = 0;
#define EXPECT(c)                                                     \
  do {                                                                \
    ++checks;                                                         \
    if (!(c)) {                                                       \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c);         \
      return 1;                                                       \
    }                                                                 \
  } while (0)

template <typename F>
static std::string throws(F f) {
  try {
    f();
  } catch (const std::runtime_error& e) {
    return e.what();
  }
  return "";
}

int main() {
  EXPECT(compute_quantized_weight_size(4096, 4096, QuantType::Q4_K) == 9437184u);
  EXPECT(compute_quantized_weight_size(1024, 8192, QuantType::Q6_K) == 6881280u);
  EXPECT(compute_quantized_weight_size(2048, 2048, QuantType::Q8_0) == 4456448u);
  EXPECT(compute_quantized_weight_size(1, 32, QuantType::Q4_0) == 18u);
  EXPECT(std::strcmp(quant_type_name(QuantType::Q4_K), "Q4_K") == 0);
  EXPECT(std::strcmp(quant_type_name(QuantType::IQ3_S), "IQ3_S") == 0);
  EXPECT(QGemmDequantPrimitive::get_default_group_size(QuantType::Q8_0) == 32);
  EXPECT(QGemmDequantPrimitive::get_default_group_size(QuantType::Q4_K) == 256);
  EXPECT(QGemmDequantPrimitive::get_default_group_size(QuantType::Q6_K) == 256);
  EXPECT(QGemmDequantPrimitive::get_bytes_per_weight(QuantType::Q4_K) == 144 / 256.0f);
  EXPECT(QGemmDequantPrimitive::get_bytes_per_weight(QuantType::Q6_K) == 210 / 256.0f);
  EXPECT(throws([] { QGemmDequantPrimitive::get_bytes_per_weight(QuantType::Q2_K); }) ==
         "Unsupported quantization type");
  EXPECT(throws([] { compute_quantized_weight_size(8, 256, QuantType::Q3_K); }) == "Unsupported quantization type");
  EXPECT(compute_quantized_weight_size(4096, 4096, QuantType::Q5_K) == 11534336u);

  QGemmDequantPrimitive a(Stream{}, 1, 4096, 4096, QuantType::Q4_K, 256, false);
  QGemmDequantPrimitive b(Stream{}, 1, 4096, 4096, QuantType::Q4_K, 256, false);
  QGemmDequantPrimitive c(Stream{}, 1, 4096, 4096, QuantType::Q4_K, 256, true);
  EXPECT(std::strcmp(a.name(), "q_gemm_dequant") == 0);
  EXPECT(a.is_equivalent(b) && !a.is_equivalent(c));
  EXPECT(a.output_shapes({})[0] == (std::vector<int>{1, 4096}));

  // shape validation happens before any device work (reference .mm:490-496)
  array x = array::borrow(nullptr, {2, 4096}, Dtype::bfloat16);
  array w = array::borrow(nullptr, {16}, Dtype::uint8);
  array bias = array::borrow(nullptr, {100}, Dtype::bfloat16);
  EXPECT(throws([&] { q_gemm_dequant(x, w, 1, 4096, 4096, QuantType::Q4_K, 256); }) == "Input shape must be [M, K]");
  EXPECT(throws([&] { q_gemm_dequant(x, w, 2, 4096, 4096, QuantType::Q4_K, 256, &bias); }) == "Bias shape must be [N]");
  std::vector<array> in = {x, w}, out;
  EXPECT(!throws([&] { a.eval_cpu(in, out); }).empty());
  std::vector<array> few = {x};
  EXPECT(throws([&] { a.eval_gpu(few, out); }) == "QGemmDequant requires input, weights, and optional bias");
  std::printf("OK %d\n", checks);
  return 0;
}
