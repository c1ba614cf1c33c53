// Linear and MLP layers (include/mlxr_linear.h) over the C ABI of mlxr_qgemm.h.
// Reference: core/graph/layers.cpp:66-99 (Linear), :383-414 (MLP).
#include "../../include/mlxr_linear.h"

#include <hip/hip_runtime.h>

#include <stdexcept>

#include "../../include/mlxr_qgemm.h"

namespace mlxr {
namespace graph {

namespace {

void check(int rc) {
  if (rc != MLXR_OK) throw std::runtime_error(mlxr_qgemm_last_error());
}

int dt_code(kernels::Dtype d) {
  switch (d) {
    case kernels::Dtype::float32: return MLXR_F32;
    case kernels::Dtype::float16: return MLXR_F16;
    case kernels::Dtype::bfloat16: return MLXR_BF16;
    default: throw std::runtime_error("activations and biases must be float32, float16 or bfloat16");
  }
}

}  // namespace

Linear::Linear(int in_features, int out_features, bool bias)
    : in_features_(in_features), out_features_(out_features), has_bias_(bias) {
  if (in_features <= 0 || out_features <= 0) throw std::runtime_error("Linear: features must be positive");
}

void Linear::load_weight(const void* gguf_host, kernels::QuantType qt, kernels::Stream s) {
  weight_ = kernels::pack_weights(gguf_host, out_features_, in_features_, qt, s);
}

void Linear::load_weight(const mlxr_gguf* file, const std::string& name, kernels::Stream s) {
  const int64_t i = mlxr_gguf_find_tensor(file, name.c_str());
  if (i < 0) throw std::runtime_error("GGUF tensor not found: " + name);
  mlxr_gguf_tensor_info t;
  check(mlxr_gguf_get_tensor(file, (uint64_t)i, &t));
  if (t.n_dims != 2 || t.dims[0] != (uint64_t)in_features_ || t.dims[1] != (uint64_t)out_features_)
    throw std::runtime_error("GGUF tensor " + name + " does not have dims {in_features, out_features}");
  const int qt = mlxr_gguf_quant_type(t.type);
  if (qt < 0) check(qt);
  if (!t.data) throw std::runtime_error("GGUF tensor " + name + ": data is outside the file");
  weight_ = kernels::pack_weights(t.data, out_features_, in_features_, (kernels::QuantType)qt, s);
}

void Linear::set_bias(const kernels::array& bias) {
  if (!has_bias_) throw std::runtime_error("Linear was built without bias");
  if (bias.ndim() != 1 || bias.shape(0) != out_features_) throw std::runtime_error("Bias shape must be [N]");
  dt_code(bias.dtype());
  bias_ = bias;
}

void Linear::run(const kernels::array& x, int M, kernels::array& y, kernels::Stream s) {
  if (weight_.dtype() != kernels::Dtype::packed) throw std::runtime_error("Linear: weight not loaded");
  if (has_bias_ && bias_.nbytes() == 0) throw std::runtime_error("Linear: bias not set");
  const int qt = (int)weight_.quant_type();
  size_t ws = 0;
  check(mlxr_qgemm_workspace_size(qt, out_features_, in_features_, M, &ws));
  if (ws > 0x7fffffffu) ws = 0;  // beyond one array: run unsplit
  if (ws > workspace_.nbytes()) {
    // the previous workspace may still be in use by queued work on this stream
    if (workspace_.nbytes()) {
      const hipError_t e = hipStreamSynchronize((hipStream_t)s.hip_stream);
      if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
    }
    workspace_ = kernels::array({(int)ws}, kernels::Dtype::uint8);
  }
  check(mlxr_qgemm_run_ws(qt, out_features_, in_features_, 0, weight_.data<void>(), x.data<void>(),
                          dt_code(x.dtype()), has_bias_ ? bias_.data<void>() : nullptr,
                          has_bias_ ? dt_code(bias_.dtype()) : MLXR_F32, y.data<void>(), dt_code(y.dtype()), M,
                          MLXR_PATH_AUTO, workspace_.nbytes() ? workspace_.data<void>() : nullptr,
                          workspace_.nbytes(), s.hip_stream));
}

kernels::array Linear::forward(const kernels::array& x, kernels::Stream s) {
  if (x.ndim() < 1 || x.shape(-1) != in_features_) throw std::runtime_error("Input shape must be [..., in_features]");
  if (x.dtype() != kernels::Dtype::bfloat16 && x.dtype() != kernels::Dtype::float16)
    throw std::runtime_error("Linear input must be bfloat16 or float16");
  long M = 1;
  for (int d = 0; d + 1 < x.ndim(); ++d) M *= x.shape(d);
  if (M > 0x7fffffffL) throw std::runtime_error("Linear: too many rows");
  std::vector<int> shape = x.shape();
  shape.back() = out_features_;
  kernels::array y(shape, x.dtype());
  if (M > 0) run(x, (int)M, y, s);
  return y;
}

MLP::MLP(int hidden_size, int intermediate_size)
    : hidden_(hidden_size),
      inter_(intermediate_size),
      gate_(hidden_size, intermediate_size, false),
      up_(hidden_size, intermediate_size, false),
      down_(intermediate_size, hidden_size, false) {}

kernels::array MLP::forward(const kernels::array& x, kernels::Stream s) {
  if (x.ndim() < 1 || x.shape(-1) != hidden_) throw std::runtime_error("Input shape must be [..., hidden_size]");
  if (x.dtype() != kernels::Dtype::bfloat16 && x.dtype() != kernels::Dtype::float16)
    throw std::runtime_error("MLP input must be bfloat16 or float16");
  if (gate_.weight_.dtype() != kernels::Dtype::packed || up_.weight_.dtype() != kernels::Dtype::packed)
    throw std::runtime_error("MLP: gate/up weights not loaded");
  long M = 1;
  for (int d = 0; d + 1 < x.ndim(); ++d) M *= x.shape(d);
  std::vector<int> hshape = x.shape();
  hshape.back() = inter_;
  kernels::array g(hshape, x.dtype());
  if (M > 0) {
    const int qt = (int)gate_.weight_.quant_type();
    if (qt != (int)up_.weight_.quant_type()) throw std::runtime_error("MLP: gate and up must share a quant type");
    const int dt = dt_code(x.dtype());
    size_t ws = 0;
    check(mlxr_qgemm_swiglu_workspace_size(qt, inter_, hidden_, (int)M, dt, &ws));
    kernels::array u;
    if (ws) u = kernels::array({(int)ws}, kernels::Dtype::uint8);
    // M <= 4: gate, up and the gating in one launch; above, up goes to u
    check(mlxr_qgemm_swiglu(qt, inter_, hidden_, gate_.weight_.data<void>(), up_.weight_.data<void>(),
                            x.data<void>(), dt, g.data<void>(), dt, (int)M, ws ? u.data<void>() : nullptr, ws,
                            s.hip_stream));
  }
  kernels::array y = down_.forward(g, s);
  // the temporaries are freed here (hipFree waits for the device), after the queued kernels
  return y;
}

}  // namespace graph
}  // namespace mlxr
