// Linear and MLP layers (include/mlxr_linear.h) over the C ABI of mlxr_qgemm.h.
// Reference: core/graph/layers.cpp:66-99 (Linear), :383-414 (MLP).
#include "../../include/mlxr_linear.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>
#include <string>

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

// Grows a layer-held stream-ordered workspace to `need` bytes for a use on s (returns
// whether it was reallocated).  The old buffer is freed (hipFreeAsync) on the stream that
// allocated it; when its last use was on another stream, that stream's work is made to
// precede the free first, so the memory is not handed out again while a kernel of that
// last use may still write into it.
bool grow_workspace(kernels::array& ws, void*& alloc_stream, void*& last_stream, size_t need, kernels::Stream s) {
  bool fresh = false;
  if (need > ws.nbytes()) {
    if (ws.nbytes() && last_stream != alloc_stream) {
      hipEvent_t ev;
      hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e == hipSuccess) {
        e = hipEventRecord(ev, (hipStream_t)last_stream);
        if (e == hipSuccess) e = hipStreamWaitEvent((hipStream_t)alloc_stream, ev, 0);
        (void)hipEventDestroy(ev);
      }
      if (e != hipSuccess) throw std::runtime_error(std::string("layer workspace release: ") + hipGetErrorString(e));
    }
    ws = kernels::array({(int)need}, kernels::Dtype::uint8, s);
    alloc_stream = s.hip_stream;
    fresh = true;
  }
  last_stream = s.hip_stream;
  return fresh;
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

size_t Linear::workspace_size(int M) const {
  if (weight_.dtype() != kernels::Dtype::packed) throw std::runtime_error("Linear: weight not loaded");
  size_t ws = 0;
  check(mlxr_qgemm_workspace_size((int)weight_.quant_type(), out_features_, in_features_, M, &ws));
  return ws;
}

void Linear::run(const kernels::array& x, int M, kernels::array& y, void* ws, size_t ws_bytes, kernels::Stream s) {
  if (weight_.dtype() != kernels::Dtype::packed) throw std::runtime_error("Linear: weight not loaded");
  if (has_bias_ && bias_.nbytes() == 0) throw std::runtime_error("Linear: bias not set");
  if (y.nbytes() < (size_t)M * (size_t)out_features_ * kernels::dtype_size(y.dtype()))
    throw std::runtime_error("Linear: output buffer is smaller than [M, out_features]");
  const int qt = (int)weight_.quant_type();
  check(mlxr_qgemm_run_ws(qt, out_features_, in_features_, 0, weight_.data<void>(), x.data<void>(),
                          dt_code(x.dtype()), has_bias_ ? bias_.data<void>() : nullptr,
                          has_bias_ ? dt_code(bias_.dtype()) : MLXR_F32, y.data<void>(), dt_code(y.dtype()), M,
                          MLXR_PATH_AUTO, ws_bytes ? ws : nullptr, ws ? ws_bytes : 0, s.hip_stream));
}

namespace {
long rows_of(const kernels::array& x, int features, const char* what) {
  if (x.ndim() < 1 || x.shape(-1) != features) throw std::runtime_error(std::string("Input shape must be [..., ") + what + "]");
  if (x.dtype() != kernels::Dtype::bfloat16 && x.dtype() != kernels::Dtype::float16)
    throw std::runtime_error("layer input must be bfloat16 or float16");
  long M = 1;
  for (int d = 0; d + 1 < x.ndim(); ++d) M *= x.shape(d);
  if (M > 0x7fffffffL) throw std::runtime_error("layer input: too many rows");
  return M;
}
}  // namespace

void Linear::forward(const kernels::array& x, kernels::array& y, void* workspace, size_t workspace_bytes,
                     kernels::Stream s) {
  const long M = rows_of(x, in_features_, "in_features");
  if (M > 0) run(x, (int)M, y, workspace, workspace_bytes, s);
}

kernels::array Linear::forward(const kernels::array& x, kernels::Stream s) {
  const long M = rows_of(x, in_features_, "in_features");
  std::vector<int> shape = x.shape();
  shape.back() = out_features_;
  kernels::array y(shape, x.dtype(), s);
  if (M > 0) {
    size_t ws = workspace_size((int)M);
    if (ws > 0x7fffffffu) ws = 0;  // beyond one array: run unsplit
    grow_workspace(workspace_, ws_alloc_stream_, ws_last_stream_, ws, s);
    run(x, (int)M, y, workspace_.nbytes() ? workspace_.data<void>() : nullptr, workspace_.nbytes(), s);
  }
  return y;
}

MLP::MLP(int hidden_size, int intermediate_size)
    : hidden_(hidden_size),
      inter_(intermediate_size),
      gate_(hidden_size, intermediate_size, false),
      up_(hidden_size, intermediate_size, false),
      down_(intermediate_size, hidden_size, false) {}

size_t MLP::workspace_size(int M, kernels::Dtype dtype) const {
  if (gate_.weight_.dtype() != kernels::Dtype::packed || up_.weight_.dtype() != kernels::Dtype::packed)
    throw std::runtime_error("MLP: gate/up weights not loaded");
  size_t ws = 0;
  check(mlxr_qgemm_swiglu_workspace_size((int)gate_.weight_.quant_type(), inter_, hidden_, M, dt_code(dtype), &ws));
  return std::max(ws, down_.workspace_size(M));
}

void MLP::forward(const kernels::array& x, kernels::array& y, kernels::array& h, void* workspace,
                  size_t workspace_bytes, kernels::Stream s) {
  const long M = rows_of(x, hidden_, "hidden_size");
  if (gate_.weight_.dtype() != kernels::Dtype::packed || up_.weight_.dtype() != kernels::Dtype::packed)
    throw std::runtime_error("MLP: gate/up weights not loaded");
  const int qt = (int)gate_.weight_.quant_type();
  if (qt != (int)up_.weight_.quant_type()) throw std::runtime_error("MLP: gate and up must share a quant type");
  if (h.dtype() != x.dtype() || h.nbytes() < (size_t)M * (size_t)inter_ * kernels::dtype_size(x.dtype()))
    throw std::runtime_error("MLP: h must hold [M, intermediate_size] in the input dtype");
  if (M == 0) return;
  const int dt = dt_code(x.dtype());
  // gate, up and the gating: one launch (the fused kernels) for every M whose operands
  // stay below 2 GiB; the workspace holds split-K partials, or up when unfused
  check(mlxr_qgemm_swiglu(qt, inter_, hidden_, gate_.weight_.data<void>(), up_.weight_.data<void>(), x.data<void>(),
                          dt, h.data<void>(), dt, (int)M, workspace_bytes ? workspace : nullptr,
                          workspace ? workspace_bytes : 0, s.hip_stream));
  std::vector<int> hshape = x.shape();
  hshape.back() = inter_;
  const kernels::array hv = kernels::array::borrow(h.data<void>(), hshape, x.dtype());
  down_.forward(hv, y, workspace, workspace_bytes, s);
}

kernels::array MLP::forward(const kernels::array& x, kernels::Stream s) {
  const long M = rows_of(x, hidden_, "hidden_size");
  kernels::array y(x.shape(), x.dtype(), s);
  if (M == 0) return y;
  if (gate_.weight_.dtype() != kernels::Dtype::packed || up_.weight_.dtype() != kernels::Dtype::packed ||
      down_.weight_.dtype() != kernels::Dtype::packed)
    throw std::runtime_error("MLP: weights not loaded");
  const int qt = (int)gate_.weight_.quant_type(), qd = (int)down_.weight_.quant_type();
  if (qt != (int)up_.weight_.quant_type()) throw std::runtime_error("MLP: gate and up must share a quant type");
  // the whole block through mlxr_qgemm_mlp: one launch at M = 1, else gate/up/gating and
  // down; its workspace (sync words, h, split-K partials) is held by the layer
  size_t need = 0;
  check(mlxr_qgemm_mlp_workspace_size(qt, qd, hidden_, inter_, (int)M, &need));
  if (need > 0x7fffffffu) throw std::runtime_error("MLP: workspace of 2 GiB or more");
  if (grow_workspace(workspace_, ws_alloc_stream_, ws_last_stream_, need, s))
    check(mlxr_qgemm_mlp_workspace_init(workspace_.data<void>(), workspace_.nbytes(), s.hip_stream));
  const int dt = dt_code(x.dtype());
  check(mlxr_qgemm_mlp(qt, qd, hidden_, inter_, gate_.weight_.data<void>(), up_.weight_.data<void>(),
                       down_.weight_.data<void>(), x.data<void>(), dt, y.data<void>(), dt, (int)M,
                       workspace_.data<void>(), workspace_.nbytes(), s.hip_stream));
  return y;
}

}  // namespace graph
}  // namespace mlxr
