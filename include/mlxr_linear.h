// Quantized Linear and MLP layers over the q_gemm_dequant operator: the caller side of the
// path, as the reference plans it for core/graph/layers.cpp:86-99 (Linear::forward,
// y = x W^T + b over x [..., in_features]) with M = batch * seq
// (docs/SESSION_2025_11_07_MODEL_LOADING.md:133-160), and MLP::forward
// (layers.cpp:391-414: down(swish(gate(x)) * up(x))).
//
// Names and meaning follow the reference classes (core/graph/layers.h:59-94 Linear; MLP
// beside it); the weight is held as packed GGUF blocks in device memory instead of an MLX
// float tensor.  forward() takes and returns device arrays (bf16 or fp16 activations,
// output in the input dtype) and runs on the given HIP stream; it is stream-ordered and
// never synchronises.  The allocating forward() uses stream-ordered allocations
// (hipMallocAsync / hipFreeAsync) for its output and temporaries; the forward() overloads
// with caller-owned outputs and workspace allocate nothing.  One layer must not run the
// allocating forward on two streams at once (its split-K workspace is per layer).  Errors
// throw std::runtime_error, as the reference does.
#pragma once

#include <string>
#include <vector>

#include "mlxr_gguf.h"
#include "q_gemm_dequant_primitive.h"

namespace mlxr {
namespace graph {

class Linear {
 public:
  // in_features = K, out_features = N (reference layers.h:67).
  Linear(int in_features, int out_features, bool bias = false);

  // Weight [out_features, in_features] as GGUF blocks in host memory (e.g. a mapped
  // tensor), packed into device memory once.
  void load_weight(const void* gguf_host, kernels::QuantType quant_type, kernels::Stream s = {});
  // Weight tensor `name` of an open GGUF file (ggml dims {in_features, out_features}).
  void load_weight(const mlxr_gguf* file, const std::string& name, kernels::Stream s = {});
  // Bias [out_features] on the device (fp32, fp16 or bf16).  Only for layers built with bias.
  void set_bias(const kernels::array& bias);

  // x [..., in_features] -> [..., out_features], M = product of the leading dims.  The
  // output (and a split-K workspace kept by the layer) are stream-ordered allocations on s.
  kernels::array forward(const kernels::array& x, kernels::Stream s = {});
  // Same into the caller's y (M * out_features elements of float32, float16 or bfloat16)
  // with the caller's workspace (NULL / too small: unsplit): allocates nothing and never
  // synchronises, so it can be captured into a HIP graph.
  void forward(const kernels::array& x, kernels::array& y, void* workspace, size_t workspace_bytes,
               kernels::Stream s = {});
  // Workspace bytes forward() can use at M rows (0: none needed).
  size_t workspace_size(int M) const;

  const kernels::array& weight() const { return weight_; }
  const kernels::array* bias() const { return has_bias_ ? &bias_ : nullptr; }
  int in_features() const { return in_features_; }
  int out_features() const { return out_features_; }

 private:
  friend class MLP;
  void run(const kernels::array& x, int M, kernels::array& y, void* ws, size_t ws_bytes, kernels::Stream s);
  int in_features_, out_features_;
  bool has_bias_;
  kernels::array weight_;  // Dtype::packed
  kernels::array bias_;
  kernels::array workspace_;  // split-K partial sums, grown on demand
  void* ws_alloc_stream_ = nullptr;  // stream workspace_ was allocated (and is freed) on
  void* ws_last_stream_ = nullptr;   // stream of its last use
};

// SwiGLU MLP (reference layers.cpp:383-414): down(swish(gate(x)) * up(x)).
class MLP {
 public:
  MLP(int hidden_size, int intermediate_size);
  Linear& gate_proj() { return gate_; }
  Linear& up_proj() { return up_; }
  Linear& down_proj() { return down_; }
  // x [..., hidden] -> [..., hidden] through mlxr_qgemm_mlp (at M = 1 the whole block is
  // one launch); the output is a stream-ordered allocation on s and the workspace (sync
  // words, h, split-K partials) is held by the layer, grown on demand.  One layer must not
  // run this forward on two streams at once.
  kernels::array forward(const kernels::array& x, kernels::Stream s = {});
  // Same into the caller's y ([..., hidden], x's dtype) with the caller's h ([M,
  // intermediate] in x's dtype: swish(gate) * up) and workspace (workspace_size bytes;
  // NULL / smaller: unsplit launches, except for operands of 2 GiB or more, which need it):
  // allocates nothing and never synchronises (HIP-graph capturable).
  void forward(const kernels::array& x, kernels::array& y, kernels::array& h, void* workspace,
               size_t workspace_bytes, kernels::Stream s = {});
  size_t workspace_size(int M, kernels::Dtype dtype = kernels::Dtype::bfloat16) const;

 private:
  int hidden_, inter_;
  Linear gate_, up_, down_;
  kernels::array workspace_;  // mlxr_qgemm_mlp workspace, grown (and initialised) on demand
  void* ws_alloc_stream_ = nullptr;
  void* ws_last_stream_ = nullptr;
};

}  // namespace graph
}  // namespace mlxr
