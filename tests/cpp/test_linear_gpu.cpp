// C++ Linear / MLP layers (include/mlxr_linear.h) on the GPU: Linear::forward over a 3-D
// input equals the q_gemm_dequant operator on the flattened rows bit for bit (same kernel
// at these M), a GGUF-loaded weight gives the same result as one packed from host bytes,
// MLP::forward equals the chain (fused mlxr_qgemm_swiglu, then down), the forward
// overloads with caller-owned outputs and workspace equal the allocating ones, and a HIP
// graph of them replays to the same bits.  With a second argument (a directory) it writes
// the Linear output at M = 3 and the MLP output at M = 24 (bf16 bits) there, which
// tests/test_layers.py checks against the oracle.  Prints "OK <n>" on success.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "mlxr_gguf.h"
#include "mlxr_linear.h"
#include "mlxr_qgemm.h"

using namespace mlxr;
using kernels::array;
using kernels::Dtype;
using kernels::QuantType;

static int checks = 0;
#define EXPECT(c)                                             \
  do {                                                        \
    ++checks;                                                 \
    if (!(c)) {                                               \
      std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
      return 1;                                               \
    }                                                         \
  } while (0)

static std::vector<uint8_t> to_host(const array& a) {
  std::vector<uint8_t> h(a.nbytes());
  if (hipMemcpy(h.data(), a.data<void>(), a.nbytes(), hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("copy");
  return h;
}

static array act(int rows, int K, uint64_t seed) {
  std::vector<uint16_t> h((size_t)rows * K);
  mlxr_synth_act(h.size(), MLXR_BF16, seed, h.data());
  array a({rows, K}, Dtype::bfloat16);
  if (hipMemcpy(a.data<void>(), h.data(), h.size() * 2, hipMemcpyHostToDevice) != hipSuccess)
    throw std::runtime_error("copy");
  return a;
}

static void dump(const char* dir, const char* name, const array& a) {
  if (!dir) return;
  const std::vector<uint8_t> h = to_host(a);
  FILE* f = std::fopen((std::string(dir) + "/" + name).c_str(), "wb");
  if (!f) throw std::runtime_error("dump");
  std::fwrite(h.data(), 1, h.size(), f);
  std::fclose(f);
}

int main(int argc, char** argv) {
  const char* gguf_path = argc > 1 ? argv[1] : nullptr;  // file with tensor "w" (Q4_K, dims {512, 384})
  const char* out_dir = argc > 2 ? argv[2] : nullptr;
  const int K = 512, N = 384;
  std::vector<uint8_t> w((size_t)N * K / 256 * 144);
  mlxr_synth_gguf(MLXR_Q4_K, N, K, 77, w.data());

  graph::Linear lin(K, N, true);
  lin.load_weight(w.data(), QuantType::Q4_K);
  std::vector<uint16_t> bh(N);
  mlxr_synth_act(N, MLXR_BF16, 5, bh.data());
  array bias({N}, Dtype::bfloat16);
  hipMemcpy(bias.data<void>(), bh.data(), N * 2, hipMemcpyHostToDevice);
  lin.set_bias(bias);

  for (int M : {1, 3, 40}) {
    array x2 = act(M, K, 100 + M);
    array x3 = array::borrow(x2.data<void>(), {1, M, K}, Dtype::bfloat16);
    array y3 = lin.forward(x3);
    EXPECT(y3.ndim() == 3 && y3.shape(0) == 1 && y3.shape(1) == M && y3.shape(2) == N);
    array yo = kernels::q_gemm_dequant(x2, lin.weight(), M, N, K, QuantType::Q4_K, 0, &bias);
    hipDeviceSynchronize();
    EXPECT(to_host(y3) == to_host(yo));
    // caller-owned output and workspace: same bits
    array yc({M, N}, Dtype::bfloat16);
    const size_t wsb = lin.workspace_size(M);
    array w({(int)wsb + 1}, Dtype::uint8);
    lin.forward(x3, yc, w.data<void>(), wsb);
    hipDeviceSynchronize();
    EXPECT(to_host(yc) == to_host(yo));
    if (M == 3) dump(out_dir, "linear_m3.bin", yc);
  }

  // The layer's split-K workspace used on a second stream and then grown there: the old
  // buffer is released only after that stream's work, and results stay exact.
  {
    graph::Linear ls(4096, 1024, false);
    std::vector<uint8_t> wl((size_t)1024 * 4096 / 256 * 144);
    mlxr_synth_gguf(MLXR_Q4_K, 1024, 4096, 78, wl.data());
    ls.load_weight(wl.data(), QuantType::Q4_K);
    hipStream_t sa, sb;
    EXPECT(hipStreamCreate(&sa) == hipSuccess && hipStreamCreate(&sb) == hipSuccess);
    array xa = act(40, 4096, 31), xb = act(300, 4096, 32);
    hipDeviceSynchronize();
    for (int rep = 0; rep < 2; ++rep) {
      array ya = ls.forward(xa, kernels::Stream{sa});  // allocates the workspace on sa
      EXPECT(hipStreamSynchronize(sa) == hipSuccess);
      array yb = ls.forward(xa, kernels::Stream{sb});  // reuses it on sb
      array yg = ls.forward(xb, kernels::Stream{sb});  // grows it: frees sa's buffer after sb's work
      EXPECT(hipStreamSynchronize(sb) == hipSuccess);
      // references: the caller-owned forward with its own workspace (same split plans)
      array ra({40, 1024}, Dtype::bfloat16), rg({300, 1024}, Dtype::bfloat16);
      const size_t wr = std::max(ls.workspace_size(40), ls.workspace_size(300));
      array wref({(int)wr + 1}, Dtype::uint8);
      ls.forward(xa, ra, wref.data<void>(), wr);
      ls.forward(xb, rg, wref.data<void>(), wr);
      hipDeviceSynchronize();
      EXPECT(to_host(ya) == to_host(ra) && to_host(yb) == to_host(ra) && to_host(yg) == to_host(rg));
      ls = graph::Linear(4096, 1024, false);  // fresh layer (empty workspace) for the second round
      ls.load_weight(wl.data(), QuantType::Q4_K);
    }
    hipStreamDestroy(sa);
    hipStreamDestroy(sb);
  }

  if (gguf_path) {
    mlxr_gguf* g = nullptr;
    EXPECT(mlxr_gguf_open(gguf_path, &g) == 0);
    graph::Linear lg(K, N, true);
    lg.load_weight(g, "w");
    lg.set_bias(bias);
    array x = act(7, K, 9);
    array a = lg.forward(x), b = lin.forward(x);
    hipDeviceSynchronize();
    EXPECT(to_host(a) == to_host(b));
    bool threw = false;
    try {
      lg.load_weight(g, "missing");
    } catch (const std::runtime_error&) {
      threw = true;
    }
    EXPECT(threw);
    mlxr_gguf_close(g);
  }

  // MLP: hidden 256, intermediate 512
  const int H = 256, I = 512;
  graph::MLP mlp(H, I);
  std::vector<uint8_t> wg((size_t)I * H / 256 * 144), wu(wg.size()), wd((size_t)H * I / 256 * 144);
  mlxr_synth_gguf(MLXR_Q4_K, I, H, 1, wg.data());
  mlxr_synth_gguf(MLXR_Q4_K, I, H, 2, wu.data());
  mlxr_synth_gguf(MLXR_Q4_K, H, I, 3, wd.data());
  mlp.gate_proj().load_weight(wg.data(), QuantType::Q4_K);
  mlp.up_proj().load_weight(wu.data(), QuantType::Q4_K);
  mlp.down_proj().load_weight(wd.data(), QuantType::Q4_K);
  for (int M : {1, 2, 24, 100}) {
    array x = act(M, H, 50 + M);
    array y = mlp.forward(x);
    array h({M, I}, Dtype::bfloat16);
    EXPECT(mlxr_qgemm_swiglu(MLXR_Q4_K, I, H, mlp.gate_proj().weight().data<void>(),
                             mlp.up_proj().weight().data<void>(), x.data<void>(), MLXR_BF16, h.data<void>(),
                             MLXR_BF16, M, nullptr, 0, nullptr) == 0);
    array y2 = mlp.down_proj().forward(h);
    hipDeviceSynchronize();
    // unsplit chain equals the layer wherever the layer's launches do not split
    size_t need = 0;
    EXPECT(mlxr_qgemm_swiglu_workspace_size(MLXR_Q4_K, I, H, M, MLXR_BF16, &need) == 0);
    if (need == 0 && mlp.down_proj().workspace_size(M) == 0) EXPECT(to_host(y) == to_host(y2));
    // caller-owned y, h and workspace (no allocation inside): same bits as the allocating
    // forward, eagerly and from a captured graph replayed three times
    const size_t wsb = mlp.workspace_size(M);
    array w({(int)wsb + 1}, Dtype::uint8);
    array yc({M, H}, Dtype::bfloat16), hc({M, I}, Dtype::bfloat16);
    mlp.forward(x, yc, hc, w.data<void>(), wsb);
    hipDeviceSynchronize();
    EXPECT(to_host(yc) == to_host(y));
    hipStream_t cs;
    EXPECT(hipStreamCreate(&cs) == hipSuccess);
    hipGraph_t graph;
    hipGraphExec_t exec;
    array yg({M, H}, Dtype::bfloat16);
    EXPECT(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal) == hipSuccess);
    mlp.forward(x, yg, hc, w.data<void>(), wsb, kernels::Stream{cs});
    EXPECT(hipStreamEndCapture(cs, &graph) == hipSuccess);
    EXPECT(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess);
    for (int rep = 0; rep < 3; ++rep) {
      EXPECT(hipMemset(yg.data<void>(), 0, yg.nbytes()) == hipSuccess);
      EXPECT(hipGraphLaunch(exec, cs) == hipSuccess);
      EXPECT(hipStreamSynchronize(cs) == hipSuccess);
      EXPECT(to_host(yg) == to_host(y));
    }
    hipGraphExecDestroy(exec);
    hipGraphDestroy(graph);
    hipStreamDestroy(cs);
    if (M == 24) dump(out_dir, "mlp_m24.bin", yc);
  }
  std::printf("OK %d\n", checks);
  return 0;
}
