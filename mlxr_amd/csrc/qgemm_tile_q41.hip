// Instantiates the prefill GEMM kernel (qgemm_tile_kernel.h) for Q4_1 weights; one
// translation unit per quant type keeps the build parallel.
#include "qgemm_tile_kernel.h"

namespace mlxr {
namespace tile {

hipError_t launch_tile_q41(const TileParams& tp, int bm, int S, bool f16, hipStream_t s) {
  return f16 ? launch_q<QT_Q4_1, X_F16>(tp, bm, S, s) : launch_q<QT_Q4_1, X_BF16>(tp, bm, S, s);
}

}  // namespace tile
}  // namespace mlxr
