// ipc_gemm_inf.hip - inference update (layout INF): C = W_lower[K][M]^T . E_lower[K][N].
#include "ipc_gemm_kernel.h"

namespace ipc {

hipError_t launch_layout_inf(const GemmProblem* probs, int count, int storage, int operand, int tile,
                             hipStream_t s) {
  if (storage == DT_F32) {
    if (operand == DT_F32) return run_tiles<float, float, LAYOUT_INF, 1>(probs, count, tile, s);
    if (operand == DT_F16) return run_tiles<float, f16, LAYOUT_INF, 1>(probs, count, tile, s);
    return run_tiles<float, bf16, LAYOUT_INF, 1>(probs, count, tile, s);
  }
  if (storage == DT_F16) return run_tiles<f16, f16, LAYOUT_INF, 1>(probs, count, tile, s);
  return run_tiles<bf16, bf16, LAYOUT_INF, 1>(probs, count, tile, s);
}

}  // namespace ipc
