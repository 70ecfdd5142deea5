// ipc_gemm_wgt.hip - weight update (layout WGT): C = E[M][Bt] . f(X_upper[N][Bt])^T.
#include "ipc_gemm_kernel.h"

namespace ipc {

hipError_t launch_layout_wgt(const GemmProblem* probs, int count, int storage, int operand, int tile,
                             hipStream_t s) {
  if (storage == DT_F32) {
    if (operand == DT_F32) return run_tiles<float, float, LAYOUT_WGT, 1>(probs, count, tile, s);
    if (operand == DT_F16) return run_tiles<float, f16, LAYOUT_WGT, 1>(probs, count, tile, s);
    return run_tiles<float, bf16, LAYOUT_WGT, 1>(probs, count, tile, s);
  }
  if (storage == DT_F16) return run_tiles<f16, f16, LAYOUT_WGT, 1>(probs, count, tile, s);
  return run_tiles<bf16, bf16, LAYOUT_WGT, 1>(probs, count, tile, s);
}

}  // namespace ipc
