// ipc_gemm_pf.hip - prediction+error and forward launches (layout PF):
// C = W[M][K] . f(X_upper[K][N]); the 16-bit operand paths can split W (and
// f(X)) into hi + lo terms for a more accurate prediction.
#include "ipc_gemm_kernel.h"

namespace ipc {

template <typename ST, typename OT>
static hipError_t pf_split(const GemmProblem* probs, int count, int split, int tile, hipStream_t s) {
  switch (split) {
    case 2: return run_tiles<ST, OT, LAYOUT_PF, 2>(probs, count, tile, s);
    case 3: return run_tiles<ST, OT, LAYOUT_PF, 3>(probs, count, tile, s);
    default: return run_tiles<ST, OT, LAYOUT_PF, 1>(probs, count, tile, s);
  }
}

hipError_t launch_layout_pf(const GemmProblem* probs, int count, int storage, int operand, int split, int tile,
                            hipStream_t s) {
  if (storage == DT_F32) {
    if (operand == DT_F32) return run_tiles<float, float, LAYOUT_PF, 1>(probs, count, tile, s);
    if (operand == DT_F16) return pf_split<float, f16>(probs, count, split, tile, s);
    return pf_split<float, bf16>(probs, count, split, tile, s);
  }
  if (storage == DT_F16) return run_tiles<f16, f16, LAYOUT_PF, 1>(probs, count, tile, s);
  return run_tiles<bf16, bf16, LAYOUT_PF, 1>(probs, count, tile, s);
}

}  // namespace ipc
