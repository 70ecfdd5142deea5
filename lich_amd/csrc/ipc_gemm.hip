// ipc_gemm.hip - dispatch of the GEMM family to its per-layout launchers.
#include "ipc_gemm_kernel.h"

namespace ipc {

TileShape tile_shape(int tile) {
  switch (tile) {
    case 0: return {32, 32, 32, 64};
    case 1: return {64, 64, 32, 256};
    default: return {128, 128, 32, 256};
  }
}

hipError_t launch_gemm(const GemmProblem* probs, int count, int storage, int operand, int split, int tile,
                       hipStream_t s) {
  if (count <= 0) return hipSuccess;
  switch (probs[0].kind) {
    case KIND_PRED:
    case KIND_FWD: return launch_layout_pf(probs, count, storage, operand, split, tile, s);
    case KIND_INFER: return launch_layout_inf(probs, count, storage, operand, tile, s);
    default: return launch_layout_wgt(probs, count, storage, operand, tile, s);
  }
}

}  // namespace ipc
