// ipc_s16_t2.hip - standalone 16-bit kernels, tile configuration 2 (128 x 128).
#include "ipc_s16_tiles.h"

namespace ipc {
namespace s16 {

hipError_t launch_tiles2(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s) {
  return Tiles<128, 128, 2, 2, 2, 2, 2>::launch(mode, probs, count, operand, act, s);
}

}  // namespace s16
}  // namespace ipc
