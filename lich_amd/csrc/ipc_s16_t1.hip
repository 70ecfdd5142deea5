// ipc_s16_t1.hip - standalone 16-bit kernels, tile configuration 1 (128 x 256).
#include "ipc_s16_tiles.h"

namespace ipc {
namespace s16 {

hipError_t launch_tiles1(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s) {
  return Tiles<128, 256, 3, 4, 4, 2, 4>::launch(mode, probs, count, operand, act, s);
}

}  // namespace s16
}  // namespace ipc
