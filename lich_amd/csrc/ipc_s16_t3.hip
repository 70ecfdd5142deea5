// ipc_s16_t3.hip - standalone 16-bit kernels, tile configuration 3 (256 x 256).
#include "ipc_s16_tiles.h"

namespace ipc {
namespace s16 {

hipError_t launch_tiles3(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s) {
  return Tiles<256, 256, 2, 2, 4, 2, 4>::launch(mode, probs, count, operand, act, s);
}

}  // namespace s16
}  // namespace ipc
