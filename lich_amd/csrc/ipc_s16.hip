// ipc_s16.hip - standalone prediction / forward / inference / weight-update
// kernels of the operator API for 16-bit storage (the reference kernels'
// storage design, src/ipc_tilelang/tilelang_kernels.py:114-349) on the
// LDS-DMA MFMA kernel of ipc_dma_gemm.h: the caller's tensors are the
// operands, f(X_upper) goes through the register path when an activation
// applies, every other operand through LDS DMA.
#include "ipc_dma_gemm.h"

namespace ipc {
namespace {

using dma::Cfg;

#ifndef S16_CFG
#define S16_CFG 256, 128, 3, 4, 2
#endif

template <typename OT>
struct S16 {
  template <int ACT>
  struct Run {
    static hipError_t run(int mode, const WideProblem* probs, int count, hipStream_t s) {
      constexpr bool R = ACT != ACT_IDENTITY;  // activation in the B loader: register path
      switch (mode) {
        case S16_PRED: return Cfg<OT, S16_PRED, 1, ACT, R, S16_CFG>::launch(probs, count, s);
        case S16_FWD: return Cfg<OT, S16_FWD, 1, ACT, R, S16_CFG>::launch(probs, count, s);
        case S16_INFER: return Cfg<OT, S16_INFER, 1, ACT, false, S16_CFG>::launch(probs, count, s);
        default: return Cfg<OT, S16_WEIGHT, 1, ACT, R, S16_CFG>::launch(probs, count, s);
      }
    }
  };
};

}  // namespace

hipError_t launch_s16(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s) {
  for (int base = 0; base < count; base += WIDE_MAX_BATCH) {
    const int n = count - base < WIDE_MAX_BATCH ? count - base : WIDE_MAX_BATCH;
    hipError_t e;
    if (operand == DT_F16) e = dma::by_act<S16<f16>::template Run>(act, mode, probs + base, n, s);
    else if (operand == DT_BF16) e = dma::by_act<S16<bf16>::template Run>(act, mode, probs + base, n, s);
    else return hipErrorInvalidValue;
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ipc
