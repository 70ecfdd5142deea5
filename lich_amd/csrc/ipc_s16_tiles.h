// ipc_s16_tiles.h - the tile configurations of the standalone 16-bit-storage
// kernels (operator API, src/ipc_tilelang/tilelang_kernels.py:114-349) on the
// LDS-DMA MFMA kernel of ipc_dma_gemm.h.  Each configuration is compiled in a
// translation unit of its own (ipc_s16.hip, ipc_s16_t1.hip .. ipc_s16_t3.hip)
// and chosen per call by its tile id, which is what the autotuner searches.
// The k order, and so every result bit, does not depend on the configuration.
#pragma once

#include "ipc_dma_gemm.h"

namespace ipc {
namespace s16 {

// BM x BN output tiles, S stages; PM x PN waves for the prediction, forward
// and inference kernels, WM x WN for the weight update.
template <int BM, int BN, int S, int PM, int PN, int WM, int WN>
struct Tiles {
  template <typename OT>
  struct ForType {
    template <int ACT>
    struct Run {
      static hipError_t run(int mode, const WideProblem* probs, int count, hipStream_t s) {
        constexpr bool R = ACT != ACT_IDENTITY;  // activation in the B loader: register path
        switch (mode) {
          case S16_PRED: return dma::Cfg<OT, S16_PRED, 1, ACT, R, BM, BN, S, PM, PN>::launch(probs, count, s);
          case S16_FWD: return dma::Cfg<OT, S16_FWD, 1, ACT, R, BM, BN, S, PM, PN>::launch(probs, count, s);
          case S16_INFER: return dma::Cfg<OT, S16_INFER, 1, ACT, false, BM, BN, S, PM, PN>::launch(probs, count, s);
          case S16_INFERT: return dma::Cfg<OT, S16_INFERT, 1, ACT, false, BM, BN, S, PM, PN>::launch(probs, count, s);
          case S16_PREDT:
          case S16_FWDT:
            // f(X_upper)^T from a caller workspace: the activation is applied
            if constexpr (ACT == ACT_IDENTITY) {
              if (mode == S16_PREDT)
                return dma::Cfg<OT, S16_PREDT, 1, ACT, false, BM, BN, S, PM, PN>::launch(probs, count, s);
              return dma::Cfg<OT, S16_FWDT, 1, ACT, false, BM, BN, S, PM, PN>::launch(probs, count, s);
            } else {
              return hipErrorInvalidValue;
            }
          default: return dma::Cfg<OT, S16_WEIGHT, 1, ACT, R, BM, BN, S, WM, WN>::launch(probs, count, s);
        }
      }
    };
  };

  static hipError_t launch(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s) {
    for (int base = 0; base < count; base += WIDE_MAX_BATCH) {
      const int n = count - base < WIDE_MAX_BATCH ? count - base : WIDE_MAX_BATCH;
      hipError_t e;
      if (operand == DT_F16) e = dma::by_act<ForType<f16>::template Run>(act, mode, probs + base, n, s);
      else if (operand == DT_BF16) e = dma::by_act<ForType<bf16>::template Run>(act, mode, probs + base, n, s);
      else return hipErrorInvalidValue;
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
};

// Configuration 1: 128 x 256 tiles (16 waves of 32 x 64; the weight update 8
// of 64 x 64), 3 stages.  Configuration 2: 128 x 128 tiles, 4 waves of
// 64 x 64, 2 stages (66 KB of LDS: two workgroups per CU), for shapes with
// few tiles.
// Configuration 3: 256 x 256 tiles, 8 waves of 128 x 64, 2 stages, finished
// from the registers (the fp32 tile exceeds the LDS).
hipError_t launch_tiles1(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s);
hipError_t launch_tiles2(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s);
hipError_t launch_tiles3(int mode, const WideProblem* probs, int count, int operand, int act, hipStream_t s);

}  // namespace s16
}  // namespace ipc
