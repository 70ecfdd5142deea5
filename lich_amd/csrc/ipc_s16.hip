// ipc_s16.hip - standalone prediction / forward / inference / weight-update
// kernels of the operator API for 16-bit storage (the reference kernels'
// storage design, src/ipc_tilelang/tilelang_kernels.py:114-349) on the
// LDS-DMA MFMA kernel of ipc_dma_gemm.h: the caller's tensors are the
// operands, f(X_upper) goes through the register path when an activation
// applies (or, for large calls given a caller workspace, is evaluated once
// into it by s16_activate_kernel and read through LDS DMA like every other
// operand).  This file holds tile configuration 0 and the dispatch over the
// configurations of ipc_s16_tiles.h.
#include "ipc_s16_tiles.h"

namespace ipc {
namespace {

// Tile configuration 0, the default (IPC_TILE_DMA_256x128): 256 x 128 tiles;
// the prediction, forward and inference kernels run 16 waves (64 x 32 per
// wave, four per SIMD to hide the LDS reads and barriers), 1-10 % faster than
// 8 waves at M = K >= 4096, B >= 2048; the weight update keeps 8 waves (64 x
// 64 each), within +-3 % of 16.
using Tiles0 = s16::Tiles<256, 128, 3, 4, 4, 4, 2>;

// out[i] = f(in[i]) rounded to the storage type: the register path's value
// (f in fp32 of the stored 16-bit input, then one rounding), 8 elements per
// thread when the buffers allow 16-byte accesses.
template <typename OT, int ACT>
__global__ void __launch_bounds__(256) s16_activate_kernel(const OT* __restrict__ in, OT* __restrict__ out,
                                                           long long n, int vec8) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec8) {
    for (; i * 8 < n; i += stride) {
      const uint4 v = reinterpret_cast<const uint4*>(in)[i];
      const unsigned w[4] = {v.x, v.y, v.z, v.w};
      unsigned o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = dma::pack2(cvt<OT>(act_t<ACT>(dma::lo16<OT>(w[j]))), cvt<OT>(act_t<ACT>(dma::hi16<OT>(w[j]))));
      reinterpret_cast<uint4*>(out)[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    for (; i < n; i += stride) out[i] = cvt<OT>(act_t<ACT>(to_f32(in[i])));
  }
}

template <typename OT>
struct Activate {
  template <int ACT>
  struct Run {
    static hipError_t run(const void* in, void* out, long long n, hipStream_t s) {
      const int vec8 = (n % 8 == 0) && (reinterpret_cast<uintptr_t>(in) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(out) % 16 == 0);
      const long long items = vec8 ? n / 8 : n;
      const int blocks = (int)std::min<long long>((items + 255) / 256, 8192);
      hipLaunchKernelGGL((s16_activate_kernel<OT, ACT>), dim3(blocks), dim3(256), 0, s,
                         static_cast<const OT*>(in), static_cast<OT*>(out), n, vec8);
      return hipGetLastError();
    }
  };
};

template <template <int> class R, typename... Args>
hipError_t by_act_only(int act, Args... a) {
  switch (act) {
    case ACT_RELU: return R<ACT_RELU>::run(a...);
    case ACT_TANH: return R<ACT_TANH>::run(a...);
    case ACT_SIGMOID: return R<ACT_SIGMOID>::run(a...);
    case ACT_SILU: return R<ACT_SILU>::run(a...);
    case ACT_GELU: return R<ACT_GELU>::run(a...);
    default: return R<ACT_IDENTITY>::run(a...);
  }
}

}  // namespace

hipError_t launch_s16_activate(const void* in, void* out, long long n, int operand, int act, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (operand == DT_F16) return by_act_only<Activate<f16>::template Run>(act, in, out, n, s);
  if (operand == DT_BF16) return by_act_only<Activate<bf16>::template Run>(act, in, out, n, s);
  return hipErrorInvalidValue;
}

hipError_t launch_s16(int mode, const WideProblem* probs, int count, int operand, int act, int cfg, hipStream_t s) {
  switch (cfg) {
    case 0: return Tiles0::launch(mode, probs, count, operand, act, s);
    case 1: return s16::launch_tiles1(mode, probs, count, operand, act, s);
    case 2: return s16::launch_tiles2(mode, probs, count, operand, act, s);
    case 3: return s16::launch_tiles3(mode, probs, count, operand, act, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ipc
