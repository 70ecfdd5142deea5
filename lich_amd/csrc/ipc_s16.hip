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

// out[g][b][k] = cvt(f(in[g][k][b])): one 64 x 64 block of group blockIdx.z
// per workgroup, read along b and written along k (both 16 elements per
// thread, 16-byte accesses when the rows allow them), transposed in LDS.
// The values are those of s16_activate_kernel.
template <typename OT, int ACT>
__global__ void __launch_bounds__(256) s16_activate_t_kernel(const OT* __restrict__ in, OT* __restrict__ out,
                                                             int K, int B, long long gstride) {
  __shared__ unsigned short tile[64][64 + 2];  // [b][k]; the padding spreads a column walk over banks
  const OT* src = in + (long long)blockIdx.z * gstride;
  OT* dst = out + (long long)blockIdx.z * gstride;
  const int k0 = blockIdx.y * 64, b0 = blockIdx.x * 64, t = threadIdx.x;
  {
    const int r = t >> 2, c0 = (t & 3) * 16, k = k0 + r;
    unsigned short v[16];
    if (k < K && b0 + c0 + 16 <= B && B % 8 == 0) {
      const uint4* p = reinterpret_cast<const uint4*>(src + (long long)k * B + b0 + c0);
      const uint4 u[2] = {p[0], p[1]};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const unsigned w[4] = {u[h].x, u[h].y, u[h].z, u[h].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[h * 8 + 2 * j] = __builtin_bit_cast(unsigned short, cvt<OT>(act_t<ACT>(dma::lo16<OT>(w[j]))));
          v[h * 8 + 2 * j + 1] = __builtin_bit_cast(unsigned short, cvt<OT>(act_t<ACT>(dma::hi16<OT>(w[j]))));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int b = b0 + c0 + i;
        v[i] = k < K && b < B ? __builtin_bit_cast(unsigned short, cvt<OT>(act_t<ACT>(to_f32(src[(long long)k * B + b]))))
                              : (unsigned short)0;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) tile[c0 + i][r] = v[i];
  }
  __syncthreads();
  {
    const int r = t >> 2, c0 = (t & 3) * 16, b = b0 + r;
    if (b >= B) return;
    unsigned short v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = tile[r][c0 + i];
    if (k0 + c0 + 16 <= K && K % 8 == 0) {
      uint4* p = reinterpret_cast<uint4*>(dst + (long long)b * K + k0 + c0);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        p[h] = make_uint4(v[h * 8] | ((unsigned)v[h * 8 + 1] << 16), v[h * 8 + 2] | ((unsigned)v[h * 8 + 3] << 16),
                          v[h * 8 + 4] | ((unsigned)v[h * 8 + 5] << 16), v[h * 8 + 6] | ((unsigned)v[h * 8 + 7] << 16));
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (k0 + c0 + i < K) dst[(long long)b * K + k0 + c0 + i] = __builtin_bit_cast(OT, v[i]);
    }
  }
}

template <typename OT>
struct ActivateT {
  template <int ACT>
  struct Run {
    static hipError_t run(const void* in, void* out, int K, int B, int groups, long long gstride, hipStream_t s) {
      hipLaunchKernelGGL((s16_activate_t_kernel<OT, ACT>), dim3((B + 63) / 64, (K + 63) / 64, groups), dim3(256), 0,
                         s, static_cast<const OT*>(in), static_cast<OT*>(out), K, B, gstride);
      return hipGetLastError();
    }
  };
};

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

hipError_t launch_s16_activate_t(const void* in, void* out, int K, int B, int groups, long long gstride,
                                 int operand, int act, hipStream_t s) {
  if (K <= 0 || B <= 0 || groups <= 0) return hipSuccess;
  if ((K + 63) / 64 > 65535 || groups > 65535) return hipErrorInvalidValue;
  if (operand == DT_F16) return by_act_only<ActivateT<f16>::template Run>(act, in, out, K, B, groups, gstride, s);
  if (operand == DT_BF16) return by_act_only<ActivateT<bf16>::template Run>(act, in, out, K, B, groups, gstride, s);
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
