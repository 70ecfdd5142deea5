// ipc_wide.hip - the GEMM path of wide nets (gfx950): one launch per phase
// over all layers of the LDS-DMA MFMA kernel of ipc_dma_gemm.h with the fused
// epilogues that keep the fp32 masters and their 16-bit operand copies in
// step, plus the kernel that re-derives the copies from the masters.
#include "ipc_dma_gemm.h"

namespace ipc {
namespace {

using dma::Cfg;

// BM, BN, stages, waves along M, waves along N
#ifndef WIDE_PRED1_CFG
#define WIDE_PRED1_CFG 256, 128, 3, 4, 2
#endif
// split-2 prediction: 128 x 128 tiles (3 stages in 144 KiB of LDS).  The wide
// configuration's 256 x 128 tiles came to 544 for 256 CUs (three rounds, the last
// one 1/8 full); 1,088 half-size tiles fill 4.25 rounds: 341 us instead of 377 us.
#ifndef WIDE_PRED2_CFG
#define WIDE_PRED2_CFG 128, 128, 3, 4, 2
#endif
#ifndef WIDE_INFER_CFG
#define WIDE_INFER_CFG 256, 128, 3, 4, 2
#endif
#ifndef WIDE_WEIGHT_CFG
#define WIDE_WEIGHT_CFG 256, 128, 3, 4, 2
#endif

template <typename OT, int ACT> using PredCfg1 = Cfg<OT, WIDE_PRED, 1, ACT_IDENTITY, false, WIDE_PRED1_CFG>;
template <typename OT, int ACT> using PredCfg2 = Cfg<OT, WIDE_PRED, 2, ACT_IDENTITY, false, WIDE_PRED2_CFG>;
template <typename OT, int ACT> using InferCfg = Cfg<OT, WIDE_INFER, 1, ACT, false, WIDE_INFER_CFG>;
template <typename OT, int ACT> using WeightCfg = Cfg<OT, WIDE_WEIGHT, 1, ACT_IDENTITY, false, WIDE_WEIGHT_CFG>;
// forward initialisation: the pred tiles (one layer per launch)
template <typename OT, int ACT> using FwdCfg1 = Cfg<OT, WIDE_FWD, 1, ACT, false, WIDE_PRED1_CFG>;
template <typename OT, int ACT> using FwdCfg2 = Cfg<OT, WIDE_FWD, 2, ACT, false, WIDE_PRED2_CFG>;

template <typename OT>
struct Phase {
  template <int ACT>
  struct Run {
    static hipError_t run(int mode, int split, const WideProblem* probs, int count, hipStream_t s) {
      switch (mode) {
        case WIDE_PRED:
          return split == 2 ? PredCfg2<OT, ACT>::launch(probs, count, s) : PredCfg1<OT, ACT>::launch(probs, count, s);
        case WIDE_INFER: return InferCfg<OT, ACT>::launch(probs, count, s);
        case WIDE_FWD:
          return split == 2 ? FwdCfg2<OT, ACT>::launch(probs, count, s) : FwdCfg1<OT, ACT>::launch(probs, count, s);
        default: return WeightCfg<OT, ACT>::launch(probs, count, s);
      }
    }
  };
  template <int ACT>
  struct Prep {
    static hipError_t run() {
      hipError_t e;
      if ((e = InferCfg<OT, ACT>::prepare()) != hipSuccess) return e;
      if ((e = FwdCfg1<OT, ACT>::prepare()) != hipSuccess) return e;
      return FwdCfg2<OT, ACT>::prepare();
    }
  };
  static hipError_t prepare() {
    hipError_t e;
    if ((e = PredCfg1<OT, 0>::prepare()) != hipSuccess) return e;
    if ((e = PredCfg2<OT, 0>::prepare()) != hipSuccess) return e;
    if ((e = WeightCfg<OT, 0>::prepare()) != hipSuccess) return e;
    for (int act = 0; act < 6; ++act)
      if ((e = dma::by_act<Prep>(act)) != hipSuccess) return e;
    return hipSuccess;
  }
};

// ---------------------------------------------------------------- copies
// 64 x 64 fp32 block per workgroup via LDS (for the transposed copy).
constexpr int CP_T = 64;
constexpr int CP_MAX = 2 * WIDE_MAX_BATCH;

struct WideCopyBatch {
  WideCopy c[CP_MAX];
  int start[CP_MAX + 1];
  int count;
};

template <typename OT>
__global__ void __launch_bounds__(256) wide_copy_kernel(const WideCopyBatch cb) {
  __shared__ float tile[CP_T][CP_T + 1];
  int ci = 0;
  const int b = blockIdx.x;
#pragma unroll 1
  while (ci + 1 < cb.count && b >= cb.start[ci + 1]) ++ci;
  const WideCopy& c = cb.c[ci];
  const int tc = (c.cols + CP_T - 1) / CP_T;
  const int local = b - cb.start[ci];
  const int r0 = (local / tc) * CP_T, c0 = (local % tc) * CP_T;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  OT* dst = reinterpret_cast<OT*>(c.dst);
  OT* lo = reinterpret_cast<OT*>(c.dst_lo);
#pragma unroll 4
  for (int rr = ty; rr < CP_T; rr += 4) {
    const int r = r0 + rr, col = c0 + tx;
    float v = 0.0f;
    if (r < c.rows && col < c.cols) {
      v = act_f(c.act, c.src[(long long)r * c.lds + col]);
      const OT hi = cvt<OT>(v);
      dst[(long long)r * c.ldd + col] = hi;
      if (lo) lo[(long long)r * c.ldl + col] = cvt<OT>(v - to_f32(hi));
      v = to_f32(hi);
    }
    tile[rr][tx] = v;
  }
  if (!c.dst_t) return;
  __syncthreads();
  OT* dt = reinterpret_cast<OT*>(c.dst_t);
#pragma unroll 4
  for (int cc = ty; cc < CP_T; cc += 4) {
    const int col = c0 + cc, r = r0 + tx;
    if (col < c.cols && r < c.rows) dt[(long long)col * c.ldt + r] = cvt<OT>(tile[tx][cc]);
  }
}

template <typename OT>
hipError_t launch_phase(int mode, const WideProblem* probs, int count, int split, int act, hipStream_t s) {
  return dma::by_act<Phase<OT>::template Run>(act, mode, split, probs, count, s);
}

}  // namespace

hipError_t wide_prepare() {
  hipError_t e = Phase<f16>::prepare();
  if (e != hipSuccess) return e;
  return Phase<bf16>::prepare();
}

hipError_t launch_wide(int mode, const WideProblem* probs, int count, int operand, int split, int act,
                       hipStream_t s) {
  for (int base = 0; base < count; base += WIDE_MAX_BATCH) {
    const int n = count - base < WIDE_MAX_BATCH ? count - base : WIDE_MAX_BATCH;
    hipError_t e;
    if (operand == DT_F16) e = launch_phase<f16>(mode, probs + base, n, split, act, s);
    else if (operand == DT_BF16) e = launch_phase<bf16>(mode, probs + base, n, split, act, s);
    else return hipErrorInvalidValue;
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_wide_copy(const WideCopy* copies, int count, int operand, hipStream_t s) {
  for (int base = 0; base < count; base += CP_MAX) {
    WideCopyBatch cb;
    cb.count = count - base < CP_MAX ? count - base : CP_MAX;
    int total = 0;
    for (int i = 0; i < cb.count; ++i) {
      const WideCopy& c = copies[base + i];
      cb.c[i] = c;
      cb.start[i] = total;
      total += ((c.rows + CP_T - 1) / CP_T) * ((c.cols + CP_T - 1) / CP_T);
    }
    for (int i = cb.count; i <= CP_MAX; ++i) cb.start[i] = total;
    if (total == 0) continue;
    if (operand == DT_F16)
      hipLaunchKernelGGL(wide_copy_kernel<f16>, dim3(total), dim3(256), 0, s, cb);
    else if (operand == DT_BF16)
      hipLaunchKernelGGL(wide_copy_kernel<bf16>, dim3(total), dim3(256), 0, s, cb);
    else
      return hipErrorInvalidValue;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ipc
