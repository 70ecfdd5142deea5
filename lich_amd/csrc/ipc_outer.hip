// ipc_outer.hip - rank-B outer-product weight update for small batches (gfx950).
//
//   W[m][k] += alpha * sum_{b<B} E[m][b] * f(X[k][b])        (B <= 32)
//
// Replaces SmallBWeightUpdater (src/ipc_tilelang/weight_update_specialization.py:63-128),
// which formed a [B,M,K] temporary with torch.bmm and reduced it; here the
// sum is formed in registers and W is streamed once (read + write), so the
// kernel is bound by HBM traffic on W.  The sign is +alpha as in the GEMM
// weight update and reference.py:57.
//
// A workgroup owns OUTER_RM rows x OUTER_TK columns of W.  The rows
// X[k0 .. k0+OUTER_TK) form one contiguous chunk of OUTER_TK*B elements and are
// staged through LDS with coalesced loads (activation applied once per
// element); the E rows are staged the same way.  Each thread then owns one
// column and reads/writes W[m][k] coalesced across the wave.
#include "ipc_device.h"
#include "ipc_launch.h"

namespace ipc {

constexpr int OUTER_TK = 256;
constexpr int OUTER_RM = 8;
constexpr int OUTER_MAXB = 32;

template <typename ST>
__global__ void __launch_bounds__(OUTER_TK) outer_kernel(const OuterProblem p) {
  __shared__ float xs[OUTER_TK * (OUTER_MAXB + 1)];
  __shared__ float es[OUTER_RM * OUTER_MAXB];
  const int B = p.B, K = p.K, M = p.M;
  const int g = blockIdx.z;
  const int k0 = blockIdx.x * OUTER_TK, m0 = blockIdx.y * OUTER_RM;
  const ST* X = reinterpret_cast<const ST*>(p.x) + (long long)g * p.x_gs;
  const ST* E = reinterpret_cast<const ST*>(p.e) + (long long)g * p.e_gs;
  ST* W = reinterpret_cast<ST*>(p.w) + (long long)g * p.w_gs;
  const int tid = threadIdx.x;

  const int kn = min(OUTER_TK, K - k0);
  const int xcount = kn * B;
  const ST* xchunk = X + (long long)k0 * B;
  for (int i = tid; i < xcount; i += OUTER_TK) {
    const int r = i / B, b = i - r * B;
    xs[r * (OUTER_MAXB + 1) + b] = act_f(p.act, to_f32(xchunk[i]));
  }
  const int mn = min(OUTER_RM, M - m0);
  const ST* echunk = E + (long long)m0 * B;
  for (int i = tid; i < mn * B; i += OUTER_TK) es[i] = to_f32(echunk[i]);
  __syncthreads();

  if (tid < kn) {
    const int k = k0 + tid;
    float acc[OUTER_RM];
#pragma unroll
    for (int r = 0; r < OUTER_RM; ++r) acc[r] = 0.0f;
    for (int b = 0; b < B; ++b) {
      const float xv = xs[tid * (OUTER_MAXB + 1) + b];
#pragma unroll
      for (int r = 0; r < OUTER_RM; ++r) acc[r] += es[r * B + b] * xv;
    }
#pragma unroll
    for (int r = 0; r < OUTER_RM; ++r) {
      if (r < mn) {
        // W + (alpha * acc), each rounded, as the fp32 reference does.
#pragma clang fp contract(off)
        const long long o = (long long)(m0 + r) * K + k;
        W[o] = cvt<ST>(to_f32(W[o]) + p.alpha * acc[r]);
      }
    }
  }
}

// Elementwise activation, used once per batch for the saved input activation
// a[L] = f(x[L]) (trainer.py:510-511).
template <typename ST>
__global__ void __launch_bounds__(256) act_kernel(const ST* src, ST* dst, long long n, int act) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    dst[i] = cvt<ST>(act_f(act, to_f32(src[i])));
}

hipError_t launch_act(const void* src, void* dst, long long n, int act, int storage, hipStream_t s) {
  const long long want = (n + 255) / 256;
  const int blocks = (int)(want < 4096 ? (want < 1 ? 1 : want) : 4096);
  if (storage == DT_F32)
    hipLaunchKernelGGL(act_kernel<float>, dim3(blocks), dim3(256), 0, s, (const float*)src, (float*)dst, n, act);
  else if (storage == DT_F16)
    hipLaunchKernelGGL(act_kernel<f16>, dim3(blocks), dim3(256), 0, s, (const f16*)src, (f16*)dst, n, act);
  else
    hipLaunchKernelGGL(act_kernel<bf16>, dim3(blocks), dim3(256), 0, s, (const bf16*)src, (bf16*)dst, n, act);
  return hipGetLastError();
}

hipError_t launch_outer(const OuterProblem& p, int storage, hipStream_t s) {
  dim3 grid((p.K + OUTER_TK - 1) / OUTER_TK, (p.M + OUTER_RM - 1) / OUTER_RM, p.groups);
  dim3 block(OUTER_TK);
  if (storage == DT_F32) hipLaunchKernelGGL(outer_kernel<float>, grid, block, 0, s, p);
  else if (storage == DT_F16) hipLaunchKernelGGL(outer_kernel<f16>, grid, block, 0, s, p);
  else hipLaunchKernelGGL(outer_kernel<bf16>, grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace ipc
