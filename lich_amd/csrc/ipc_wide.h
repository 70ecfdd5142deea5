// ipc_wide.h - host interface of the GEMM path for wide nets (gfx950).
//
// Wide layers (hundreds to thousands of units, batch in the hundreds or
// more) are MFMA-bound.  This path keeps the fp32 masters x, eps and W of the
// plan and, next to them, 16-bit operand copies laid out k-contiguous for
// every GEMM that reads them, so each GEMM streams both operands straight
// from HBM into LDS (global_load_lds) with no conversion, transpose or
// activation in its loaders:
//
//   pred   eps[l] = x[l] - W[l] f(x[l+1])       A = Wh[l] (+ Wl[l])  [d_l][d_{l+1}]
//                                               B = FT[l+1]          [B][d_{l+1}]
//   infer  x[l] += g(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1])
//                                               A = WT[l-1]          [d_l][d_{l-1}]
//                                               B = ET[l-1]          [B][d_{l-1}]
//   weight W[l] += a eps[l] f(x[l+1])^T         A = E[l]             [d_l][B]
//                                               B = F[l+1]           [d_{l+1}][B]
//
// Each epilogue writes the copies that later GEMMs read: pred writes E and
// ET, infer writes F and FT of the updated states, weight writes Wh, Wl
// (W - Wh, the error-compensation term) and WT.  The forward initialisation
// x[l] = W[l] f(x[l+1]) (one layer per launch, l = L-1 .. 1) is the pred GEMM
// with an epilogue that writes x[l], F[l] and FT[l], so that the first step's
// prediction reproduces it exactly.  Every copy has its rows
// padded to WIDE_ROW_PAD and its k extent to WIDE_BK with zeros, which the
// kernel relies on: its main loop has no bounds checks.
#pragma once

#include <hip/hip_runtime.h>

namespace ipc {

constexpr int WIDE_BK = 64;         // k per pipeline stage (16-bit elements, 128-byte rows)
constexpr int WIDE_ROW_PAD = 256;   // row padding of every operand copy (largest tile edge)
constexpr int WIDE_MAX_BATCH = 16;  // layers per launch

enum { WIDE_PRED = 0, WIDE_INFER = 1, WIDE_WEIGHT = 2, WIDE_FWD = 3 };

inline long long wide_pad(long long v, long long m) { return (v + m - 1) / m * m; }

// One layer's GEMM C[M][N] = sum_k A[m][k] B[n][k] with its fused epilogue.
// K is a multiple of WIDE_BK; A (and A_lo) hold >= wide_pad(M, 256) rows and
// B >= wide_pad(N, 256) rows, zero beyond M / N / the true contraction.
struct WideProblem {
  int M, N, K;
  const void* a; const void* a_lo; long long lda;  // a_lo: split-2 term (pred) or nullptr
  const void* b; long long ldb;
  float* out; long long ldo;        // pred: eps[l], fwd: x[l] (written); infer: x[l], weight: W[l] (updated)
  const float* aux; long long ldx;  // pred: x[l], infer: eps[l]
  void* h; long long ldh;           // 16-bit copy [M][ldh]: pred E, infer/fwd F, weight Wh
  void* hl; long long ldhl;         // weight: Wl [M][ldhl]
  void* t; long long ldt;           // 16-bit transposed copy [N][ldt]: pred ET, infer/fwd FT, weight WT; may be null
  float* out2; long long ld2;       // infer, save mode: f(x_new) fp32 [M][ld2], or null
  float scal;                       // infer: gamma, weight: alpha
  int vec;                          // 1: out/aux/out2 rows 16-byte aligned, h/hl rows 8-byte aligned
};

struct WideBatch {
  WideProblem p[WIDE_MAX_BATCH];
  int start[WIDE_MAX_BATCH + 1];  // first tile of each problem
  int count, act;
};

// Tile edge (rows of A, rows of B) the launch of `mode` uses.
void wide_tile(int mode, int split, int* bm, int* bn);

// Launches one phase over `count` layers (one launch per WIDE_MAX_BATCH layers).
// `operand` is DT_F16 or DT_BF16, `split` 1 or 2 (pred and fwd).
hipError_t launch_wide(int mode, const WideProblem* probs, int count, int operand, int split, int act,
                       hipStream_t s);

// Raises the dynamic-LDS limit of every wide kernel instantiation.
hipError_t wide_prepare();

// Refresh of the 16-bit copies from the fp32 masters (after the masters were
// written outside a step):
//   dst[r][c] = cvt(f(src[r][c]))      (and dst_lo = cvt(v - hi) when given)
//   dst_t[c][r] = the same hi value    (when given)
// for r < rows, c < cols; f is the activation `act` (ACT_IDENTITY for W).
struct WideCopy {
  const float* src; long long lds;
  int rows, cols, act;
  void* dst; long long ldd;
  void* dst_lo; long long ldl;
  void* dst_t; long long ldt;
};
hipError_t launch_wide_copy(const WideCopy* copies, int count, int operand, hipStream_t s);

}  // namespace ipc
