// ipc_wide.h - host interface of the LDS-DMA MFMA GEMM family (gfx950).
//
// One kernel template (ipc_dma_gemm.h) serves two callers:
//
// * the GEMM path of wide nets (modes WIDE_*): the plan keeps the fp32
//   masters x, eps and W and, next to them, 16-bit operand copies of W, f(x)
//   and eps that the GEMMs stream straight from HBM into LDS
//   (global_load_lds, no VGPR staging), and fused epilogues that update the
//   masters and rewrite the copies:
//
//     pred   eps[l] = x[l] - W[l] f(x[l+1])    A = Wh[l] (+ Wl[l])  [d_l][d_{l+1}]
//                                              B = FT[l+1]           [B][d_{l+1}]
//     infer  x[l] += g(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1])
//                                              A = WT[l-1]           [d_l][d_{l-1}]
//                                              B = ET[l-1]           [B][d_{l-1}]
//     weight W[l] += a eps[l] f(x[l+1])^T      A = E[l]              [d_l][B]
//                                              B = F[l+1]            [d_{l+1}][B]
//
//   Every copy is k-contiguous for the GEMM that reads it, so all fragment
//   reads are plain 16-byte LDS reads (measured faster here than reading a
//   copy transposed with ds_read_b64_tr_b16, whose 8-byte reads need twice
//   the LDS instructions, even after paying the weight epilogue's extra W^T
//   write).  pred writes eps, E and ET, infer x, F and FT, weight W, Wh, Wl
//   (W - Wh, the error-compensation term of split 2) and WT; the forward
//   initialisation x[l] = W[l] f(x[l+1]) (one layer per launch, l = L-1 .. 1)
//   is the pred GEMM with an epilogue that writes x[l], F[l] and FT[l].
//   Every copy has its rows and columns padded to WIDE_PAD with zeros, which
//   the main loop relies on (it has no k bounds checks).
//
// * the standalone kernels of the operator API with 16-bit storage (modes
//   S16_*; src/ipc_tilelang/tilelang_kernels.py:114-349 semantics, rounding as
//   there): operands are the caller's tensors, k contiguous or not as above
//   (S16_WEIGHT's B is X_upper [K][B] read as [n][k]); operands whose
//   contraction index is not the contiguous one (W_lower, X_upper and E_lower
//   of pred / infer) are read from LDS with gfx950's transposing LDS read
//   (ds_read_b64_tr_b16); f(X_upper) goes through registers (global load,
//   activation, LDS store) instead of the DMA.
#pragma once

#include <hip/hip_runtime.h>

namespace ipc {

constexpr int WIDE_BK = 64;         // k per pipeline stage (16-bit elements, 128-byte rows)
constexpr int WIDE_PAD = 64;        // row and column padding of every operand copy
constexpr int WIDE_MAX_BATCH = 16;  // problems per launch

enum {
  WIDE_PRED = 0, WIDE_INFER = 1, WIDE_WEIGHT = 2, WIDE_FWD = 3,
  S16_PRED = 4, S16_FWD = 5, S16_INFER = 6, S16_WEIGHT = 7,
  // S16_PRED / S16_FWD whose B operand is f(X_upper)^T [N][K] (k-contiguous,
  // ldb = K): the copy a caller workspace holds after launch_s16_activate_t
  S16_PREDT = 8, S16_FWDT = 9,
  // S16_INFER reading W_lower^T [M][K] and E_lower^T [B][K] (both
  // k-contiguous, lda = ldb = K): the transposed copies of a caller workspace
  S16_INFERT = 10,
};

inline long long wide_pad(long long v, long long m) { return (v + m - 1) / m * m; }

// One GEMM C[M][N] = sum_k A(m, k) B(n, k) with its fused epilogue.
// K is a multiple of WIDE_BK and every operand element with k < K is
// readable (zero beyond the true contraction).  a_lim / b_lim bound the
// other index of each operand: the rows that may be read of a k-contiguous
// operand, the columns (a multiple of 8, <= its ld) of an m/n-contiguous one;
// tiles that reach past M or N clamp their loads there and mask their stores.
struct WideProblem {
  int M, N, K;
  const void* a; const void* a_lo; long long lda; int a_lim;  // a_lo: split-2 term (pred) or nullptr;
                                                              // a fp32 (a_lo unused) in launch_wide's a32 mode
  const void* b; long long ldb; int b_lim;
  void* out; long long ldo;        // WIDE: pred eps[l], fwd x[l] (written); infer x[l], weight W[l] (updated), fp32
                                   // S16:  pred E, fwd OUT (written); infer X, weight W (updated), 16-bit
  const void* aux; long long ldx;  // WIDE pred: x[l], infer: eps[l] (fp32); S16 pred: X_lower, infer: E (16-bit)
  void* h; long long ldh;          // WIDE: 16-bit copy [M][ldh]: pred E, infer/fwd F, weight Wh (or null)
  void* hl; long long ldhl;        // WIDE weight: Wl [M][ldhl]
  void* t; long long ldt;          // WIDE: transposed 16-bit copy [N][ldt] (pred ET, infer/fwd FT, weight WT), or null
  void* out2; long long ld2;       // infer, save mode: f(x_new) (fp32 for WIDE, 16-bit for S16), or null
  float scal;                      // infer: gamma, weight: alpha
  int vec;                         // 1: out/aux/out2 rows allow 4-element vector access, h/hl rows 8-byte aligned
  // WIDE_PRED only: ksplit > 1 cuts the contraction into ksplit equal slices
  // (K / ksplit a multiple of WIDE_BK); slice s stores its raw fp32 partial
  // product at out + s * part_stride ([M][ldo]) and nothing else, and
  // launch_wide_reduce finishes the epilogue.  Split problems come last in a
  // launch: their tiles are dispatched after every whole tile, so they fill
  // the launch's last round of CUs.
  int ksplit;
  long long part_stride;
};

// The epilogue of a k-split prediction: eps = x - sum of the slices (added in
// slice order), written with its 16-bit copy E and transposed copy ET.
struct WideReduce {
  const float* part; long long part_stride; long long ldp;
  int slices, M, N;
  const float* x; long long ldx;
  float* eps; long long lde;
  void* h; long long ldh;
  void* t; long long ldt;
  int vec;  // 1: part, x and eps rows allow 4-element vector access
};
hipError_t launch_wide_reduce(const WideReduce& r, int operand, hipStream_t s);

// Tile configurations a phase offers (WIDE_PRED with split 1 or 2,
// WIDE_INFER, WIDE_WEIGHT; 1 for WIDE_FWD); configuration 0 is the default.
int wide_config_count(int mode, int split);

// Output tile of prediction configuration `cfg` for `split` (1 or 2).
void wide_pred_tile(int split, int cfg, int* bm, int* bn);

// Launches one phase of the wide path over `count` layers (one launch per
// WIDE_MAX_BATCH layers) on tile configuration `cfg`.  `operand` is DT_F16
// or DT_BF16, `split` 1 or 2 (pred and fwd), `act` the activation of the
// infer / fwd epilogues.  `a32` (split-2 pred and fwd): each problem's `a`
// is the fp32 W itself (a_lo unused, K a multiple of WIDE_BK, rows 16-byte
// aligned), split into its hi and lo operands as the kernel reads it.
hipError_t launch_wide(int mode, const WideProblem* probs, int count, int operand, int split, int act,
                       hipStream_t s, int cfg = 0, bool a32 = false);

// The host-side check every LDS-DMA launch makes of each problem before any
// HIP call (mode WIDE_PRED / _INFER / _WEIGHT / _FWD or an S16_* mode).
bool wide_problem_ok(int mode, int split, bool a32, const WideProblem& q);

// Raises the dynamic-LDS limit of every wide-path kernel instantiation.
hipError_t wide_prepare();

// Standalone 16-bit-storage launches (modes S16_*) over `count` problems.
// `act`: the loader activation of S16_PRED / S16_FWD / S16_WEIGHT (ACT_IDENTITY
// for a saved activation), the epilogue activation of S16_INFER.
hipError_t launch_s16(int mode, const WideProblem* probs, int count, int operand, int act, int cfg, hipStream_t s);
// out[i] = cvt(f(in[i])) over n 16-bit elements: the B operand of a standalone
// S16_PRED / S16_FWD / recomputing S16_WEIGHT call evaluated once, so that the
// call then runs with ACT_IDENTITY on the LDS-DMA path for that operand.
hipError_t launch_s16_activate(const void* in, void* out, long long n, int operand, int act, hipStream_t s);
// The same values transposed: out[g][b][k] = cvt(f(in[g][k][b])) for `groups`
// [K][B] operands gstride elements apart (the copies gstride apart as well):
// the B operand of S16_PREDT / S16_FWDT.
hipError_t launch_s16_activate_t(const void* in, void* out, int K, int B, int groups, long long gstride,
                                 int operand, int act, hipStream_t s);

// Refresh of the 16-bit copies from the fp32 masters (after the masters were
// written outside a step):
//   dst[r][c] = cvt(f(src[r][c]))      (when given; dst_lo = cvt(v - hi) when given)
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
