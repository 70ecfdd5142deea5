// ipc_wide.hip - the GEMM path of wide nets (gfx950): one launch per phase
// over all layers of the LDS-DMA MFMA kernel of ipc_dma_gemm.h with the fused
// epilogues that keep the fp32 masters and their 16-bit operand copies in
// step, plus the kernel that re-derives the copies from the masters.
#include "ipc_dma_gemm.h"

namespace ipc {
namespace {

using dma::Cfg;

// Tile configurations (BM, BN, stages, waves along M, waves along N) of each
// phase; index 0 is the default, the others are the alternatives a plan can
// select (ipc_plan_set_wide_config) after tuning.  The configurations of one
// phase give bit-identical results: every output element sums its
// contraction in the same k order whatever the tile.
//   split-1 prediction: 256 x 128 (3 stages, waves 4 x 2); 128 x 256 (3, 2 x 4)
//   split-2 prediction: 128 x 256 (2 stages, waves 2 x 4): 281 us per launch on the wide
//       configuration against 317 us for 128 x 128 (3 stages, 4 x 2), the alternative;
//       256 x 128 (2 stages) measured 349 us
//   inference and weight update: 256 x 256 (2 stages, 8 waves 2 x 4: 128 x 64 per wave),
//       finished from the registers (their fp32 tile exceeds the LDS): 170 and 268 us
//       against 199 and 298 us for 128 x 256 (3 stages, 16 waves 4 x 4, LDS-staged
//       epilogue), the previous defaults, in the same process; the wide step's main loops
//       read half the LDS bytes per MFMA on 128 x 64 wave tiles.  Alternatives: 128 x 256
//       with waves 4 x 4 or 2 x 4, 256 x 128 (3, 4 x 2) and, for the weight update,
//       128 x 128 (4 stages, 4 x 2)
#define WIDE_PRED1_CFGS(X) X(256, 128, 3, 4, 2) X(128, 256, 3, 2, 4)
#define WIDE_PRED2_CFGS(X) X(128, 256, 2, 2, 4) X(128, 128, 3, 4, 2)
// the split-2 prediction reading the fp32 W (a32): waves 4 x 2, so that each
// wave splits its 32-row A fragment for 4 column blocks (two waves share it);
// on 128 x 256 tiles the W block has three stages and the B block two
// (a32_extra_stage)
#define WIDE_PRED2A_CFGS(X) X(128, 256, 2, 4, 2) X(128, 128, 3, 4, 2)
#define WIDE_INFER_CFGS(X) X(256, 256, 2, 2, 4) X(128, 256, 3, 4, 4) X(128, 256, 3, 2, 4) X(256, 128, 3, 4, 2)
#define WIDE_WEIGHT_CFGS(X) \
  X(256, 256, 2, 2, 4) X(128, 256, 3, 4, 4) X(128, 256, 3, 2, 4) X(256, 128, 3, 4, 2) X(128, 128, 4, 4, 2)
#define IPC_COUNT1(...) +1
constexpr int kPred1Cfgs = 0 WIDE_PRED1_CFGS(IPC_COUNT1), kPred2Cfgs = 0 WIDE_PRED2_CFGS(IPC_COUNT1);
constexpr int kInferCfgs = 0 WIDE_INFER_CFGS(IPC_COUNT1), kWeightCfgs = 0 WIDE_WEIGHT_CFGS(IPC_COUNT1);
// the a32 list mirrors the split-2 one tile for tile (the plan sizes the
// k-split and the workspace from wide_pred_tile, which reads the latter)
#define IPC_TILE_CODE(BM_, BN_, S_, WM_, WN_) BM_ * 4096 + BN_,
constexpr int kPred2Tiles[] = {WIDE_PRED2_CFGS(IPC_TILE_CODE)};
constexpr int kPred2ATiles[] = {WIDE_PRED2A_CFGS(IPC_TILE_CODE)};
constexpr bool same_tiles() {
  for (int i = 0; i < kPred2Cfgs; ++i)
    if (kPred2Tiles[i] != kPred2ATiles[i]) return false;
  return true;
}
static_assert(sizeof(kPred2ATiles) == sizeof(kPred2Tiles) && same_tiles(),
              "one a32 configuration, of the same tile, per split-2 prediction one");

// forward initialisation: the split-1 prediction tiles; split 2 keeps 128 x 128
// (one layer per launch: its tiles fill all CUs once per 4096-row layer, 82 us
// per layer against 120 us on the prediction's 128 x 256 tiles; the sums per
// element do not depend on the tile, so the first prediction errors stay exactly 0)
template <typename OT, int ACT> using FwdCfg1 = Cfg<OT, WIDE_FWD, 1, ACT, false, 256, 128, 3, 4, 2>;
template <typename OT, int ACT, bool A32> using FwdCfg2 = Cfg<OT, WIDE_FWD, 2, ACT, false, 128, 128, 3, 4, 2, A32>;

// Launches (or prepares) configuration `cfg` of a list: the i-th X(...) entry.
#define IPC_CFG_CASE(MODE_, SPLIT_, ACT_, A32_, BM_, BN_, S_, WM_, WN_)                                   \
  if (cfg == i++) return prep ? Cfg<OT, MODE_, SPLIT_, ACT_, false, BM_, BN_, S_, WM_, WN_, A32_>::prepare()  \
                              : Cfg<OT, MODE_, SPLIT_, ACT_, false, BM_, BN_, S_, WM_, WN_, A32_>::launch(    \
                                    probs, count, s);
#define IPC_P1(BM_, BN_, S_, WM_, WN_) IPC_CFG_CASE(WIDE_PRED, 1, ACT_IDENTITY, false, BM_, BN_, S_, WM_, WN_)
#define IPC_P2(BM_, BN_, S_, WM_, WN_) IPC_CFG_CASE(WIDE_PRED, 2, ACT_IDENTITY, false, BM_, BN_, S_, WM_, WN_)
#define IPC_P2A(BM_, BN_, S_, WM_, WN_) IPC_CFG_CASE(WIDE_PRED, 2, ACT_IDENTITY, true, BM_, BN_, S_, WM_, WN_)
#define IPC_IN(BM_, BN_, S_, WM_, WN_) IPC_CFG_CASE(WIDE_INFER, 1, ACT, false, BM_, BN_, S_, WM_, WN_)
#define IPC_WT(BM_, BN_, S_, WM_, WN_) IPC_CFG_CASE(WIDE_WEIGHT, 1, ACT_IDENTITY, false, BM_, BN_, S_, WM_, WN_)

template <typename OT>
struct Phase {
  template <int ACT>
  struct Run {
    // prep: raise the LDS limit of configuration `cfg` instead of launching it;
    // a32: the split-2 prediction / forward read the fp32 W (problems' a) itself
    static hipError_t run(int mode, int split, int cfg, bool prep, const WideProblem* probs, int count,
                          hipStream_t s, bool a32) {
      int i = 0;
      switch (mode) {
        case WIDE_PRED:
          if (split == 2 && a32) { WIDE_PRED2A_CFGS(IPC_P2A) }
          else if (split == 2) { WIDE_PRED2_CFGS(IPC_P2) }
          else { WIDE_PRED1_CFGS(IPC_P1) }
          return hipErrorInvalidValue;
        case WIDE_INFER: { WIDE_INFER_CFGS(IPC_IN) } return hipErrorInvalidValue;
        case WIDE_WEIGHT: { WIDE_WEIGHT_CFGS(IPC_WT) } return hipErrorInvalidValue;
        default:  // WIDE_FWD
          if (split != 2) return prep ? FwdCfg1<OT, ACT>::prepare() : FwdCfg1<OT, ACT>::launch(probs, count, s);
          if (a32) return prep ? FwdCfg2<OT, ACT, true>::prepare() : FwdCfg2<OT, ACT, true>::launch(probs, count, s);
          return prep ? FwdCfg2<OT, ACT, false>::prepare() : FwdCfg2<OT, ACT, false>::launch(probs, count, s);
      }
    }
  };
  static hipError_t prepare() {
    hipError_t e;
    for (int act = 0; act < 6; ++act) {
      for (int c = 0; c < kInferCfgs; ++c)
        if ((e = dma::by_act<Run>(act, WIDE_INFER, 1, c, true, nullptr, 0, nullptr, false)) != hipSuccess) return e;
      for (int sp = 1; sp <= 2; ++sp)
        for (int a32 = 0; a32 <= (sp == 2 ? 1 : 0); ++a32)
          if ((e = dma::by_act<Run>(act, WIDE_FWD, sp, 0, true, nullptr, 0, nullptr, a32 != 0)) != hipSuccess)
            return e;
    }
    for (int c = 0; c < kPred1Cfgs; ++c)
      if ((e = Run<0>::run(WIDE_PRED, 1, c, true, nullptr, 0, nullptr, false)) != hipSuccess) return e;
    for (int c = 0; c < kPred2Cfgs; ++c)
      for (int a32 = 0; a32 <= 1; ++a32)
        if ((e = Run<0>::run(WIDE_PRED, 2, c, true, nullptr, 0, nullptr, a32 != 0)) != hipSuccess) return e;
    for (int c = 0; c < kWeightCfgs; ++c)
      if ((e = Run<0>::run(WIDE_WEIGHT, 1, c, true, nullptr, 0, nullptr, false)) != hipSuccess) return e;
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
      if (dst) dst[(long long)r * c.ldd + col] = hi;
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

// Epilogue of a k-split prediction, 64 x 64 block per workgroup: the slices'
// partial products are added in slice order, then eps = x - sum and its
// copies, with the rounding steps of the whole-tile prediction epilogue.  A
// thread owns 4 columns of 4 rows (16 rows apart); the loads of all four rows
// are issued before their sums, and the transposed copy goes through LDS so
// that each thread stores 4 consecutive rows of one column at once.
template <typename OT>
__global__ void __launch_bounds__(256) wide_reduce_kernel(const WideReduce r) {
  __shared__ float tile[CP_T][CP_T + 1];
  const int tc = (r.N + CP_T - 1) / CP_T;
  const int r0 = (blockIdx.x / tc) * CP_T, c0 = (blockIdx.x % tc) * CP_T;
  const int cq = (threadIdx.x & 15) * 4, ty = threadIdx.x >> 4;
  const int n = c0 + cq;
  const int nv = n < r.N ? (r.N - n < 4 ? r.N - n : 4) : 0;
  const bool vec = r.vec && nv == 4;
  OT* h = reinterpret_cast<OT*>(r.h);
  float a[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int m = r0 + u * 16 + ty;
#pragma unroll
    for (int j = 0; j < 4; ++j) a[u][j] = 0.0f;
    if (m >= r.M || nv == 0) continue;
    const float* src = r.part + (long long)m * r.ldp + n;
    if (vec) {
      const float4 t = *reinterpret_cast<const float4*>(src);
      a[u][0] = t.x; a[u][1] = t.y; a[u][2] = t.z; a[u][3] = t.w;
    } else {
      for (int j = 0; j < nv; ++j) a[u][j] = src[j];
    }
  }
#pragma unroll 2
  for (int q = 1; q < r.slices; ++q) {
    float b[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int m = r0 + u * 16 + ty;
#pragma unroll
      for (int j = 0; j < 4; ++j) b[u][j] = 0.0f;
      if (m >= r.M || nv == 0) continue;
      const float* src = r.part + q * r.part_stride + (long long)m * r.ldp + n;
      if (vec) {
        const float4 t = *reinterpret_cast<const float4*>(src);
        b[u][0] = t.x; b[u][1] = t.y; b[u][2] = t.z; b[u][3] = t.w;
      } else {
        for (int j = 0; j < nv; ++j) b[u][j] = src[j];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) a[u][j] = a[u][j] + b[u][j];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int rr = u * 16 + ty, m = r0 + rr;
    float hv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m < r.M && nv > 0) {
#pragma clang fp contract(off)
      const float* xs = r.x + (long long)m * r.ldx + n;
      float* es = r.eps + (long long)m * r.lde + n;
      OT* hs = h + (long long)m * r.ldh + n;
      float v[4];
      OT o[4];
      if (vec) {
        const float4 t = *reinterpret_cast<const float4*>(xs);
        v[0] = t.x - a[u][0]; v[1] = t.y - a[u][1]; v[2] = t.z - a[u][2]; v[3] = t.w - a[u][3];
        *reinterpret_cast<float4*>(es) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = cvt<OT>(v[j]);
        uint2 pk;
        pk.x = dma::pack2(o[0], o[1]);
        pk.y = dma::pack2(o[2], o[3]);
        *reinterpret_cast<uint2*>(hs) = pk;
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = to_f32(o[j]);
      } else {
        for (int j = 0; j < nv; ++j) {
          v[j] = xs[j] - a[u][j];
          es[j] = v[j];
          o[j] = cvt<OT>(v[j]);
          hs[j] = o[j];
          hv[j] = to_f32(o[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[rr][cq + j] = hv[j];
  }
  if (!r.t) return;
  __syncthreads();
  OT* t = reinterpret_cast<OT*>(r.t);
  // 64 columns x 16 groups of 4 rows: one 8-byte store of 4 consecutive rows
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = it * 256 + threadIdx.x;
    const int cc = idx >> 4, mg = (idx & 15) * 4;
    const int nn = c0 + cc, m = r0 + mg;
    if (nn >= r.N || m >= r.M) continue;
    OT* dst = t + (long long)nn * r.ldt + m;
    if (m + 4 <= r.M) {
      uint2 pk;
      pk.x = dma::pack2(cvt<OT>(tile[mg][cc]), cvt<OT>(tile[mg + 1][cc]));
      pk.y = dma::pack2(cvt<OT>(tile[mg + 2][cc]), cvt<OT>(tile[mg + 3][cc]));
      *reinterpret_cast<uint2*>(dst) = pk;
    } else {
      for (int j = 0; m + j < r.M; ++j) dst[j] = cvt<OT>(tile[mg + j][cc]);
    }
  }
}

template <typename OT>
hipError_t launch_phase(int mode, const WideProblem* probs, int count, int split, int act, int cfg, hipStream_t s,
                        bool a32) {
  return dma::by_act<Phase<OT>::template Run>(act, mode, split, cfg, false, probs, count, s, a32);
}

}  // namespace

hipError_t wide_prepare() {
  hipError_t e = Phase<f16>::prepare();
  if (e != hipSuccess) return e;
  return Phase<bf16>::prepare();
}

hipError_t launch_wide(int mode, const WideProblem* probs, int count, int operand, int split, int act,
                       hipStream_t s, int cfg, bool a32) {
  if (cfg < 0 || cfg >= wide_config_count(mode, split)) return hipErrorInvalidValue;
  if (a32 && (split != 2 || (mode != WIDE_PRED && mode != WIDE_FWD))) return hipErrorInvalidValue;
  for (int base = 0; base < count; base += WIDE_MAX_BATCH) {
    const int n = count - base < WIDE_MAX_BATCH ? count - base : WIDE_MAX_BATCH;
    hipError_t e;
    if (operand == DT_F16) e = launch_phase<f16>(mode, probs + base, n, split, act, cfg, s, a32);
    else if (operand == DT_BF16) e = launch_phase<bf16>(mode, probs + base, n, split, act, cfg, s, a32);
    else return hipErrorInvalidValue;
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool wide_problem_ok(int mode, int split, bool a32, const WideProblem& q) {
  return dma::problem_ok(mode, split, a32, q);
}

hipError_t launch_wide_reduce(const WideReduce& r, int operand, hipStream_t s) {
  if (r.slices < 1 || r.M <= 0 || r.N <= 0) return hipErrorInvalidValue;
  const dim3 grid(((r.M + CP_T - 1) / CP_T) * ((r.N + CP_T - 1) / CP_T));
  if (operand == DT_F16)
    hipLaunchKernelGGL(wide_reduce_kernel<f16>, grid, dim3(256), 0, s, r);
  else if (operand == DT_BF16)
    hipLaunchKernelGGL(wide_reduce_kernel<bf16>, grid, dim3(256), 0, s, r);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

int wide_config_count(int mode, int split) {
  switch (mode) {
    case WIDE_PRED: return split == 2 ? kPred2Cfgs : kPred1Cfgs;
    case WIDE_INFER: return kInferCfgs;
    case WIDE_WEIGHT: return kWeightCfgs;
    default: return 1;
  }
}

#define IPC_TILE_XY(BM_, BN_, S_, WM_, WN_) if (cfg == i++) { *bm = BM_; *bn = BN_; return; }
void wide_pred_tile(int split, int cfg, int* bm, int* bn) {
  int i = 0;
  if (split == 2) { WIDE_PRED2_CFGS(IPC_TILE_XY) }
  else { WIDE_PRED1_CFGS(IPC_TILE_XY) }
  *bm = *bn = 0;
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
