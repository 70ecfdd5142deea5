// ipc_wide.hip - MFMA GEMM path for wide nets (gfx950): one launch per phase
// over all layers, fused epilogues, multi-stage LDS-DMA pipeline.
//
// Kernel structure (one workgroup = 4 waves = one BM x BN output tile):
//   * operands are 16-bit, row-major with k contiguous, zero padded (rows to
//     WIDE_ROW_PAD, k to WIDE_BK), so the main loop has no bounds checks;
//   * each k-step of 64 is moved HBM -> LDS by global_load_lds_dwordx4 (no
//     VGPR staging), S stages deep; 8 rows x 128 bytes per wave instruction,
//     16-byte chunk c of row r placed at chunk c ^ ((r >> 1) & 7).  The LDS
//     has 64 banks (256 bytes per bank row, two tile rows): a 16-byte read
//     by 16 lanes of 16 consecutive rows then touches all 64 banks once;
//   * one barrier per k-step: a wave waits for its own loads of the step it
//     is about to read (s_waitcnt vmcnt), the barrier publishes everybody's,
//     then the wave refills the stage everybody finished with;
//   * each wave owns (BM/2) x (BN/2) of the tile as 32x32 fp32 MFMA blocks
//     (v_mfma_f32_32x32x16_{f16,bf16}); split 2 adds the A_lo.B products;
//   * workgroups are renumbered so that the tiles one XCD runs are
//     consecutive (the tiles that share rows of A share that XCD's L2).
//
// Epilogues (reference: src/ipc_tilelang/tilelang_kernels.py:173 prediction
// error, :227-231 inference update, :319-320 weight update; the fp32
// rounding sequence is that of src/ipc_tilelang/reference.py:49-57, every
// operation rounded on its own).
#include "ipc_device.h"
#include "ipc_launch.h"
#include "ipc_wide.h"

namespace ipc {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the fence of __syncthreads: that fence makes the
// compiler wait for every outstanding LDS-DMA load, which would reduce the
// pipeline to one stage.  Each wave waits for its own loads before it.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Rows r0 .. r0+7 (r0 a multiple of 8), k columns k0 .. k0+63 of a row-major
// 16-bit matrix into 1024 contiguous LDS bytes: lane l writes chunk position
// l & 7 of row r0 + l / 8, so it fetches the global chunk that the swizzle
// puts there.
__device__ __forceinline__ int chunk_swizzle(int row) { return (row >> 1) & 7; }

template <typename OT>
__device__ __forceinline__ void dma_rows8(const OT* g, long long ld, int r0, int k0, unsigned char* lds,
                                          int lane) {
  const int r = r0 + (lane >> 3);
  const int c = (lane & 7) ^ chunk_swizzle(r);
  const OT* src = g + (long long)r * ld + k0 + c * 8;
  __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)lds, 16, 0, 0);
}

template <typename OT>
__device__ __forceinline__ unsigned pack2(OT a, OT b) {
  return (unsigned)__builtin_bit_cast(unsigned short, a) | ((unsigned)__builtin_bit_cast(unsigned short, b) << 16);
}

// Dynamic LDS of a configuration: the pipeline stages, reused by the fp32
// epilogue tile (BM rows of BN + 1 floats).
constexpr int wide_smem(int BM, int BN, int S, bool LO) {
  return S * (BM * 128 * (LO ? 2 : 1) + BN * 128) > BM * (BN + 1) * 4 ? S * (BM * 128 * (LO ? 2 : 1) + BN * 128)
                                                                     : BM * (BN + 1) * 4;
}

template <int BM, int BN, bool LO, int NW>
struct WideGeom {
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int STAGE = A_BYTES * (LO ? 2 : 1) + B_BYTES;
  static constexpr int QA = BM / (8 * NW), QB = BN / (8 * NW);  // 8-row groups per wave
  static constexpr int LPS = QA * (LO ? 2 : 1) + QB;            // DMA instructions per wave per stage
};

// WGM x WGN waves per workgroup, each owning (BM/WGM) x (BN/WGN) of the tile.
// ACT: activation of the infer / fwd epilogue (compile time; ACT_IDENTITY
// for pred and weight, whose epilogues apply none).
template <typename OT, int MODE, int SPLIT, int BM, int BN, int S, int WGM, int WGN, int ACT>
__global__ void __launch_bounds__(WGM * WGN * 64) wide_kernel(const WideBatch bt) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr bool LO = SPLIT == 2;
  constexpr int NW = WGM * WGN, NT = NW * 64;
  using Geo = WideGeom<BM, BN, LO, NW>;
  static_assert(Geo::QA * 8 * NW == BM && Geo::QB * 8 * NW == BN, "DMA row groups");
  constexpr int WTM = BM / WGM, WTN = BN / WGN, RM = WTM / 32, RN = WTN / 32;
  using MF = Mfma32<OT>;
  typedef typename MF::operand V;
  static_assert(S >= 2 && BM % 32 == 0 && BN % 64 == 0 && BM <= WIDE_ROW_PAD && BN <= WIDE_ROW_PAD, "tile");

  // XCD-aware renumbering: workgroup b runs on XCD b % 8; give every XCD a
  // contiguous range of tiles.
  const int G = gridDim.x, b = blockIdx.x;
  const int xcd = b & 7, per = G >> 3, rem = G & 7;
  const int tile = xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
  int pi = 0;
#pragma unroll 1
  while (pi + 1 < bt.count && tile >= bt.start[pi + 1]) ++pi;
  const WideProblem& p = bt.p[pi];
  const int tn = (p.N + BN - 1) / BN;
  const int local = tile - bt.start[pi];
  const int m0 = (local / tn) * BM, n0 = (local % tn) * BN;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w / WGN, wn = w % WGN;
  const OT* A = reinterpret_cast<const OT*>(p.a);
  const OT* Al = reinterpret_cast<const OT*>(p.a_lo);
  const OT* Bm = reinterpret_cast<const OT*>(p.b);
  const long long lda = p.lda, ldb = p.ldb;
  const int nk = p.K / WIDE_BK;

  auto issue = [&](int kt, int stage) {
    unsigned char* st = smem + stage * Geo::STAGE;
    const int k0 = kt * WIDE_BK;
#pragma unroll
    for (int q = 0; q < Geo::QA; ++q) {
      const int g = q * NW + w;
      dma_rows8(A, lda, m0 + g * 8, k0, st + g * 1024, lane);
      if (LO) dma_rows8(Al, lda, m0 + g * 8, k0, st + Geo::A_BYTES + g * 1024, lane);
    }
#pragma unroll
    for (int q = 0; q < Geo::QB; ++q) {
      const int g = q * NW + w;
      dma_rows8(Bm, ldb, n0 + g * 8, k0, st + Geo::A_BYTES * (LO ? 2 : 1) + g * 1024, lane);
    }
  };

  // The epilogue's fp32 input (x for pred/infer, W for weight) is fetched
  // now, ahead of the main loop, in the row-major 4-column groups pass 1 of
  // the epilogue walks: its latency hides behind the MFMAs and the epilogue
  // only issues stores.
  constexpr int IT = BM * BN / 4 / NT, CH = IT < 8 ? IT : 8;
  static_assert(IT % CH == 0, "epilogue chunking");
  const int M = p.M, N = p.N;
  const bool vec = p.vec != 0;
  auto load_group = [&](const float* base, long long ld, int u, float (&o)[4]) {
    const int idx = u * NT + tid;
    const int r = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
    const int m = m0 + r, n = n0 + c;
    const int nv = (m < M && n < N) ? (N - n < 4 ? N - n : 4) : 0;
    const float* src = base + (long long)m * ld + n;
    if (vec && nv == 4) {
      const float4 t4 = *reinterpret_cast<const float4*>(src);
      o[0] = t4.x; o[1] = t4.y; o[2] = t4.z; o[3] = t4.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = q < nv ? src[q] : 0.0f;
    }
  };
  float pre[IT][4];
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    if (MODE == WIDE_FWD) {
      pre[u][0] = pre[u][1] = pre[u][2] = pre[u][3] = 0.0f;  // the forward reads no fp32 input
    } else {
      load_group(MODE == WIDE_PRED ? p.aux : p.out, MODE == WIDE_PRED ? p.ldx : p.ldo, u, pre[u]);
    }
  }

  f32x16 acc[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s, s);

  // every row an operand read touches is (multiple of 16) + lr
  const int lr = lane & 31, lk = lane >> 5, sw = chunk_swizzle(lr);
  int stage = 0, fill = S - 1;
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    // this wave's loads of step kt are done once at most S-2 later steps are in flight
    if (kt + S - 2 < nk) wait_vmcnt<(S - 2) * Geo::LPS>();
    else wait_vmcnt<0>();
    wg_barrier();
    if (kt + S - 1 < nk) issue(kt + S - 1, fill);
    fill = fill + 1 == S ? 0 : fill + 1;

    const unsigned char* st = smem + stage * Geo::STAGE;
    const unsigned char* sa = st + (wm * WTM + lr) * 128;
    const unsigned char* sb = st + Geo::A_BYTES * (LO ? 2 : 1) + (wn * WTN + lr) * 128;
#pragma unroll
    for (int kk = 0; kk < WIDE_BK / 16; ++kk) {
      const int pos = ((kk * 2 + lk) ^ sw) * 16;
      V af[RM], bf[RN];
#pragma unroll
      for (int i = 0; i < RM; ++i) af[i] = *reinterpret_cast<const V*>(sa + i * 32 * 128 + pos);
#pragma unroll
      for (int j = 0; j < RN; ++j) bf[j] = *reinterpret_cast<const V*>(sb + j * 32 * 128 + pos);
#pragma unroll
      for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(af[i], bf[j], acc[i][j]);
      if (LO) {
#pragma unroll
        for (int i = 0; i < RM; ++i) {
          const V al = *reinterpret_cast<const V*>(sa + Geo::A_BYTES + i * 32 * 128 + pos);
#pragma unroll
          for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(al, bf[j], acc[i][j]);
        }
      }
    }
    stage = stage + 1 == S ? 0 : stage + 1;
  }

  // ------------------------------------------------------------ epilogue
  // The accumulator tile goes through LDS (the pipeline stages are free now)
  // so that every global access of the epilogue is coalesced: pass 1 walks
  // the tile row-major, 4 columns per thread (fp32 master, natural 16-bit
  // copy), pass 2 column-major (transposed 16-bit copy).
  constexpr int CS = BN + 1;  // fp32 row stride: conflict-free column walk in pass 2
  static_assert(BM * CS * 4 <= wide_smem(BM, BN, S, LO), "epilogue tile exceeds the LDS");
  float* cs = reinterpret_cast<float*>(smem);
  wait_vmcnt<0>();
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q)
        cs[(wm * WTM + i * 32 + 8 * (q >> 2) + 4 * lk + (q & 3)) * CS + wn * WTN + j * 32 + lr] = acc[i][j][q];
  __syncthreads();

  OT* hcopy = reinterpret_cast<OT*>(p.h);
  // Pass 1: IT groups of 4 columns per thread (inputs prefetched in pre[]).
#pragma unroll
  for (int c0 = 0; c0 < IT; c0 += CH) {
    float ein[CH][4];
    if (MODE == WIDE_INFER) {
#pragma unroll
      for (int u = 0; u < CH; ++u) load_group(p.aux, p.ldx, c0 + u, ein[u]);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int idx = (c0 + u) * NT + tid;
      const int r = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
      const int m = m0 + r, n = n0 + c;
      if (m >= M || n >= N) continue;
      const int nv = N - n < 4 ? N - n : 4;
      float* cr = cs + r * CS + c;
      float v[4], fv[4];
      OT hv[4], lv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
        const float acc_v = cr[q];
        const float x = pre[c0 + u][q];
        if (MODE == WIDE_PRED) {
          v[q] = x - acc_v;                                          // eps
          hv[q] = cvt<OT>(v[q]);
        } else if (MODE == WIDE_INFER) {
          v[q] = x + p.scal * (-ein[u][q] + dact_t<ACT>(x) * acc_v);  // x_new
          fv[q] = act_t<ACT>(v[q]);
          hv[q] = cvt<OT>(fv[q]);
        } else if (MODE == WIDE_FWD) {
          v[q] = acc_v;                                              // x = W f(x_upper)
          fv[q] = act_t<ACT>(v[q]);
          hv[q] = cvt<OT>(fv[q]);
        } else {
          v[q] = x + p.scal * acc_v;                                 // W_new
          hv[q] = cvt<OT>(v[q]);
          lv[q] = cvt<OT>(v[q] - to_f32(hv[q]));
        }
        cr[q] = to_f32(hv[q]);
      }
      float* op = p.out + (long long)m * p.ldo + n;
      OT* hp = hcopy + (long long)m * p.ldh + n;
      if (vec && nv == 4) {
        *reinterpret_cast<float4*>(op) = make_float4(v[0], v[1], v[2], v[3]);
        uint2 hh; hh.x = pack2(hv[0], hv[1]); hh.y = pack2(hv[2], hv[3]);
        *reinterpret_cast<uint2*>(hp) = hh;
        if (MODE == WIDE_WEIGHT && p.hl) {
          uint2 ll; ll.x = pack2(lv[0], lv[1]); ll.y = pack2(lv[2], lv[3]);
          *reinterpret_cast<uint2*>(reinterpret_cast<OT*>(p.hl) + (long long)m * p.ldhl + n) = ll;
        }
        if (MODE == WIDE_INFER && p.out2)
          *reinterpret_cast<float4*>(p.out2 + (long long)m * p.ld2 + n) = make_float4(fv[0], fv[1], fv[2], fv[3]);
      } else {
        for (int q = 0; q < nv; ++q) {
          op[q] = v[q];
          hp[q] = hv[q];
          if (MODE == WIDE_WEIGHT && p.hl) reinterpret_cast<OT*>(p.hl)[(long long)m * p.ldhl + n + q] = lv[q];
          if (MODE == WIDE_INFER && p.out2) p.out2[(long long)m * p.ld2 + n + q] = fv[q];
        }
      }
    }
  }
  if (!p.t) return;
  __syncthreads();
  OT* tcopy = reinterpret_cast<OT*>(p.t);
  // Pass 2: two consecutive rows per thread -> one 4-byte store along m.
#pragma unroll 4
  for (int idx = tid; idx < BM * BN / 2; idx += NT) {
    const int c = idx / (BM / 2), r = (idx % (BM / 2)) * 2;
    const int m = m0 + r, n = n0 + c;
    if (m < M && n < N) {
      const OT h0 = cvt<OT>(cs[r * CS + c]);
      const OT h1 = cvt<OT>(m + 1 < M ? cs[(r + 1) * CS + c] : 0.0f);
      *reinterpret_cast<unsigned*>(tcopy + (long long)n * p.ldt + m) = pack2(h0, h1);
    }
  }
}

template <typename OT, int MODE, int SPLIT, int BM, int BN, int S, int WGM, int WGN>
struct WideCfg {
  static constexpr int smem = wide_smem(BM, BN, S, SPLIT == 2);
  template <int ACT>
  static const void* fn() {
    return reinterpret_cast<const void*>(&wide_kernel<OT, MODE, SPLIT, BM, BN, S, WGM, WGN, ACT>);
  }
  static const void* kernel(int act) {
    if (MODE != WIDE_INFER && MODE != WIDE_FWD) return fn<ACT_IDENTITY>();
    switch (act) {
      case ACT_RELU: return fn<ACT_RELU>();
      case ACT_TANH: return fn<ACT_TANH>();
      case ACT_SIGMOID: return fn<ACT_SIGMOID>();
      case ACT_SILU: return fn<ACT_SILU>();
      case ACT_GELU: return fn<ACT_GELU>();
      default: return fn<ACT_IDENTITY>();
    }
  }
  static hipError_t prepare() {
    for (int act = 0; act < (MODE == WIDE_INFER || MODE == WIDE_FWD ? 6 : 1); ++act) {
      const hipError_t e = hipFuncSetAttribute(kernel(act), hipFuncAttributeMaxDynamicSharedMemorySize, smem);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  static hipError_t launch(const WideProblem* probs, int count, int act, hipStream_t s) {
    WideBatch bt;
    bt.count = count;
    bt.act = act;
    int total = 0;
    for (int i = 0; i < count; ++i) {
      bt.p[i] = probs[i];
      bt.start[i] = total;
      total += ((probs[i].M + BM - 1) / BM) * ((probs[i].N + BN - 1) / BN);
    }
    for (int i = count; i <= WIDE_MAX_BATCH; ++i) bt.start[i] = total;
    if (total == 0) return hipSuccess;
    void* args[] = {&bt};
    return hipLaunchKernel(kernel(act), dim3(total), dim3(WGM * WGN * 64), args, smem, s);
  }
};

// BM, BN, stages, waves along M, waves along N
#ifndef WIDE_PRED1_CFG
#define WIDE_PRED1_CFG 256, 128, 3, 4, 2
#endif
#ifndef WIDE_PRED2_CFG
#define WIDE_PRED2_CFG 256, 128, 2, 4, 2
#endif
#ifndef WIDE_INFER_CFG
#define WIDE_INFER_CFG 256, 128, 3, 4, 2
#endif
#ifndef WIDE_WEIGHT_CFG
#define WIDE_WEIGHT_CFG 256, 128, 3, 4, 2
#endif
template <typename OT> using PredCfg1 = WideCfg<OT, WIDE_PRED, 1, WIDE_PRED1_CFG>;
template <typename OT> using PredCfg2 = WideCfg<OT, WIDE_PRED, 2, WIDE_PRED2_CFG>;
template <typename OT> using InferCfg = WideCfg<OT, WIDE_INFER, 1, WIDE_INFER_CFG>;
template <typename OT> using WeightCfg = WideCfg<OT, WIDE_WEIGHT, 1, WIDE_WEIGHT_CFG>;
// forward initialisation: the pred tiles (one layer per launch, not timed)
template <typename OT> using FwdCfg1 = WideCfg<OT, WIDE_FWD, 1, WIDE_PRED1_CFG>;
template <typename OT> using FwdCfg2 = WideCfg<OT, WIDE_FWD, 2, WIDE_PRED2_CFG>;

template <typename OT>
hipError_t launch_typed(int mode, const WideProblem* probs, int count, int split, int act, hipStream_t s) {
  switch (mode) {
    case WIDE_PRED:
      return split == 2 ? PredCfg2<OT>::launch(probs, count, act, s) : PredCfg1<OT>::launch(probs, count, act, s);
    case WIDE_INFER: return InferCfg<OT>::launch(probs, count, act, s);
    case WIDE_FWD:
      return split == 2 ? FwdCfg2<OT>::launch(probs, count, act, s) : FwdCfg1<OT>::launch(probs, count, act, s);
    default: return WeightCfg<OT>::launch(probs, count, act, s);
  }
}

template <typename OT>
hipError_t prepare_typed() {
  hipError_t e;
  if ((e = PredCfg1<OT>::prepare()) != hipSuccess) return e;
  if ((e = PredCfg2<OT>::prepare()) != hipSuccess) return e;
  if ((e = InferCfg<OT>::prepare()) != hipSuccess) return e;
  if ((e = FwdCfg1<OT>::prepare()) != hipSuccess) return e;
  if ((e = FwdCfg2<OT>::prepare()) != hipSuccess) return e;
  return WeightCfg<OT>::prepare();
}

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

}  // namespace

void wide_tile(int mode, int split, int* bm, int* bn) {
  (void)mode;
  (void)split;
  *bm = 256;
  *bn = 128;
}

hipError_t wide_prepare() {
  hipError_t e = prepare_typed<f16>();
  if (e != hipSuccess) return e;
  return prepare_typed<bf16>();
}

hipError_t launch_wide(int mode, const WideProblem* probs, int count, int operand, int split, int act,
                       hipStream_t s) {
  for (int base = 0; base < count; base += WIDE_MAX_BATCH) {
    const int n = count - base < WIDE_MAX_BATCH ? count - base : WIDE_MAX_BATCH;
    hipError_t e;
    if (operand == DT_F16) e = launch_typed<f16>(mode, probs + base, n, split, act, s);
    else if (operand == DT_BF16) e = launch_typed<bf16>(mode, probs + base, n, split, act, s);
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
