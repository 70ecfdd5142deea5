// ipc_gemm_kernel.h - the templated MFMA tile kernel of the GEMM family (gfx950).
//
// One templated tile kernel covers the three reference kernel families
// (src/ipc_tilelang/tilelang_kernels.py:114-349) and their grid.z batched
// forms (src/ipc_tilelang/layer_batching.py:89-346):
//
//   LAYOUT_PF  prediction+error / forward: C = W[M][K] . f(X_upper[K][N])
//   LAYOUT_INF inference update:           C = W_lower[K][M]^T . E_lower[K][N]
//   LAYOUT_WGT weight update:              C = E[M][Bt] . f(X_upper[N][Bt])^T
//
// Tiles are staged global -> registers -> LDS with the conversion to the
// 16-bit (or fp32) operand type and the activation applied on the way in, so
// both LDS operands are stored k-contiguous ([row][k]) whatever their global
// layout: W_lower is transposed here, not in a separate pass.  Each wave
// computes (BM/WGM) x (BN/WGN) with 32x32 MFMA blocks and fp32 accumulators;
// the next k-tile's global loads are issued before the current tile's MFMAs.
#pragma once

#include "ipc_device.h"
#include "ipc_launch.h"

namespace ipc {

enum { LAYOUT_PF = 0, LAYOUT_INF = 1, LAYOUT_WGT = 2 };

// Loads the idx-th 4-element vector of a tile whose global source is
// [rows][cols] (cols contiguous) with tile origin (r0, c0) and tile width
// TW in the contiguous dimension.  Out-of-range elements read as 0.
template <typename ST, int TW>
__device__ __forceinline__ void gload4(const ST* base, long long ld, int r0, int c0, int nrows,
                                       int ncols, int vec, int idx, float o[4]) {
  const int r = idx / (TW / 4);
  const int c = (idx % (TW / 4)) * 4;
  const int gr = r0 + r, gc = c0 + c;
  o[0] = o[1] = o[2] = o[3] = 0.0f;
  if (gr < nrows) {
    const ST* ptr = base + (long long)gr * ld + gc;
    if (vec && gc + 4 <= ncols) {
      load4(ptr, o);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (gc + i < ncols) o[i] = to_f32(ptr[i]);
    }
  }
}

template <typename ST, typename OT, int LAYOUT, int SPLIT, int BM, int BN, int BK, int WGM, int WGN>
__global__ void __launch_bounds__(WGM * WGN * 64) gemm_kernel(const GemmBatch batch) {
  constexpr int NT = WGM * WGN * 64;
  constexpr bool A_KMAJ = (LAYOUT != LAYOUT_INF);  // A global layout has k contiguous
  constexpr bool B_KMAJ = (LAYOUT == LAYOUT_WGT);  // B global layout has k contiguous
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int RM = WTM / 32, RN = WTN / 32;
  constexpr int PAD = (sizeof(OT) == 4) ? 4 : 8;
  constexpr int LDK = BK + PAD;
  constexpr int VA = (BM * BK) / (4 * NT);
  constexpr int VB = (BN * BK) / (4 * NT);
  static_assert(VA * 4 * NT == BM * BK && VB * 4 * NT == BN * BK, "tile/threads mismatch");
  static_assert(RM >= 1 && RN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  using MF = Mfma32<OT>;
  static_assert(BK % MF::KI == 0, "BK");
  // SPLIT 2: A = A_hi + A_lo (two 16-bit terms), 2 MFMAs per block;
  // SPLIT 3: A and B both split, A_hi B_hi + A_lo B_hi + A_hi B_lo.
  constexpr bool SPLIT_A = SPLIT >= 2;
  constexpr bool SPLIT_B = SPLIT >= 3;
  static_assert(SPLIT == 1 || (sizeof(OT) == 2 && LAYOUT == 0), "split only for 16-bit prediction operands");

  __shared__ __align__(16) OT As[BM * LDK];
  __shared__ __align__(16) OT Bs[BN * LDK];
  __shared__ __align__(16) OT Al[SPLIT_A ? BM * LDK : 8];
  __shared__ __align__(16) OT Bl[SPLIT_B ? BN * LDK : 8];

  // Which problem of the batch, which group and which output tile this
  // workgroup owns (tiles along N vary fastest).
  const int bid = blockIdx.x;
  int pi = 0;
#pragma unroll 1
  while (pi + 1 < batch.count && bid >= batch.start[pi + 1]) ++pi;
  const GemmProblem& p = batch.p[pi];
  const int M = p.M, N = p.N, K = p.K;
  const int tn = (N + BN - 1) / BN, tm = (M + BM - 1) / BM;
  const int local = bid - batch.start[pi];
  const int g = local / (tn * tm);
  const int rem = local - g * (tn * tm);
  const int m0 = (rem / tn) * BM, n0 = (rem % tn) * BN;
  const ST* A = reinterpret_cast<const ST*>(p.a) + (long long)g * p.a_gs;
  const ST* Bm = reinterpret_cast<const ST*>(p.b) + (long long)g * p.b_gs;
  const int tid = threadIdx.x;
  const int act_b = p.act_b;

  float ra[VA][4], rb[VB][4];

  auto gload = [&](int k0) {
#pragma unroll
    for (int v = 0; v < VA; ++v) {
      const int idx = tid + v * NT;
      if (A_KMAJ) gload4<ST, BK>(A, p.lda, m0, k0, M, K, p.vec_a, idx, ra[v]);
      else        gload4<ST, BM>(A, p.lda, k0, m0, K, M, p.vec_a, idx, ra[v]);
    }
#pragma unroll
    for (int v = 0; v < VB; ++v) {
      const int idx = tid + v * NT;
      if (B_KMAJ) gload4<ST, BK>(Bm, p.ldb, n0, k0, N, K, p.vec_b, idx, rb[v]);
      else        gload4<ST, BN>(Bm, p.ldb, k0, n0, K, N, p.vec_b, idx, rb[v]);
    }
  };

  auto lstore = [&](int k0) {
#pragma unroll
    for (int v = 0; v < VA; ++v) {
      const int idx = tid + v * NT;
      if (A_KMAJ) {
        const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const OT hi = cvt<OT>(ra[v][i]);
          As[r * LDK + c + i] = hi;
          if (SPLIT_A) Al[r * LDK + c + i] = cvt<OT>(ra[v][i] - to_f32(hi));
        }
      } else {
        const int r = idx / (BM / 4), c = (idx % (BM / 4)) * 4;  // r = k, c = m
#pragma unroll
        for (int i = 0; i < 4; ++i) As[(c + i) * LDK + r] = cvt<OT>(ra[v][i]);
      }
    }
#pragma unroll
    for (int v = 0; v < VB; ++v) {
      const int idx = tid + v * NT;
      if (B_KMAJ) {
        const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;  // r = n, c = k
        const bool rin = (n0 + r) < N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool in = rin && (k0 + c + i) < K;
          Bs[r * LDK + c + i] = cvt<OT>(in ? act_f(act_b, rb[v][i]) : 0.0f);
        }
      } else {
        const int r = idx / (BN / 4), c = (idx % (BN / 4)) * 4;  // r = k, c = n
        const bool rin = (k0 + r) < K;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool in = rin && (n0 + c + i) < N;
          const float bv = in ? act_f(act_b, rb[v][i]) : 0.0f;
          const OT hi = cvt<OT>(bv);
          Bs[(c + i) * LDK + r] = hi;
          if (SPLIT_B) Bl[(c + i) * LDK + r] = cvt<OT>(bv - to_f32(hi));
        }
      }
    }
  };

  f32x16 acc[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int lr = lane & 31, lk = lane >> 5;

  const int nkt = (K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int t = 0; t < nkt; ++t) {
    if (t + 1 < nkt) gload((t + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += MF::KI) {
      typename MF::operand af[RM], bfr[RN];
#pragma unroll
      for (int i = 0; i < RM; ++i)
        af[i] = *reinterpret_cast<const typename MF::operand*>(
            &As[(wm * WTM + i * 32 + lr) * LDK + kk + lk * MF::KPL]);
#pragma unroll
      for (int j = 0; j < RN; ++j)
        bfr[j] = *reinterpret_cast<const typename MF::operand*>(
            &Bs[(wn * WTN + j * 32 + lr) * LDK + kk + lk * MF::KPL]);
#pragma unroll
      for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(af[i], bfr[j], acc[i][j]);
      if (SPLIT_A) {
#pragma unroll
        for (int i = 0; i < RM; ++i) {
          const typename MF::operand alo = *reinterpret_cast<const typename MF::operand*>(
              &Al[(wm * WTM + i * 32 + lr) * LDK + kk + lk * MF::KPL]);
#pragma unroll
          for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(alo, bfr[j], acc[i][j]);
        }
      }
      if (SPLIT_B) {
#pragma unroll
        for (int j = 0; j < RN; ++j) {
          const typename MF::operand blo = *reinterpret_cast<const typename MF::operand*>(
              &Bl[(wn * WTN + j * 32 + lr) * LDK + kk + lk * MF::KPL]);
#pragma unroll
          for (int i = 0; i < RM; ++i) acc[i][j] = MF::run(af[i], blo, acc[i][j]);
        }
      }
    }
    __syncthreads();
    if (t + 1 < nkt) {
      lstore((t + 1) * BK);
      __syncthreads();
    }
  }

  // ------------------------------------------------------------ epilogue
  ST* out = reinterpret_cast<ST*>(p.out) + (long long)g * p.o_gs;
  const ST* aux = p.aux ? reinterpret_cast<const ST*>(p.aux) + (long long)g * p.x_gs : nullptr;
  ST* out2 = p.out2 ? reinterpret_cast<ST*>(p.out2) + (long long)g * p.o2_gs : nullptr;
  const float scal = p.scal;
  const int act_e = p.act_epi;
#pragma unroll
  for (int i = 0; i < RM; ++i) {
#pragma unroll
    for (int j = 0; j < RN; ++j) {
      const int n = n0 + wn * WTN + j * 32 + lr;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int m = m0 + wm * WTM + i * 32 + 8 * (q >> 2) + 4 * lk + (q & 3);
        if (m < M && n < N) {
          // Every epilogue operation rounds on its own, in the order of the
          // fp32 reference (reference.py:49,57), never fused into an FMA: the
          // weight delta is far below W's own ulp scale, so a fused
          // W + alpha*acc would differ from the reference by one ulp of W per step.
#pragma clang fp contract(off)
          const float c = acc[i][j][q];
          const long long o = (long long)m * p.ldo + n;
          if (LAYOUT == LAYOUT_PF) {
            if (p.kind == KIND_PRED) {
              // tilelang_kernels.py:173: E = cast(X_lower) - cast(acc) in storage precision.
              const float xl = to_f32(aux[(long long)m * p.ldx + n]);
              out[o] = cvt<ST>(xl - to_f32(cvt<ST>(c)));
            } else {
              out[o] = cvt<ST>(c);
            }
          } else if (LAYOUT == LAYOUT_INF) {
            // tilelang_kernels.py:227-231 / 259-262.
            const float x = to_f32(out[o]);
            const float e = to_f32(aux[(long long)m * p.ldx + n]);
            const float xn = x + scal * (-e + act_df(act_e, x) * c);  // rounded term by term
            out[o] = cvt<ST>(xn);
            if (out2) out2[(long long)m * p.ld2 + n] = cvt<ST>(act_f(act_e, xn));
          } else {
            // tilelang_kernels.py:319-320: W = cast(float(W) + alpha * acc).
            out[o] = cvt<ST>(to_f32(out[o]) + scal * c);
          }
        }
      }
    }
  }
}

// Launch of one tile configuration over a ragged batch (count <= MAX_BATCH
// per launch; longer lists are split).
template <typename ST, typename OT, int LAYOUT, int SPLIT, int BM, int BN, int BK, int WGM, int WGN>
static hipError_t run_tile(const GemmProblem* probs, int count, hipStream_t s) {
  for (int base = 0; base < count; base += MAX_BATCH) {
    GemmBatch batch;
    batch.count = count - base < MAX_BATCH ? count - base : MAX_BATCH;
    int total = 0;
    for (int i = 0; i < batch.count; ++i) {
      const GemmProblem& q = probs[base + i];
      batch.p[i] = q;
      batch.start[i] = total;
      total += ((q.N + BN - 1) / BN) * ((q.M + BM - 1) / BM) * q.groups;
    }
    for (int i = batch.count; i <= MAX_BATCH; ++i) batch.start[i] = total;
    if (total == 0) continue;
    hipLaunchKernelGGL((gemm_kernel<ST, OT, LAYOUT, SPLIT, BM, BN, BK, WGM, WGN>), dim3(total),
                       dim3(WGM * WGN * 64), 0, s, batch);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename ST, typename OT, int LAYOUT, int SPLIT>
static hipError_t run_tiles(const GemmProblem* probs, int count, int tile, hipStream_t s) {
  switch (tile) {
    case 0: return run_tile<ST, OT, LAYOUT, SPLIT, 32, 32, 32, 1, 1>(probs, count, s);
    case 1: return run_tile<ST, OT, LAYOUT, SPLIT, 64, 64, 32, 2, 2>(probs, count, s);
    default: return run_tile<ST, OT, LAYOUT, SPLIT, 128, 128, 32, 2, 2>(probs, count, s);
  }
}

// Per-layout entry points, one translation unit each (ipc_gemm_pf.hip,
// ipc_gemm_inf.hip, ipc_gemm_wgt.hip).
hipError_t launch_layout_pf(const GemmProblem* probs, int count, int storage, int operand, int split, int tile,
                            hipStream_t s);
hipError_t launch_layout_inf(const GemmProblem* probs, int count, int storage, int operand, int tile,
                             hipStream_t s);
hipError_t launch_layout_wgt(const GemmProblem* probs, int count, int storage, int operand, int tile,
                             hipStream_t s);

}  // namespace ipc
