// ipc_narrow.hip - whole-step kernel for narrow iPC nets (gfx950).
//
// For nets whose every output width d_0..d_{L-1} is <= 128 (the paper
// efficiency profile 784 -> 64^d -> 10, the small-batch profile), a step is a
// few tens of MFLOP spread over ~3L small GEMMs: dependency latency, not
// bandwidth or MFMA rate, bounds it.  One kernel therefore runs whole steps
// (reference trainer.py:601-679 semantics) with as few dependent memory
// round trips as the math allows:
//
//   phase A (column-parallel, one workgroup per 16 batch columns):
//     1. stage every layer's x[l] (fp32) and f(x[l]) (operand type,
//        [column][k]) for the block's columns into LDS;
//     2. every prediction unit (layer, 16-row tile) at once - they are
//        mutually independent - eps = x[l] - W[l] f(x[l+1]); W rows are
//        prefetched a chunk of k-steps at a time straight into MFMA 16x16
//        operand registers;
//     3. every inference unit at once, x[l] += gamma(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1]),
//        W[l-1] read transposed from global memory, eps[l-1] from LDS; the
//        epilogue also writes f(x_new) for phase B and refreshes the LDS copies.
//     No column block depends on another, so phase A has no inter-workgroup
//     synchronisation.  In a multi-step launch every workgroup owns one column
//     block for all steps and its LDS copies stay resident: only W is re-read.
//   phase B (weight update): 64x64 tiles of every W[l] are spread over the
//     workgroups, W[l] += alpha eps[l] f(x_new[l+1])^T contracting over the
//     batch with MFMA (f(x_new) comes pre-evaluated from phase A), or, for
//     B <= 16, as a rank-B outer product on the VALU.
//
// The phases are separated by a grid barrier (a monotonically increasing
// arrival counter in a caller-provided workspace, every wait bounded by a spin
// limit that raises a flag instead of hanging), so T steps run in one launch.
// Each phase can also be launched on its own (modes PHASE_A / PHASE_B), and
// FORWARD runs the forward initialisation x[l] = W[l] f(x[l+1]) layer by layer
// with the same prediction units as phase A, so the hidden prediction errors
// are exactly 0 after it, as in trainer.py:512-515.
//
// Inner loops issue their global loads first (branch-free: clamped address,
// masked value) and compute afterwards, so each chunk of loads costs one
// memory latency instead of one per k-step.  The activation is a template
// parameter, so no switch sits in any inner loop.
#include "ipc_device.h"
#include "ipc_launch.h"
#include "ipc_narrow.h"

namespace ipc {

namespace {

constexpr int NT = 512;  // threads per workgroup (8 waves)
constexpr int NW = NT / 64;
constexpr int NC = NARROW_NC;
constexpr int WT = 64;   // weight-update tile edge
constexpr int SCH = 8;   // staging: elements per thread per load batch

// acc(16x16) += A(16 x KS) B(KS x 16).  Lane (r = lane % 16, g = lane / 16)
// supplies a[q] = A[r][k0 + g*KL + q] and b[q] = B[k0 + g*KL + q][r], q < KL.
// Result element j of lane l is C[4*(l/16) + j][l % 16].
template <typename OT> struct Mma16;
template <> struct Mma16<float> {
  static constexpr int KS = 16, KL = 4, PAD = 4;
  __device__ __forceinline__ static f32x4 run(const float* a, const float* b, f32x4 c) {
    // four 16x16x4 instructions; instruction s takes k = k0 + 4g + s from lane group g
#pragma unroll
    for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
    return c;
  }
};
template <> struct Mma16<f16> {
  static constexpr int KS = 32, KL = 8, PAD = 8;
  __device__ __forceinline__ static f32x4 run(const f16* a, const f16* b, f32x4 c) {
    f16x8 va, vb;
#pragma unroll
    for (int q = 0; q < 8; ++q) { va[q] = a[q]; vb[q] = b[q]; }
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(va, vb, c, 0, 0, 0);
  }
};
template <> struct Mma16<bf16> {
  static constexpr int KS = 32, KL = 8, PAD = 8;
  __device__ __forceinline__ static f32x4 run(const bf16* a, const bf16* b, f32x4 c) {
    bf16x8 va, vb;
#pragma unroll
    for (int q = 0; q < 8; ++q) { va[q] = a[q]; vb[q] = b[q]; }
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, vb, c, 0, 0, 0);
  }
};

__device__ __forceinline__ int round_up(int v, int m) { return (v + m - 1) / m * m; }

// KL consecutive values row[k .. k+KL), zero outside [0, K) or when !ok.
// Every lane loads from an in-bounds address (row[0] when masked): no branch.
// VEC (K % KL == 0, 16-byte aligned matrix): 16-byte loads; a run is then
// wholly in or wholly out of range.
template <int KL, bool VEC>
__device__ __forceinline__ void load_run(const float* row, int k, int K, bool ok, float* o) {
  if (VEC) {
    const bool in = ok && k < K;
    const float4* src = reinterpret_cast<const float4*>(row + (in ? k : 0));
#pragma unroll
    for (int q = 0; q < KL / 4; ++q) {
      const float4 v = src[q];
      o[4 * q] = in ? v.x : 0.0f;
      o[4 * q + 1] = in ? v.y : 0.0f;
      o[4 * q + 2] = in ? v.z : 0.0f;
      o[4 * q + 3] = in ? v.w : 0.0f;
    }
  } else {
#pragma unroll
    for (int q = 0; q < KL; ++q) {
      const bool in = ok && (k + q) < K;
      const float v = row[in ? k + q : 0];
      o[q] = in ? v : 0.0f;
    }
  }
}

// Grid barrier over the launch's workgroups: arrival number `nbar` completes
// when the counter reaches (nbar + 1) * nblocks.  Bounded: after spin_limit
// polls the timeout flag is raised and the wait ends.
__device__ void grid_barrier(unsigned* bar, int nblocks, int nbar, int spin_limit) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const unsigned target = (unsigned)(nbar + 1) * (unsigned)nblocks;
    __hip_atomic_fetch_add(&bar[0], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    int spins = 0;
    while (__hip_atomic_load(&bar[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > spin_limit) {
        __hip_atomic_store(&bar[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __threadfence();
  }
  __syncthreads();
}

// Last workgroup out resets the arrival counter for the next launch.
__device__ void barrier_exit(unsigned* bar, int nblocks) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&bar[1], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (unsigned)nblocks - 1) {
      __hip_atomic_store(&bar[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&bar[1], 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <typename OT, int SPLIT, int ACT>
struct Narrow {
  using MM = Mma16<OT>;
  static constexpr int KS = MM::KS, KL = MM::KL, PAD = MM::PAD;
  static constexpr bool SA = SPLIT >= 2, SB = SPLIT >= 3;
  static constexpr int NPF = 64 / KL;  // k-steps per prefetched chunk (64 floats per lane)

  const NarrowArgs& p;
  const NarrowLds& lay;
  char* lds;
  const int tid, lane, wave, lr, lg;

  __device__ __forceinline__ Narrow(const NarrowArgs& args, const NarrowLds& layout, char* base)
      : p(args), lay(layout), lds(base), tid(threadIdx.x), lane(threadIdx.x & 63), wave(threadIdx.x >> 6),
        lr(threadIdx.x & 15), lg((threadIdx.x & 63) >> 4) {}

  __device__ __forceinline__ static int ldk(int d) { return narrow_ldk(d, KS, PAD); }
  __device__ __forceinline__ float* xr(int l) { return reinterpret_cast<float*>(lds) + lay.xr_row[l] * NC; }
  __device__ __forceinline__ float* ef(int l) {
    return reinterpret_cast<float*>(lds + lay.ef_base) + lay.ef_row[l] * NC;
  }
  __device__ __forceinline__ OT* fs_hi(int l) { return reinterpret_cast<OT*>(lds + lay.fs_base) + lay.fs_off[l]; }
  __device__ __forceinline__ OT* fs_lo(int l) { return fs_hi(l) + NC * ldk(p.dims[l]); }
  __device__ __forceinline__ OT* es(int l) { return reinterpret_cast<OT*>(lds + lay.es_base) + lay.es_off[l]; }

  // Stages layer l of column block [c0, c0+ncols): raw x into xr (keep_raw),
  // f(x) into the fs block ([n][k], zero for k >= d_l or n >= ncols) and, with
  // fx_out, f(x) into the global pre-activation buffer.  Loads are issued SCH
  // at a time before any of them is used.
  __device__ __forceinline__ void stage_layer(int l, int c0, int ncols, bool keep_raw, bool want_f, float* fx_out) {
    const int d = p.dims[l], ld = ldk(d), B = p.B;
    const float* X = p.x[l];
    const int rows = want_f ? ld : d;
    const int total = rows * NC;
    for (int base = tid; base < total; base += NT * SCH) {
      float v[SCH];
#pragma unroll
      for (int i = 0; i < SCH; ++i) {
        const int idx = base + i * NT;
        const int k = idx / NC, n = idx - k * NC;
        const bool in = idx < total && k < d && n < ncols;
        const float t = X[in ? (long long)k * B + c0 + n : 0];
        v[i] = in ? t : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < SCH; ++i) {
        const int idx = base + i * NT;
        if (idx < total) {
          const int k = idx / NC, n = idx - k * NC;
          const bool in = k < d && n < ncols;
          if (keep_raw && k < d) xr(l)[k * NC + n] = v[i];
          if (want_f) {
            const float fv = in ? act_t<ACT>(v[i]) : 0.0f;
            const OT hi = cvt<OT>(fv);
            fs_hi(l)[n * ld + k] = hi;
            if (SB) fs_lo(l)[n * ld + k] = cvt<OT>(fv - to_f32(hi));
            if (fx_out && in) fx_out[(long long)k * B + c0 + n] = fv;
          }
        }
      }
    }
  }

  // The contraction is accumulated in partials of NARROW_KCHUNK columns that
  // are summed in order, the order in which the layer-resident kernel adds
  // its top-layer column chunks: a forward initialisation by this kernel then
  // leaves that kernel's first prediction errors exactly zero as well.
  template <bool VEC, int CH>
  __device__ __forceinline__ f32x4 pred_loop(const float* wrow, bool rok, int K, const OT* fh, const OT* fl,
                                             int nsteps) {
    constexpr int KPC = NARROW_KCHUNK / KS;  // k-steps per partial
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f}, sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < nsteps; s0 += CH) {
      float av[CH][KL];
#pragma unroll
      for (int i = 0; i < CH; ++i)
        load_run<KL, VEC>(wrow, (s0 + i) * KS + lg * KL, K, rok && (s0 + i) < nsteps, av[i]);
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        if (s0 + i < nsteps) {
          if (s0 + i > 0 && (s0 + i) % KPC == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) sum[q] = sum[q] + c[q];
            c = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
          const int kk = (s0 + i) * KS;
          OT ah[KL], al[KL], bh[KL], bl[KL];
#pragma unroll
          for (int q = 0; q < KL; ++q) {
            ah[q] = cvt<OT>(av[i][q]);
            if (SA) al[q] = cvt<OT>(av[i][q] - to_f32(ah[q]));
            bh[q] = fh[kk + q];
            if (SB) bl[q] = fl[kk + q];
          }
          c = MM::run(ah, bh, c);
          if (SA) c = MM::run(al, bh, c);
          if (SB) c = MM::run(ah, bl, c);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) sum[q] = sum[q] + c[q];
    return sum;
  }

  // One prediction unit: acc = W[l][rt*16 .. +16][:] f(x[l+1])[:, cols] from the staged fs block.
  __device__ __forceinline__ f32x4 pred_unit(int l, int rt) {
    const int M = p.dims[l], K = p.dims[l + 1], ld = ldk(K);
    const float* W = p.w[l];
    const int row = rt * 16 + lr;
    const bool rok = row < M;
    const float* wrow = W + (long long)(rok ? row : 0) * K;
    const bool vec = (K % KL == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
    const OT* fh = fs_hi(l + 1) + lr * ld + lg * KL;
    const OT* fl = SB ? fs_lo(l + 1) + lr * ld + lg * KL : nullptr;
    const int nsteps = round_up(K, KS) / KS;
    // one loop body per load type keeps the kernel's code small
    if (vec) return pred_loop<true, NPF>(wrow, rok, K, fh, fl, nsteps);
    return pred_loop<false, 4>(wrow, rok, K, fh, fl, nsteps);
  }

  // One inference unit: acc = W[l-1]^T[rt*16 .. +16][:] eps[l-1][:, cols]
  // (contraction d_{l-1} <= 128: every load of the unit is issued first).
  __device__ __forceinline__ f32x4 infer_unit(int l, int rt) {
    constexpr int MAXS = NARROW_MAX_WIDTH / KS;
    const int M = p.dims[l], Kp = p.dims[l - 1], ld = ldk(Kp);
    const float* Wl = p.w[l - 1];  // [Kp][M]
    const int m = rt * 16 + lr;
    const bool mok = m < M;
    const OT* eb = es(l - 1) + lr * ld + lg * KL;
    const int nsteps = round_up(Kp, KS) / KS;
    float av[MAXS][KL];
#pragma unroll
    for (int i = 0; i < MAXS; ++i)
#pragma unroll
      for (int q = 0; q < KL; ++q) {
        const int k = i * KS + lg * KL + q;
        const bool in = mok && k < Kp && i < nsteps;
        const float v = Wl[in ? (long long)k * M + m : 0];
        av[i][q] = in ? v : 0.0f;
      }
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < MAXS; ++i) {
      if (i < nsteps) {
        OT ah[KL], bh[KL];
#pragma unroll
        for (int q = 0; q < KL; ++q) {
          ah[q] = cvt<OT>(av[i][q]);
          bh[q] = eb[i * KS + q];
        }
        c = MM::run(ah, bh, c);
      }
    }
    return c;
  }

  // Stages column block cb: every layer's x (raw) and f(x), zeroed eps blocks,
  // and f(x[L]) of the block's columns into the pre-activation buffer.
  __device__ __forceinline__ void stage_all(int cb) {
    const int B = p.B, L = p.L, c0 = cb * NC, ncols = min(NC, B - c0);
    __syncthreads();  // LDS of the previous column block / phase is free
    // eps blocks are the zero-padded B operands of the inference units
    for (int l = 0; l + 1 < L; ++l) {
      OT* e_l = es(l);
      const int n_el = NC * ldk(p.dims[l]);
      for (int i = tid; i < n_el; i += NT) e_l[i] = cvt<OT>(0.0f);
    }
    for (int l = 0; l <= L; ++l) stage_layer(l, c0, ncols, l < L, l >= 1, l == L ? p.fx[L] : nullptr);
  }

  // Phase A for column block cb.  With `resident` the block's LDS already
  // holds this column block's x, f(x) and eps padding from the previous step
  // (the inference epilogue keeps them current), so nothing is restaged.
  __device__ __forceinline__ void phase_a(int cb, bool resident) {
    const int B = p.B, L = p.L, c0 = cb * NC, ncols = min(NC, B - c0);
    const float gamma = p.gamma;
    if (!resident) stage_all(cb);
    __syncthreads();
    // ---- every prediction unit: eps = x[l] - W[l] f(x[l+1])
    for (int u = wave; u < p.n_units; u += NW) {
      const int l = p.unit_l[u], rt = p.unit_rt[u];
      const int M = p.dims[l];
      const f32x4 c = pred_unit(l, rt);
      const int ld_e = ldk(M);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = rt * 16 + lg * 4 + j;
        if (row < M && lr < ncols) {
          const float ev = xr(l)[row * NC + lr] - c[j];
          p.e[l][(long long)row * B + c0 + lr] = ev;
          if (l >= 1) ef(l)[row * NC + lr] = ev;
          if (l + 1 < L) es(l)[lr * ld_e + row] = cvt<OT>(ev);
        }
      }
    }
    __syncthreads();
    // ---- every inference unit: x[l] += gamma(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1])
    for (int u = wave; u < p.n_units; u += NW) {
      const int l = p.unit_l[u], rt = p.unit_rt[u];
      if (l == 0) continue;
      const int M = p.dims[l];
      const f32x4 c = infer_unit(l, rt);
      float* fxl = p.fx[l];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = rt * 16 + lg * 4 + j;
        if (row < M && lr < ncols) {
#pragma clang fp contract(off)
          const long long o = (long long)row * B + c0 + lr;
          const float x = xr(l)[row * NC + lr];
          const float xn = x + gamma * (-ef(l)[row * NC + lr] + dact_t<ACT>(x) * c[j]);
          p.x[l][o] = xn;
          const float fxn = act_t<ACT>(xn);
          fxl[o] = fxn;
          if (resident) {
            // keep the block's staged copies current for the next step
            xr(l)[row * NC + lr] = xn;
            const int ld = ldk(M);
            const OT hi = cvt<OT>(fxn);
            fs_hi(l)[lr * ld + row] = hi;
            if (SB) fs_lo(l)[lr * ld + row] = cvt<OT>(fxn - to_f32(hi));
          }
        }
      }
    }
  }

  // Forward initialisation for column block cb: x[l] = W[l] f(x[l+1]), l = L-1 .. 1.
  __device__ __forceinline__ void forward(int cb) {
    const int B = p.B, L = p.L, c0 = cb * NC, ncols = min(NC, B - c0);
    for (int l = L - 1; l >= 1; --l) {
      __syncthreads();
      stage_layer(l + 1, c0, ncols, false, true, nullptr);
      __syncthreads();
      const int M = p.dims[l];
      for (int rt = wave; rt * 16 < M; rt += NW) {
        const f32x4 c = pred_unit(l, rt);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = rt * 16 + lg * 4 + j;
          if (row < M && lr < ncols) p.x[l][(long long)row * B + c0 + lr] = c[j];
        }
      }
    }
    if (p.a[L]) {
      for (int i = tid; i < p.dims[L] * NC; i += NT) {
        const int k = i / NC, n = i - k * NC;
        if (n < ncols) p.a[L][(long long)k * B + c0 + n] = act_t<ACT>(p.x[L][(long long)k * B + c0 + n]);
      }
    }
  }

  // Phase B for weight tile `tile`: W[l] tile += alpha eps[l] f(x_new[l+1])^T,
  // f(x_new[l+1]) read pre-evaluated from fx[l+1].
  __device__ __forceinline__ void phase_b(int tile) {
    int l = 0;
    while (l + 1 < p.L && tile >= p.wtile_start[l + 1]) ++l;
    const int M = p.dims[l], N = p.dims[l + 1], B = p.B;
    const int tn = (N + WT - 1) / WT;
    const int local = tile - p.wtile_start[l];
    const int m0 = (local / tn) * WT, n0 = (local % tn) * WT;
    const float* E = p.e[l];
    const float* X = p.fx[l + 1];
    float* W = p.w[l];
    const float alpha = p.alpha;
    if (p.outer) {
      // rank-B outer product on the VALU (B <= NC)
      float* so_e = reinterpret_cast<float*>(lds + lay.outer_base);
      float* so_x = so_e + WT * (NC + 1);
      __syncthreads();
      for (int i = tid; i < WT * B; i += NT) {
        const int r = i / B, b = i - r * B;
        so_e[r * (NC + 1) + b] = (m0 + r < M) ? E[(long long)(m0 + r) * B + b] : 0.0f;
        so_x[r * (NC + 1) + b] = (n0 + r < N) ? X[(long long)(n0 + r) * B + b] : 0.0f;
      }
      __syncthreads();
      for (int i = tid; i < WT * WT; i += NT) {
        const int r = i / WT, c = i - r * WT;
        const int m = m0 + r, n = n0 + c;
        if (m < M && n < N) {
          float s = 0.0f;
          // fused multiply-adds from zero in batch order (the layer-resident
          // kernel's rank-B update computes the same sums)
          for (int b = 0; b < B; ++b) s = __builtin_fmaf(so_e[r * (NC + 1) + b], so_x[c * (NC + 1) + b], s);
          {
#pragma clang fp contract(off)
            const long long o = (long long)m * N + n;
            W[o] = W[o] + alpha * s;
          }
        }
      }
      return;
    }
    // wave w: rows m0 + (w % 4) * 16, columns n0 + (w / 4) * 32 .. +32 (two 16-column blocks)
    const int rb = wave & 3, ch = wave >> 2;
    const bool vec = (B % KL == 0) && ((reinterpret_cast<uintptr_t>(E) & 15) == 0) &&
                     ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
    const int m = m0 + rb * 16 + lr;
    const bool mok = m < M;
    const float* erow = E + (long long)(mok ? m : 0) * B;
    const float* xrow[2];
    bool nok[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = n0 + ch * 32 + s * 16 + lr;
      nok[s] = n < N;
      xrow[s] = X + (long long)(nok[s] ? n : 0) * B;
    }
    // the W tile values of the epilogue, fetched before the contraction
    float wv[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = m0 + rb * 16 + lg * 4 + j;
        const int col = n0 + ch * 32 + s * 16 + lr;
        const bool in = row < M && col < N;
        const float v = W[in ? (long long)row * N + col : 0];
        wv[s][j] = in ? v : 0.0f;
      }
    f32x4 acc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) acc[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int BCH = 16 / KL;  // k-steps per load batch (16 floats per operand row)
    const int nsteps = round_up(B, KS) / KS;
    for (int s0 = 0; s0 < nsteps; s0 += BCH) {
      float av[BCH][KL], xv[2][BCH][KL];
      if (vec) {
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
          const int b = (s0 + i) * KS + lg * KL;
          load_run<KL, true>(erow, b, B, mok, av[i]);
          load_run<KL, true>(xrow[0], b, B, nok[0], xv[0][i]);
          load_run<KL, true>(xrow[1], b, B, nok[1], xv[1][i]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
          const int b = (s0 + i) * KS + lg * KL;
          load_run<KL, false>(erow, b, B, mok, av[i]);
          load_run<KL, false>(xrow[0], b, B, nok[0], xv[0][i]);
          load_run<KL, false>(xrow[1], b, B, nok[1], xv[1][i]);
        }
      }
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        if (s0 + i < nsteps) {
          OT ah[KL], b0h[KL], b1h[KL];
#pragma unroll
          for (int q = 0; q < KL; ++q) {
            ah[q] = cvt<OT>(av[i][q]);
            b0h[q] = cvt<OT>(xv[0][i][q]);
            b1h[q] = cvt<OT>(xv[1][i][q]);
          }
          acc[0] = MM::run(ah, b0h, acc[0]);
          acc[1] = MM::run(ah, b1h, acc[1]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = m0 + rb * 16 + lg * 4 + j;
        const int col = n0 + ch * 32 + s * 16 + lr;
        if (row < M && col < N) {
#pragma clang fp contract(off)
          W[(long long)row * N + col] = wv[s][j] + alpha * acc[s][j];
        }
      }
    }
  }
};

template <typename OT, int SPLIT, int ACT>
__global__ void __launch_bounds__(NT) narrow_kernel(const NarrowArgs p) {
  using N = Narrow<OT, SPLIT, ACT>;
  extern __shared__ __align__(16) char lds[];
  __shared__ NarrowLds layout;
  // The argument block (unit lists, dimensions, per-layer pointers) is read
  // with layer / unit indices known only at run time, which the compiler
  // serves from the kernel-argument segment in memory: a memory round trip in
  // front of every unit's loads.  A copy in LDS answers in LDS latency.
  __shared__ NarrowArgs sp;
  static_assert(sizeof(NarrowArgs) % 4 == 0, "argument block copy");
  for (int i = threadIdx.x; i < (int)(sizeof(NarrowArgs) / 4); i += NT)
    reinterpret_cast<int*>(&sp)[i] = reinterpret_cast<const int*>(&p)[i];
  if (threadIdx.x == 0)
    narrow_lds_layout(p.dims, p.L, N::KS, N::PAD, (int)sizeof(OT), N::SB, layout);
  __syncthreads();
  N k(sp, layout, lds);
  const int ncb = (p.B + NC - 1) / NC;
  const int ntile = p.wtile_start[p.L];
  const int nb = gridDim.x;
  // a launch of this kernel on a layer-resident plan (the forward
  // initialisation, which may change x[L], or a single phase, which changes x
  // or W) makes that kernel's cached operands (input images, f(x) copies,
  // first-step partial products) stale: a new generation marks them so
  if (p.res_image_flag && blockIdx.x == 0 && threadIdx.x == 0) *p.res_image_flag += 1u;
  if (p.mode == NMODE_FORWARD) {
    for (int cb = blockIdx.x; cb < ncb; cb += nb) k.forward(cb);
    return;
  }
  // One loop serves the multi-step launch and the single-phase launches, so
  // each phase's code exists once in the kernel.  In a multi-step launch in
  // which every column block has its own workgroup, each workgroup stages its
  // block once and keeps it LDS-resident for all steps.
  const bool do_a = p.mode != NMODE_PHASE_B, do_b = p.mode != NMODE_PHASE_A;
  const bool multi = p.mode == NMODE_STEPS;
  const bool resident = multi && ncb <= nb;
  if (resident && (int)blockIdx.x < ncb) k.stage_all(blockIdx.x);
  const int steps = multi ? p.steps : 1;
  int nbar = 0;
  for (int s = 0; s < steps; ++s) {
    if (do_a)
      for (int cb = blockIdx.x; cb < ncb; cb += nb) k.phase_a(cb, resident);
    if (multi) grid_barrier(p.bar, nb, nbar++, p.spin_limit);
    if (do_b)
      for (int t = blockIdx.x; t < ntile; t += nb) k.phase_b(t);
    if (multi && s + 1 < steps) grid_barrier(p.bar, nb, nbar++, p.spin_limit);
  }
  if (multi) barrier_exit(p.bar, nb);
}

// ---------------------------------------------------------------- dispatch
template <typename OT, int SPLIT, int ACT>
struct KernelRef {
  static const void* get() { return reinterpret_cast<const void*>(&narrow_kernel<OT, SPLIT, ACT>); }
  static void launch(const NarrowArgs& p, dim3 g, dim3 b, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((narrow_kernel<OT, SPLIT, ACT>), g, b, lds, s, p);
  }
};

template <template <typename, int, int> class F, typename OT, int SPLIT, typename... Args>
auto by_act(int act, Args&&... a) {
  switch (act) {
    case ACT_RELU: return F<OT, SPLIT, ACT_RELU>::run(a...);
    case ACT_TANH: return F<OT, SPLIT, ACT_TANH>::run(a...);
    case ACT_SIGMOID: return F<OT, SPLIT, ACT_SIGMOID>::run(a...);
    case ACT_SILU: return F<OT, SPLIT, ACT_SILU>::run(a...);
    case ACT_GELU: return F<OT, SPLIT, ACT_GELU>::run(a...);
    default: return F<OT, SPLIT, ACT_IDENTITY>::run(a...);
  }
}

template <template <typename, int, int> class F, typename... Args>
auto by_type(int operand, int split, int act, Args&&... a) {
  if (operand == DT_F32) return by_act<F, float, 1>(act, a...);
  if (operand == DT_F16) {
    if (split >= 3) return by_act<F, f16, 3>(act, a...);
    return by_act<F, f16, 1>(act, a...);
  }
  if (split >= 3) return by_act<F, bf16, 3>(act, a...);
  return by_act<F, bf16, 1>(act, a...);
}

template <typename OT, int SPLIT, int ACT>
struct SetLds {
  static hipError_t run(int bytes) {
    return hipFuncSetAttribute(KernelRef<OT, SPLIT, ACT>::get(), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  }
};

template <typename OT, int SPLIT, int ACT>
struct Occupancy {
  static hipError_t run(int bytes, int* per_cu) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, KernelRef<OT, SPLIT, ACT>::get(), NT, (size_t)bytes);
  }
};

template <typename OT, int SPLIT, int ACT>
struct Launch {
  static hipError_t run(const NarrowArgs& p, hipStream_t s) {
    KernelRef<OT, SPLIT, ACT>::launch(p, dim3(p.nblocks), dim3(NT), (size_t)p.lds_bytes, s);
    return hipGetLastError();
  }
};

}  // namespace

int narrow_tiles(const int* dims, int L) {
  int total = 0;
  for (int l = 0; l < L; ++l) total += ((dims[l] + WT - 1) / WT) * ((dims[l + 1] + WT - 1) / WT);
  return total;
}

int narrow_lds_bytes(const int* dims, int L, int operand, int split) {
  NarrowLds o;
  if (operand == DT_F32) narrow_lds_layout(dims, L, Mma16<float>::KS, Mma16<float>::PAD, 4, false, o);
  else narrow_lds_layout(dims, L, Mma16<f16>::KS, Mma16<f16>::PAD, 2, split >= 3, o);
  return o.total;
}

hipError_t narrow_prepare(int operand, int split, int act, int lds_bytes) {
  return by_type<SetLds>(operand, split, act, lds_bytes);
}

hipError_t narrow_occupancy(int operand, int split, int act, int lds_bytes, int* per_cu) {
  *per_cu = 0;
  return by_type<Occupancy>(operand, split, act, lds_bytes, per_cu);
}

hipError_t launch_narrow(const NarrowArgs& p, int operand, int split, hipStream_t s) {
  return by_type<Launch>(operand, split, p.act, p, s);
}

}  // namespace ipc
