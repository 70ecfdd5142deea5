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
//     1. stage, in one round trip, every layer's x[l] (fp32) and f(x[l])
//        (operand type, [column][k]) for the block's columns into LDS;
//     2. every prediction unit (layer, 16-row tile) at once - they are
//        mutually independent - eps = x[l] - W[l] f(x[l+1]), W rows streaming
//        from L2 straight into MFMA 16x16 operand registers;
//     3. every inference unit at once, x[l] += gamma(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1]),
//        W[l-1] read transposed from global memory, eps[l-1] from LDS.
//     No column block depends on another, so phase A has no inter-workgroup
//     synchronisation.
//   phase B (weight update): 64x64 tiles of every W[l] are spread over the
//     workgroups, W[l] += alpha eps[l] f(x_new[l+1])^T contracting over the
//     batch with MFMA, or, for B <= 16, as a rank-B outer product on the VALU.
//
// The phases are separated by a grid barrier (a monotonically increasing
// arrival counter in a caller-provided workspace, every wait bounded by a spin
// limit that raises a flag instead of hanging), so T steps run in one launch.
// Each phase can also be launched on its own (modes PHASE_A / PHASE_B), and
// FORWARD runs the forward initialisation x[l] = W[l] f(x[l+1]) layer by layer
// with the same prediction units as phase A, so the hidden prediction errors
// are exactly 0 after it, as in trainer.py:512-515.
//
// Global loads in the inner loops are branch-free (clamped address, masked
// value) so the compiler can issue several of them before the first wait.
#include "ipc_device.h"
#include "ipc_launch.h"
#include "ipc_narrow.h"

namespace ipc {

namespace {

constexpr int NT = 512;  // threads per workgroup (8 waves)
constexpr int NW = NT / 64;
constexpr int NC = NARROW_NC;
constexpr int WT = 64;  // weight-update tile edge

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
// Every lane loads from an in-bounds address (row[0] when masked), so the
// loads carry no branches.  `vec` (K % KL == 0 and a 16-byte aligned matrix)
// selects 16-byte loads; then a KL-run is either wholly in or wholly out.
template <int KL>
__device__ __forceinline__ void load_run(const float* row, int k, int K, bool ok, bool vec, float* o) {
  if (vec) {
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

template <typename OT, int SPLIT>
struct Narrow {
  using MM = Mma16<OT>;
  static constexpr int KS = MM::KS, KL = MM::KL, PAD = MM::PAD;
  static constexpr bool SA = SPLIT >= 2, SB = SPLIT >= 3;

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

  // f(x[l][:, c0:c0+ncols]) -> fs block of layer l as [n][k], zero for k >= d_l or n >= ncols;
  // with keep_raw the raw values also go to xr (layer l < L).
  __device__ __forceinline__ void stage_layer(int l, int c0, int ncols, bool keep_raw, bool want_f) {
    const int d = p.dims[l], ld = ldk(d), B = p.B, act = p.act;
    const float* X = p.x[l];
    OT* fh = want_f ? fs_hi(l) : nullptr;
    OT* fl = (want_f && SB) ? fs_lo(l) : nullptr;
    float* raw = keep_raw ? xr(l) : nullptr;
    const int rows = want_f ? ld : d;
    for (int i = tid; i < rows * NC; i += NT) {
      const int k = i / NC, n = i - k * NC;
      const bool in = k < d && n < ncols;
      const float v = in ? X[(long long)k * B + c0 + n] : 0.0f;
      if (raw && k < d) raw[k * NC + n] = v;
      if (want_f) {
        const float fv = in ? act_f(act, v) : 0.0f;
        const OT hi = cvt<OT>(fv);
        fh[n * ld + k] = hi;
        if (SB) fl[n * ld + k] = cvt<OT>(fv - to_f32(hi));
      }
    }
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
    const int kpad = round_up(K, KS);
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int kk = 0; kk < kpad; kk += KS) {
      float av[KL];
      load_run<KL>(wrow, kk + lg * KL, K, rok, vec, av);
      OT ah[KL], al[KL], bh[KL], bl[KL];
#pragma unroll
      for (int q = 0; q < KL; ++q) {
        ah[q] = cvt<OT>(av[q]);
        if (SA) al[q] = cvt<OT>(av[q] - to_f32(ah[q]));
        bh[q] = fh[kk + q];
        if (SB) bl[q] = fl[kk + q];
      }
      c = MM::run(ah, bh, c);
      if (SA) c = MM::run(al, bh, c);
      if (SB) c = MM::run(ah, bl, c);
    }
    return c;
  }

  // One inference unit: acc = W[l-1]^T[rt*16 .. +16][:] eps[l-1][:, cols].
  __device__ __forceinline__ f32x4 infer_unit(int l, int rt) {
    const int M = p.dims[l], Kp = p.dims[l - 1], ld = ldk(Kp);
    const float* Wl = p.w[l - 1];  // [Kp][M]
    const int m = rt * 16 + lr;
    const bool mok = m < M;
    const OT* eb = es(l - 1) + lr * ld + lg * KL;
    const int kpad = round_up(Kp, KS);
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
    for (int kk = 0; kk < kpad; kk += KS) {
      OT ah[KL], bh[KL];
#pragma unroll
      for (int q = 0; q < KL; ++q) {
        const int k = kk + lg * KL + q;
        const bool in = mok && k < Kp;
        const float v = Wl[in ? (long long)k * M + m : 0];
        ah[q] = cvt<OT>(in ? v : 0.0f);
        bh[q] = eb[kk + q];
      }
      c = MM::run(ah, bh, c);
    }
    return c;
  }

  // Phase A for column block cb.
  __device__ __forceinline__ void phase_a(int cb) {
    const int B = p.B, L = p.L, c0 = cb * NC, ncols = min(NC, B - c0);
    const float gamma = p.gamma;
    const int act = p.act;
    __syncthreads();  // LDS of the previous column block / phase is free
    // eps blocks are the zero-padded B operands of the inference units
    for (int l = 0; l + 1 < L; ++l) {
      OT* e_l = es(l);
      const int n_el = NC * ldk(p.dims[l]);
      for (int i = tid; i < n_el; i += NT) e_l[i] = cvt<OT>(0.0f);
    }
    for (int l = 0; l <= L; ++l) stage_layer(l, c0, ncols, l < L, l >= 1);
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
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = rt * 16 + lg * 4 + j;
        if (row < M && lr < ncols) {
#pragma clang fp contract(off)
          const long long o = (long long)row * B + c0 + lr;
          const float x = xr(l)[row * NC + lr];
          const float xn = x + gamma * (-ef(l)[row * NC + lr] + act_df(act, x) * c[j]);
          p.x[l][o] = xn;
          if (p.a[l]) p.a[l][o] = act_f(act, xn);
        }
      }
    }
  }

  // Forward initialisation for column block cb: x[l] = W[l] f(x[l+1]), l = L-1 .. 1.
  __device__ __forceinline__ void forward(int cb) {
    const int B = p.B, L = p.L, c0 = cb * NC, ncols = min(NC, B - c0);
    for (int l = L - 1; l >= 1; --l) {
      __syncthreads();
      stage_layer(l + 1, c0, ncols, false, true);
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
      __threadfence_block();
    }
    if (p.a[L]) {
      const int act = p.act;
      for (int i = tid; i < p.dims[L] * NC; i += NT) {
        const int k = i / NC, n = i - k * NC;
        if (n < ncols) p.a[L][(long long)k * B + c0 + n] = act_f(act, p.x[L][(long long)k * B + c0 + n]);
      }
    }
  }

  // Phase B for weight tile `tile`: W[l] tile += alpha eps[l] f(x_new[l+1])^T.
  __device__ __forceinline__ void phase_b(int tile) {
    int l = 0;
    while (l + 1 < p.L && tile >= p.wtile_start[l + 1]) ++l;
    const int M = p.dims[l], N = p.dims[l + 1], B = p.B;
    const int tn = (N + WT - 1) / WT;
    const int local = tile - p.wtile_start[l];
    const int m0 = (local / tn) * WT, n0 = (local % tn) * WT;
    const float* E = p.e[l];
    const bool saved = p.a[l + 1] != nullptr;
    const float* X = saved ? p.a[l + 1] : p.x[l + 1];
    const int act = saved ? (int)ACT_IDENTITY : p.act;
    float* W = p.w[l];
    const float alpha = p.alpha;
    if (p.outer) {
      // rank-B outer product on the VALU (B <= NC)
      float* so_e = reinterpret_cast<float*>(lds);
      float* so_x = so_e + WT * (NC + 1);
      __syncthreads();
      for (int i = tid; i < WT * B; i += NT) {
        const int r = i / B, b = i - r * B;
        so_e[r * (NC + 1) + b] = (m0 + r < M) ? E[(long long)(m0 + r) * B + b] : 0.0f;
        so_x[r * (NC + 1) + b] = (n0 + r < N) ? act_f(act, X[(long long)(n0 + r) * B + b]) : 0.0f;
      }
      __syncthreads();
      for (int i = tid; i < WT * WT; i += NT) {
        const int r = i / WT, c = i - r * WT;
        const int m = m0 + r, n = n0 + c;
        if (m < M && n < N) {
          float s = 0.0f;
          for (int b = 0; b < B; ++b) s += so_e[r * (NC + 1) + b] * so_x[c * (NC + 1) + b];
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
    const int bpad = round_up(B, KS);
#pragma unroll 4
    for (int b0 = 0; b0 < bpad; b0 += KS) {
      float av[KL];
      load_run<KL>(erow, b0 + lg * KL, B, mok, vec, av);
      float xv[2][KL];
#pragma unroll
      for (int s = 0; s < 2; ++s) load_run<KL>(xrow[s], b0 + lg * KL, B, nok[s], vec, xv[s]);
      OT ah[KL];
#pragma unroll
      for (int q = 0; q < KL; ++q) ah[q] = cvt<OT>(av[q]);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        OT bh[KL];
#pragma unroll
        for (int q = 0; q < KL; ++q) {
          const bool in = nok[s] && (b0 + lg * KL + q < B);
          bh[q] = cvt<OT>(in ? act_f(act, xv[s][q]) : 0.0f);
        }
        acc[s] = MM::run(ah, bh, acc[s]);
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

template <typename OT, int SPLIT>
__global__ void __launch_bounds__(NT) narrow_kernel(const NarrowArgs p) {
  using N = Narrow<OT, SPLIT>;
  extern __shared__ __align__(16) char lds[];
  __shared__ NarrowLds layout;
  if (threadIdx.x == 0)
    narrow_lds_layout(p.dims, p.L, N::KS, N::PAD, (int)sizeof(OT), N::SB, layout);
  __syncthreads();
  N k(p, layout, lds);
  const int ncb = (p.B + NC - 1) / NC;
  const int ntile = p.wtile_start[p.L];
  const int nb = gridDim.x;
  if (p.mode == NMODE_FORWARD) {
    for (int cb = blockIdx.x; cb < ncb; cb += nb) k.forward(cb);
    return;
  }
  if (p.mode == NMODE_PHASE_A) {
    for (int cb = blockIdx.x; cb < ncb; cb += nb) k.phase_a(cb);
    return;
  }
  if (p.mode == NMODE_PHASE_B) {
    for (int t = blockIdx.x; t < ntile; t += nb) k.phase_b(t);
    return;
  }
  int nbar = 0;
  for (int s = 0; s < p.steps; ++s) {
    for (int cb = blockIdx.x; cb < ncb; cb += nb) k.phase_a(cb);
    grid_barrier(p.bar, nb, nbar++, p.spin_limit);
    for (int t = blockIdx.x; t < ntile; t += nb) k.phase_b(t);
    if (s + 1 < p.steps) grid_barrier(p.bar, nb, nbar++, p.spin_limit);
  }
  barrier_exit(p.bar, nb);
}

template <typename OT, int SPLIT>
hipError_t set_lds(int bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&narrow_kernel<OT, SPLIT>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

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

hipError_t narrow_prepare(int operand, int split, int lds_bytes) {
  if (operand == DT_F32) return set_lds<float, 1>(lds_bytes);
  if (operand == DT_F16) {
    if (split >= 3) return set_lds<f16, 3>(lds_bytes);
    if (split == 2) return set_lds<f16, 2>(lds_bytes);
    return set_lds<f16, 1>(lds_bytes);
  }
  if (split >= 3) return set_lds<bf16, 3>(lds_bytes);
  if (split == 2) return set_lds<bf16, 2>(lds_bytes);
  return set_lds<bf16, 1>(lds_bytes);
}

hipError_t launch_narrow(const NarrowArgs& p, int operand, int split, hipStream_t s) {
  const dim3 grid(p.nblocks), block(NT);
  const size_t lds = (size_t)p.lds_bytes;
  if (operand == DT_F32) {
    hipLaunchKernelGGL((narrow_kernel<float, 1>), grid, block, lds, s, p);
  } else if (operand == DT_F16) {
    if (split >= 3) hipLaunchKernelGGL((narrow_kernel<f16, 3>), grid, block, lds, s, p);
    else if (split == 2) hipLaunchKernelGGL((narrow_kernel<f16, 2>), grid, block, lds, s, p);
    else hipLaunchKernelGGL((narrow_kernel<f16, 1>), grid, block, lds, s, p);
  } else {
    if (split >= 3) hipLaunchKernelGGL((narrow_kernel<bf16, 3>), grid, block, lds, s, p);
    else if (split == 2) hipLaunchKernelGGL((narrow_kernel<bf16, 2>), grid, block, lds, s, p);
    else hipLaunchKernelGGL((narrow_kernel<bf16, 1>), grid, block, lds, s, p);
  }
  return hipGetLastError();
}

}  // namespace ipc
