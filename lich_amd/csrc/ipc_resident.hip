// ipc_resident.hip - layer-resident whole-step kernel for narrow iPC nets (gfx950).
//
// The column-block whole-step kernel re-reads every W from memory in each
// phase of each step: its grid barriers write back and invalidate the L2, and
// a 64-wide net leaves each of those reads a serial memory round trip.  This
// kernel keeps the weights still instead (reference trainer.py:601-679
// semantics, T steps per launch):
//
//   workgroup l (l = 0 .. L-2) owns W[l] (d_l x d_{l+1}, fp32 master in MFMA
//   result registers, 16-bit hi / lo / transposed operand copies in LDS),
//   x[l] and x[l+1] for the whole batch; the top layer's W[L-1], whose
//   contraction runs over the input width, is split into column chunks and
//   row blocks, one workgroup per chunk and block, every one holding f(x[L])
//   for its chunk (x[L] is clamped).
//
// A step, per workgroup:
//   1. P = W f(x[l+1]) with 16-bit MFMA (one product with unsplit operands,
//      three with split 3: hi*hi + lo*hi + hi*lo), or fp32 MFMA;
//      eps[l] = x[l] - P; g = W[l]^T eps[l] (the inference term of layer l+1)
//      and its product with f'(x[l+1]) of the old state.  Top chunks publish
//      their partial P instead.
//   2. publish eps[l] and f'(x[l+1]) g (16x16 result tiles, one 16-byte
//      record per lane) and raise the workgroup's flag; wait for the flags of
//      the workgroups it exchanges with (the same set both ways, so a
//      double-buffered exchange is safe).
//   3. x[l] += gamma(-eps[l] + f'(x[l]) g[l]) with that product from
//      workgroup l-1 and x[l+1] += gamma(-eps[l+1] + f'(x[l+1]) g) with
//      eps[l+1] from workgroup l+1.  eps[L-1] = x[L-1] minus the top chunks'
//      partials summed in chunk order (per row block); each block's chunk 0
//      hands its rows to workgroup L-2 as one record under a flag of its own.
//      The top workgroups apply x[L-1]'s update one step late (with workgroup
//      L-2's product of the previous step), so they never wait for workgroup
//      L-2's current step.  Both
//      neighbours evaluate every shared state with the same operands in the
//      same order, so their copies stay bit-identical without a second
//      exchange.
//   4. W[l] += alpha eps[l] f(x_new[l+1])^T over the batch with MFMA, operand
//      copies restaged in LDS.
// One flag exchange per step replaces the two grid barriers; W, the states
// and the staged operands never leave the chip between steps.  The launch ends
// by writing e, x, f(x) and W, as the column kernel's multi-step launch does.
// The step flags count steps across launches and are never cleared; operands
// that do not change between launches (the top chunks' f(x[L]) copies, the
// hidden workgroups' f(x[l+1]), the top layer's next first-step partial
// products) are kept in the workspace under a cache generation (load_epoch).
//
// Every wait is bounded by a spin limit that raises the timeout flag shared
// with the column kernel instead of hanging.
#include "ipc_device.h"
#include "ipc_launch.h"
#include "ipc_narrow.h"

namespace ipc {

namespace {

constexpr int NT = 1024;  // threads per workgroup (16 waves)
constexpr int NWV = NT / 64;
constexpr int MAXT = 2;  // output tiles per wave and phase (32 tiles at most)

// MFMA operands per operand type.  Per k-step of KSTEP, lane (r = lane % 16,
// g = lane / 16) supplies the KL consecutive elements k = g * KL .. g * KL +
// KL - 1 of its row (one fragment V); V4 holds four elements for staging.
// 16-bit operands take one 16x16x32 MFMA per k-step.  fp32 operands take four
// 16x16x4 MFMAs, instruction s taking k = 4 g + s from lane group g: the
// order of the column kernel's fp32 products, so both kernels give the same
// bits.
template <typename OT> struct Op;
template <> struct Op<f16> {
  typedef f16x8 V;
  typedef _Float16 V4 __attribute__((ext_vector_type(4)));
  static constexpr int KSTEP = 32, KL = 8;
  __device__ __forceinline__ static f32x4 mma(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Op<bf16> {
  typedef bf16x8 V;
  typedef __bf16 V4 __attribute__((ext_vector_type(4)));
  static constexpr int KSTEP = 32, KL = 8;
  __device__ __forceinline__ static f32x4 mma(V a, V b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Op<float> {
  typedef f32x4 V;
  typedef f32x4 V4;
  static constexpr int KSTEP = 16, KL = 4;
  __device__ __forceinline__ static f32x4 mma(V a, V b, f32x4 c) {
#pragma unroll
    for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
    return c;
  }
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.0f, 0.0f, 0.0f, 0.0f}; }

// floor(n / d) for 0 <= n < 2^21 and inv = 1 / d within one ulp (the
// hardware reciprocal): (n + 0.5) / d is never an integer and lies at least
// 0.5 / d from one, more than the error of inv and of the product, so the
// float quotient truncates to the exact result (a few instructions instead of
// an integer-division sequence).
__device__ __forceinline__ int qdiv(int n, float inv) { return (int)(((float)n + 0.5f) * inv); }

// Global-memory (address space 1) views.  The state and workspace pointers
// arrive through the LDS copy of the argument block, which hides their address
// space; flat accesses would count against the LDS wait counter as well, so
// every LDS wait after one would also wait for memory.
typedef __attribute__((address_space(1))) float gf32;
typedef __attribute__((address_space(1))) f32x4 gf32x4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 gu32x4;
__device__ __forceinline__ gf32* gbl(float* p) { return (gf32*)p; }
__device__ __forceinline__ const gf32* gbl(const float* p) { return (const gf32*)p; }
typedef __attribute__((address_space(1))) char gchar;
// v at byte `off` (32-bit) of a uniform base: the store takes the scalar base
// and the lane's 32-bit offset
__device__ __forceinline__ void st_at(gf32* base, unsigned off, float v) { *(gf32*)((gchar*)base + off) = v; }
// the four values of a result-tile lane (rows `stride` bytes apart) from byte `off`
__device__ __forceinline__ void st4_rows(gf32* base, unsigned off, unsigned stride, f32x4 v) {
#pragma unroll
  for (int q = 0; q < 4; ++q) st_at(base, off + q * stride, v[q]);
}

// A pointer every lane holds the same value of, moved to scalar registers
// (accesses through it then take a 32-bit per-lane offset instead of a 64-bit
// per-lane address).
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
  const unsigned long long v = reinterpret_cast<unsigned long long>(p);
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
  return reinterpret_cast<T*>(((unsigned long long)hi << 32) | lo);
}

// Element idx of a state or weight matrix (a uniform pointer) when `in`,
// else element 0 of it.  The load is issued for every lane, so a wave's loads
// leave together instead of one branch, and one memory latency, each; and
// the value is not masked here, so nothing waits for it before its first use.
// Out-of-range values never reach an output: every use of one (staging,
// errors, stores) checks the range again.
__device__ __forceinline__ float ld_at(const float* m, int idx, bool in) { return gbl(m)[in ? idx : 0]; }

// A block of memory read through a buffer resource (word 3 0x00020000: the
// gfx9 descriptor's 32-bit data format): loads at byte offsets past `bytes`
// return 0 by the hardware's range check, so a load needs neither a range
// test nor a clamped 64-bit address, only a 32-bit offset.  The prologue's
// loads use it: its per-wave instruction count, four waves to a SIMD, sets
// when the last wave's loads leave.  Values outside the matrix's rows and
// columns are never used (every use checks the range again).
struct BufRead {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ BufRead(const void* base, unsigned bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000)) {}
  __device__ __forceinline__ float f32(unsigned off) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  }
  __device__ __forceinline__ u32x4 u128(unsigned off) const { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
};

// An exchange record is one 16x16 result tile stored as every lane's four
// result registers (16 bytes per lane), so each access is one 16-byte load or
// store per lane.
__device__ __forceinline__ f32x4 ld_rec(const float* r) { return *(const gf32x4*)r; }
__device__ __forceinline__ void st_rec(float* r, f32x4 v) { *(gf32x4*)r = v; }

constexpr int PBATCH = 8;  // top-layer partial products loaded per batch

// P_0 + P_1 + ... + P_{C-1} of the exchange record at `off` (partials
// `stride` floats apart), added in chunk order; every load of a batch is
// issued before the first add, so a batch costs one memory latency.
__device__ __forceinline__ f32x4 sum_partials(const float* base, long long stride, int C, int off) {
  f32x4 sum = zero4();
  for (int c0 = 0; c0 < C; c0 += PBATCH) {
    f32x4 v[PBATCH];
#pragma unroll
    for (int u = 0; u < PBATCH; ++u) v[u] = c0 + u < C ? ld_rec(base + (c0 + u) * stride + off) : zero4();
#pragma unroll
    for (int u = 0; u < PBATCH; ++u) {
      if (c0 + u == 0) {
        sum = v[u];
      } else if (c0 + u < C) {
#pragma unroll
        for (int q = 0; q < 4; ++q) sum[q] = sum[q] + v[u][q];
      }
    }
  }
  return sum;
}

// x + gamma(-e + dg) with dg = f'(x) g, evaluated without contraction so that
// every workgroup holding a copy of the state computes the same bits.  f'(x)
// depends on the old state only: the workgroup that computes g = W^T eps holds
// f(x) of that state as well, forms the product (one rounded fp32 multiply)
// and exchanges it in place of g, so its receivers evaluate no f'.
__device__ __forceinline__ float state_update(float x, float e, float dg, float gamma) {
#pragma clang fp contract(off)
  return x + gamma * (-e + dg);
}

__device__ __forceinline__ f32x4 mul4(f32x4 a, f32x4 b) {
  f32x4 c;
#pragma unroll
  for (int q = 0; q < 4; ++q) c[q] = a[q] * b[q];
  return c;
}

// f'(x) given f(x) as well (the value staged for the MFMAs)
template <int ACT>
__device__ __forceinline__ f32x4 dact4_from(f32x4 x, f32x4 f) {
  f32x4 d;
#pragma unroll
  for (int q = 0; q < 4; ++q) d[q] = dact_from_t<ACT>(x[q], f[q]);
  return d;
}

template <typename OT, int SPLIT, int ACT>
struct Resident {
  typedef typename Op<OT>::V V8;
  typedef typename Op<OT>::V4 V4;
  static constexpr bool S3 = SPLIT >= 3;
  static constexpr int KSTEP = Op<OT>::KSTEP, KL = Op<OT>::KL;
  // 16-bit hidden workgroups: the weight update reads eps and f(x) from the
  // inference and prediction operands (eb, fh), and the prediction reads W
  // from the inference operand W^T (wt; split 3: its lo half in wl), all with
  // transposing loads, so their staging writes no [m][b], [k][b] or [m][k]
  // copies (ea, ft, wh)
  static constexpr bool TRH = sizeof(OT) == 2;

  // a * b for the kernel's small non-negative index products (LDS element
  // offsets and tile counts, all well below 2^23): the full-rate 24-bit
  // multiply, where the compiler, unable to bound lane-varying operands times
  // a layout stride, issues the quarter-rate 32-bit one (the fp16 launch of
  // the depth-6 profile: 33.8 -> 32.9 us).  The split-3 instantiations keep
  // the 32-bit multiply: with it they measured 0.35 us faster per launch.
  __device__ __forceinline__ static int m24(int a, int b) {
    if constexpr (S3) return a * b;
    else return __mul24(a, b);
  }

  const ResidentArgs& p;
  OT* lds;
  ResidentLds lay;
  int tid, lane, wave, lr, lg;
  int wg, L, B, l, j, M, K, k0, ldw_g;  // ldw_g: row stride of W[l] in memory
  // top workgroups: row block h (rows row0 .. row0 + M - 1 of W[L-1]); toff: the
  // block's first tile in the layer's exchange records of npr_full tiles
  int h, row0, toff, npr_full;
  // the prologue's operands in memory (from the kernel arguments): x[l],
  // x[l + 1] and f(x[l + 1]) (hidden workgroups), W[l], and a top chunk's
  // input image
  const float *x_g, *xu_g, *fu_g, *w_g;
  char* image_g;
  bool hidden;
  int nbt, n_pred, n_inf, n_upd, ktl, ks_k, ks_m, ks_b;
  float inv_nbt, inv_ktl, inv_B;

  __device__ __forceinline__ Resident(const ResidentArgs& a, char* base, int role)
      : p(a), lds(reinterpret_cast<OT*>(base)), tid(threadIdx.x), lane(threadIdx.x & 63), wave(threadIdx.x >> 6),
        lr(threadIdx.x & 15), lg((threadIdx.x & 63) >> 4) {
    wg = role;
    L = p.L;
    B = p.B;
    hidden = wg < L - 1;
    l = hidden ? wg : L - 1;
    // the layer's argument scalars in one batch of loads with one wait (loaded
    // where first used, they would cost a memory round trip each)
    const int dm = p.dims[l], dk = p.dims[l + 1], din = p.dims[L], kc = p.kc, nch = p.chunks, trows = p.top_rows;
    const long long istride = p.image_stride;
    x_g = p.x[l];
    xu_g = p.x[l + 1];
    fu_g = p.fx[l + 1];
    w_g = p.w[l];
    image_g = p.image;
    asm volatile("" ::"s"(dm), "s"(dk), "s"(din), "s"(kc), "s"(nch), "s"(trows), "s"(istride), "s"(x_g), "s"(xu_g),
                 "s"(fu_g), "s"(w_g), "s"(image_g), "s"(p.flags));
    const int top = hidden ? 0 : wg - (L - 1);
    j = hidden ? 0 : top % nch;
    image_g += (long long)j * istride;
    h = hidden ? 0 : top / nch;
    row0 = h * trows;
    M = hidden ? dm : min(trows, dm - row0);
    k0 = hidden ? 0 : j * kc;
    K = hidden ? dk : min(kc, din - k0);
    ldw_g = dk;
    resident_lds_layout(M, K, B, hidden, S3, (int)sizeof(OT), lay);
    nbt = (B + 15) / 16;
    const int mtl = (M + 15) / 16;
    ktl = (K + 15) / 16;
    n_pred = mtl * nbt;
    toff = (row0 / 16) * nbt;
    npr_full = ((dm + 15) / 16) * nbt;
    n_inf = hidden ? ktl * nbt : 0;
    n_upd = mtl * ktl;
    ks_k = (K + KSTEP - 1) / KSTEP;
    ks_m = (M + KSTEP - 1) / KSTEP;
    ks_b = (B + KSTEP - 1) / KSTEP;
    inv_nbt = __builtin_amdgcn_rcpf((float)nbt);
    inv_ktl = __builtin_amdgcn_rcpf((float)ktl);
    inv_B = __builtin_amdgcn_rcpf((float)B);
  }

  // Re-derives the lane indices from an opaque copy of the thread id: every
  // per-lane address is then recomputed in each step instead of being held
  // in registers across the whole step loop.
  __device__ __forceinline__ void refresh() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    tid = t;
    lane = t & 63;
    lr = t & 15;
    lg = (t & 63) >> 4;
  }

  __device__ __forceinline__ V8 ld8(int off) const { return *reinterpret_cast<const V8*>(lds + off); }

  // Four values rounded to the operand type as one vector (two packed
  // conversions).  The vector is pinned, so the 2-byte stores of single
  // elements take their halves from these registers instead of converting
  // the values a second time.
  __device__ __forceinline__ static V4 cvt4(f32x4 v) {
    V4 h = V4{cvt<OT>(v[0]), cvt<OT>(v[1]), cvt<OT>(v[2]), cvt<OT>(v[3])};
    asm("" : "+v"(h));
    return h;
  }
  // the lo terms cvt(v - hi) of a split operand
  __device__ __forceinline__ static V4 cvt4_lo(f32x4 v, V4 h) {
    return cvt4(f32x4{v[0] - to_f32(h[0]), v[1] - to_f32(h[1]), v[2] - to_f32(h[2]), v[3] - to_f32(h[3])});
  }

  // f(v) as 16-bit hi (and lo) terms into the prediction B operand [b][k] and
  // hi into the weight-update B operand [k][b]; (k, b) outside K x B is left
  // zero.  Returns f(v).
  __device__ __forceinline__ float stage_f(int k, int b, float v) {
    const float f = act_t<ACT>(v);
    if (k < K && b < B) {
      const OT hi = cvt<OT>(f);
      lds[lay.fh + m24(b, lay.ldf) + k] = hi;
      if (S3) lds[lay.fl + m24(b, lay.ldf) + k] = cvt<OT>(f - to_f32(hi));
      lds[lay.ft + m24(k, lay.ldft) + b] = hi;
    }
    return f;
  }

  // The same for the four rows r0 .. r0 + 3 (r0 a multiple of 4) of column b
  // that one lane holds of a result tile: they are contiguous in the [b][k]
  // block, written with one 8-byte store each when all four exist.
  __device__ __forceinline__ f32x4 stage_f4(int r0, int b, f32x4 v) {
    f32x4 f;
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = act_t<ACT>(v[q]);
    return stage_fv4(r0, b, f);
  }

  // The same with f(v) given (its operand terms only).
  __device__ __forceinline__ f32x4 stage_fv4(int r0, int b, f32x4 f) {
    const V4 hi = cvt4(f);
    V4 lo;
    if (S3) lo = cvt4_lo(f, hi);
    if (b < B) {
      if (r0 + 4 <= K) {
        *reinterpret_cast<V4*>(lds + lay.fh + m24(b, lay.ldf) + r0) = hi;
        if (S3) *reinterpret_cast<V4*>(lds + lay.fl + m24(b, lay.ldf) + r0) = lo;
        if (!TRH)
#pragma unroll
          for (int q = 0; q < 4; ++q) lds[lay.ft + m24(r0 + q, lay.ldft) + b] = hi[q];
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (r0 + q < K) {
            lds[lay.fh + m24(b, lay.ldf) + r0 + q] = hi[q];
            if (S3) lds[lay.fl + m24(b, lay.ldf) + r0 + q] = lo[q];
            if (!TRH) lds[lay.ft + m24(r0 + q, lay.ldft) + b] = hi[q];
          }
      }
    }
    return f;
  }

  // stage_f4 for a lane whose four rows (r0 + 4 <= K) and column (b < B) all
  // exist: the same values and stores, without the tests.
  __device__ __forceinline__ f32x4 stage_f4_full(int r0, int b, f32x4 v) {
    f32x4 f;
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = act_t<ACT>(v[q]);
    const V4 hi = cvt4(f);
    *reinterpret_cast<V4*>(lds + lay.fh + m24(b, lay.ldf) + r0) = hi;
    if (S3) *reinterpret_cast<V4*>(lds + lay.fl + m24(b, lay.ldf) + r0) = cvt4_lo(f, hi);
    if (!TRH)
#pragma unroll
      for (int q = 0; q < 4; ++q) lds[lay.ft + m24(r0 + q, lay.ldft) + b] = hi[q];
    return f;
  }

  // stage_e4 for a lane whose four rows (r0 + 4 <= M) and column (b < B) all exist.
  __device__ __forceinline__ void stage_e4_full(int r0, int b, f32x4 e) {
    const V4 eo = cvt4(e);
    *reinterpret_cast<V4*>(lds + lay.eb + m24(b, lay.lde) + r0) = eo;
    if (!TRH)
#pragma unroll
      for (int q = 0; q < 4; ++q) lds[lay.ea + m24(r0 + q, lay.lda) + b] = eo[q];
  }

  // eps rows r0 .. r0 + 3 of column b (zero outside M x B) into the inference
  // B operand [b][m] (contiguous) and the weight-update A operand [m][b].
  __device__ __forceinline__ void stage_e4(int r0, int b, f32x4 e) {
    if (b >= B) return;
    const V4 eo = cvt4(e);
    if (r0 + 4 <= M) {
      *reinterpret_cast<V4*>(lds + lay.eb + m24(b, lay.lde) + r0) = eo;
      if (!TRH)
#pragma unroll
        for (int q = 0; q < 4; ++q) lds[lay.ea + m24(r0 + q, lay.lda) + b] = eo[q];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (r0 + q < M) {
          lds[lay.eb + m24(b, lay.lde) + r0 + q] = eo[q];
          if (!TRH) lds[lay.ea + m24(r0 + q, lay.lda) + b] = eo[q];
        }
    }
  }

  // W rows m0 .. m0 + 3 of column k (the four values of one update-tile lane)
  // into the operand copies; the transposed copy [k][m] takes them with one
  // 8-byte store when all four rows exist.
  __device__ __forceinline__ void stage_w4(int m0, int k, f32x4 w) {
    if (k >= K) return;
    const V4 hi = cvt4(w);
    V4 lo;
    if (S3) lo = cvt4_lo(w, hi);
    const bool tr = TRH && hidden;  // (W^T copies only; lo in wt's layout)
    if (!tr)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (m0 + q < M) {
          lds[lay.wh + m24(m0 + q, lay.ldw) + k] = hi[q];
          if (S3) lds[lay.wl + m24(m0 + q, lay.ldw) + k] = lo[q];
        }
      }
    if (hidden) {
      if (m0 + 4 <= M) {
        *reinterpret_cast<V4*>(lds + lay.wt + m24(k, lay.ldwt) + m0) = hi;
        if (S3 && tr) *reinterpret_cast<V4*>(lds + lay.wl + m24(k, lay.ldwt) + m0) = lo;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (m0 + q < M) {
            lds[lay.wt + m24(k, lay.ldwt) + m0 + q] = hi[q];
            if (S3 && tr) lds[lay.wl + m24(k, lay.ldwt) + m0 + q] = lo[q];
          }
      }
    }
  }

  // stage_w4 of a hidden workgroup for a lane whose four rows (m0 + 4 <= M)
  // and column (k < K) all exist: the same values and stores, without the tests.
  __device__ __forceinline__ void stage_w4_full(int m0, int k, f32x4 w) {
    const V4 hi = cvt4(w);
    V4 lo;
    if (S3) lo = cvt4_lo(w, hi);
    if (!TRH)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        lds[lay.wh + m24(m0 + q, lay.ldw) + k] = hi[q];
        if (S3) lds[lay.wl + m24(m0 + q, lay.ldw) + k] = lo[q];
      }
    *reinterpret_cast<V4*>(lds + lay.wt + m24(k, lay.ldwt) + m0) = hi;
    if (S3 && TRH) *reinterpret_cast<V4*>(lds + lay.wl + m24(k, lay.ldwt) + m0) = lo;
  }

  // W element (m, k) of the block into its operand copies.
  __device__ __forceinline__ void stage_w(int m, int k, float w) {
    const OT hi = cvt<OT>(w);
    lds[lay.wh + m24(m, lay.ldw) + k] = hi;
    if (S3) lds[lay.wl + m24(m, lay.ldw) + k] = cvt<OT>(w - to_f32(hi));
    if (hidden) lds[lay.wt + m24(k, lay.ldwt) + m] = hi;
  }

  // Tile t of a [rows][B] matrix: row of result element i of this lane, and its column.
  __device__ __forceinline__ int trow(int t, int i) const { return qdiv(t, inv_nbt) * 16 + 4 * lg + i; }
  __device__ __forceinline__ int tcol(int t) const { return (t - m24(qdiv(t, inv_nbt), nbt)) * 16 + lr; }
  // update tile t: row tile over M, column tile over K
  __device__ __forceinline__ int urt(int t) const { return qdiv(t, inv_ktl); }
  __device__ __forceinline__ int uct(int t) const { return t - m24(qdiv(t, inv_ktl), ktl); }
  __device__ __forceinline__ int rec(int t) const { return t * RES_TILE + lane * 4; }

  // acc = W_block f(x upper) for prediction tile t
  __device__ __forceinline__ f32x4 pred_tile(int t) const {
    const int rt = qdiv(t, inv_nbt), ct = t - m24(rt, nbt);
    const int a0 = m24(rt * 16 + lr, lay.ldw) + lg * KL;
    const int b0 = m24(ct * 16 + lr, lay.ldf) + lg * KL;
    f32x4 c = zero4();
    for (int ks = 0; ks < ks_k; ++ks) {
      const V8 ah = ld8(lay.wh + a0 + ks * KSTEP);
      const V8 bh = ld8(lay.fh + b0 + ks * KSTEP);
      c = Op<OT>::mma(ah, bh, c);
      if (S3) {
        const V8 al = ld8(lay.wl + a0 + ks * KSTEP);
        const V8 bl = ld8(lay.fl + b0 + ks * KSTEP);
        c = Op<OT>::mma(al, bh, c);
        c = Op<OT>::mma(ah, bl, c);
      }
    }
    return c;
  }

  // acc = W^T eps for inference tile t (rows over K)
  __device__ __forceinline__ f32x4 infer_tile(int t) const {
    const int rt = qdiv(t, inv_nbt), ct = t - m24(rt, nbt);
    const int a0 = lay.wt + m24(rt * 16 + lr, lay.ldwt) + lg * KL;
    const int b0 = lay.eb + m24(ct * 16 + lr, lay.lde) + lg * KL;
    f32x4 c = zero4();
    for (int ks = 0; ks < ks_m; ++ks) c = Op<OT>::mma(ld8(a0 + ks * KSTEP), ld8(b0 + ks * KSTEP), c);
    return c;
  }

  // acc = eps f(x upper)^T over the batch as a rank-B outer product on the
  // VALU (fp32 operands, B <= NARROW_OUTER_MAX_B): each of the lane's four
  // sums runs over b = 0 .. B-1 with fused multiply-adds from zero, as the
  // column kernel's rank-B update does.
  __device__ __forceinline__ f32x4 outer_tile(int t) const {
    const int c = uct(t) * 16 + lr, r0 = urt(t) * 16 + 4 * lg;
    const OT* fr = lds + lay.ft + m24(c, lay.ldft);
    f32x4 acc = zero4();
    for (int b = 0; b < B; ++b) {
      const float f = to_f32(fr[b]);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = __builtin_fmaf(to_f32(lds[lay.ea + m24(r0 + q, lay.lda) + b]), f, acc[q]);
    }
    return acc;
  }

  // acc = eps f(x upper)^T over the batch for update tile t (rows over M, columns over K)
  __device__ __forceinline__ f32x4 update_tile(int t) const {
    if (p.outer) return outer_tile(t);
    const int rt = urt(t), ct = uct(t);
    const int a0 = lay.ea + m24(rt * 16 + lr, lay.lda) + lg * KL;
    const int b0 = lay.ft + m24(ct * 16 + lr, lay.ldft) + lg * KL;
    f32x4 c = zero4();
    int ks = 0;
    if constexpr (!S3) {
      // four k-steps' fragments read before their MFMAs (one LDS latency
      // instead of four; the same MFMA sequence)
      for (; ks + 4 <= ks_b; ks += 4) {
        V8 a[4], b[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          a[u] = ld8(a0 + (ks + u) * KSTEP);
          b[u] = ld8(b0 + (ks + u) * KSTEP);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) c = Op<OT>::mma(a[u], b[u], c);
      }
    }
    for (; ks < ks_b; ++ks) c = Op<OT>::mma(ld8(a0 + ks * KSTEP), ld8(b0 + ks * KSTEP), c);
    return c;
  }

  // Eight consecutive contraction rows b0 .. b0 + 7 of column c of a [b][c]
  // 16-bit block (row stride ld elements) as one MFMA fragment, through two
  // transposing loads: each 16-lane group reads a 4 x 16 block, lane i the
  // 8-byte piece of row i / 4 and columns 4 (i % 4) .. 4 (i % 4) + 3, and
  // gets column i of it back.  `off`: the lane's piece in rows b0 .. b0 + 3
  // (rows b0 + 4 .. b0 + 7 are 4 ld further).
  __device__ __forceinline__ V8 ld8_tr(int off, int ld) const {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + off));
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + off + 4 * ld));
    return __builtin_bit_cast(V8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // update_tile of a hidden workgroup.  16-bit operands: eps from eb [b][m]
  // and f(x) from fh [b][k] through transposing loads, the same fragment
  // values and MFMA sequence as from ea and ft (lane (g, r) gets rows
  // 8g .. 8g + 7 of column r in both forms).
  __device__ __forceinline__ f32x4 update_tile_h(int t) const {
    if constexpr (!TRH) {
      return update_tile(t);
    } else {
      const int rt = urt(t), ct = uct(t);
      const int brow = 8 * lg + (lr >> 2), col = 4 * (lr & 3);
      const int a0 = lay.eb + m24(brow, lay.lde) + rt * 16 + col;
      const int b0 = lay.fh + m24(brow, lay.ldf) + ct * 16 + col;
      const int sa = KSTEP * lay.lde, sb = KSTEP * lay.ldf;  // one k-step further
      f32x4 c = zero4();
      int ks = 0;
      if constexpr (!S3) {
        // two k-steps' fragments read before their MFMAs (four need more
        // registers than the loop has)
        for (; ks + 2 <= ks_b; ks += 2) {
          V8 a[2], b[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            a[u] = ld8_tr(a0 + (ks + u) * sa, lay.lde);
            b[u] = ld8_tr(b0 + (ks + u) * sb, lay.ldf);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) c = Op<OT>::mma(a[u], b[u], c);
        }
      }
      for (; ks < ks_b; ++ks) c = Op<OT>::mma(ld8_tr(a0 + ks * sa, lay.lde), ld8_tr(b0 + ks * sb, lay.ldf), c);
      return c;
    }
  }

  // pred_tile / pred_tiles of a hidden workgroup.  16-bit operands: the W
  // fragments (row m, eight consecutive k) read transposed from W^T (wt, and
  // wl for the lo half), the same values and MFMA sequence as from [m][k]
  // copies.  wtr: the lane's piece of row tile rt in k-step 0.
  __device__ __forceinline__ int wtr(int rt) const {
    return m24(8 * lg + (lr >> 2), lay.ldwt) + rt * 16 + 4 * (lr & 3);
  }
  __device__ __forceinline__ f32x4 pred_tile_h(int t) const {
    if constexpr (!TRH) {
      return pred_tile(t);
    } else {
      const int rt = qdiv(t, inv_nbt), ct = t - m24(rt, nbt);
      const int a0 = wtr(rt), sa = KSTEP * lay.ldwt;
      const int b0 = m24(ct * 16 + lr, lay.ldf) + lg * KL;
      f32x4 c = zero4();
      for (int ks = 0; ks < ks_k; ++ks) {
        const V8 ah = ld8_tr(lay.wt + a0 + ks * sa, lay.ldwt);
        const V8 bh = ld8(lay.fh + b0 + ks * KSTEP);
        c = Op<OT>::mma(ah, bh, c);
        if (S3) {
          const V8 al = ld8_tr(lay.wl + a0 + ks * sa, lay.ldwt);
          const V8 bl = ld8(lay.fl + b0 + ks * KSTEP);
          c = Op<OT>::mma(al, bh, c);
          c = Op<OT>::mma(ah, bl, c);
        }
      }
      return c;
    }
  }
  __device__ __forceinline__ void pred_tiles_h(int n, f32x4 (&c)[MAXT]) const {
    if constexpr (!TRH) {
      pred_tiles(n, c);
    } else {
      const int t0 = wave, t1 = wave + NWV;
      if (t1 < n && NWV % nbt == 0) {
        const int rt0 = qdiv(t0, inv_nbt), ct = t0 - m24(rt0, nbt), rt1 = rt0 + NWV / nbt;
        const int a0 = wtr(rt0), a1 = wtr(rt1), sa = KSTEP * lay.ldwt;
        const int b0 = m24(ct * 16 + lr, lay.ldf) + lg * KL;
        f32x4 c0 = zero4(), c1 = zero4();
        int ks = 0;
        if constexpr (!S3) {
          for (; ks + 2 <= ks_k; ks += 2) {
            V8 bh[2], ah0[2], ah1[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              bh[u] = ld8(lay.fh + b0 + (ks + u) * KSTEP);
              ah0[u] = ld8_tr(lay.wt + a0 + (ks + u) * sa, lay.ldwt);
              ah1[u] = ld8_tr(lay.wt + a1 + (ks + u) * sa, lay.ldwt);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              c0 = Op<OT>::mma(ah0[u], bh[u], c0);
              c1 = Op<OT>::mma(ah1[u], bh[u], c1);
            }
          }
        }
        for (; ks < ks_k; ++ks) {
          const V8 bh = ld8(lay.fh + b0 + ks * KSTEP);
          const V8 ah0 = ld8_tr(lay.wt + a0 + ks * sa, lay.ldwt), ah1 = ld8_tr(lay.wt + a1 + ks * sa, lay.ldwt);
          c0 = Op<OT>::mma(ah0, bh, c0);
          c1 = Op<OT>::mma(ah1, bh, c1);
          if (S3) {
            const V8 bl = ld8(lay.fl + b0 + ks * KSTEP);
            const V8 al0 = ld8_tr(lay.wl + a0 + ks * sa, lay.ldwt), al1 = ld8_tr(lay.wl + a1 + ks * sa, lay.ldwt);
            c0 = Op<OT>::mma(al0, bh, c0);
            c1 = Op<OT>::mma(al1, bh, c1);
            c0 = Op<OT>::mma(ah0, bl, c0);
            c1 = Op<OT>::mma(ah1, bl, c1);
          }
        }
        c[0] = c0;
        c[1] = c1;
      } else {
        c[0] = t0 < n ? pred_tile_h(t0) : zero4();
        c[1] = t1 < n ? pred_tile_h(t1) : zero4();
      }
    }
  }

  // The wave's tiles t = wave and wave + NWV of a [rows][cols] tiling with
  // `nct` column tiles lie in the same column tile when nct divides NWV.  The
  // paired forms below then read every B fragment from LDS once for both
  // tiles and run the two accumulation chains interleaved; each accumulator
  // still sees exactly the MFMA sequence of the single-tile form.
  static_assert(MAXT == 2, "the paired tile forms cover two tiles per wave");

  __device__ __forceinline__ void pred_tiles(int n, f32x4 (&c)[MAXT]) const {
    const int t0 = wave, t1 = wave + NWV;
    if (t1 < n && NWV % nbt == 0) {
      const int rt0 = qdiv(t0, inv_nbt), ct = t0 - m24(rt0, nbt), rt1 = rt0 + NWV / nbt;
      const int a0 = m24(rt0 * 16 + lr, lay.ldw) + lg * KL, a1 = m24(rt1 * 16 + lr, lay.ldw) + lg * KL;
      const int b0 = m24(ct * 16 + lr, lay.ldf) + lg * KL;
      f32x4 c0 = zero4(), c1 = zero4();
      int ks = 0;
      if constexpr (!S3) {
        // two k-steps' fragments read before their MFMAs (the same sequence)
        for (; ks + 2 <= ks_k; ks += 2) {
          V8 bh[2], ah0[2], ah1[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            bh[u] = ld8(lay.fh + b0 + (ks + u) * KSTEP);
            ah0[u] = ld8(lay.wh + a0 + (ks + u) * KSTEP);
            ah1[u] = ld8(lay.wh + a1 + (ks + u) * KSTEP);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            c0 = Op<OT>::mma(ah0[u], bh[u], c0);
            c1 = Op<OT>::mma(ah1[u], bh[u], c1);
          }
        }
      }
      for (; ks < ks_k; ++ks) {
        const V8 bh = ld8(lay.fh + b0 + ks * KSTEP);
        const V8 ah0 = ld8(lay.wh + a0 + ks * KSTEP), ah1 = ld8(lay.wh + a1 + ks * KSTEP);
        c0 = Op<OT>::mma(ah0, bh, c0);
        c1 = Op<OT>::mma(ah1, bh, c1);
        if (S3) {
          const V8 bl = ld8(lay.fl + b0 + ks * KSTEP);
          const V8 al0 = ld8(lay.wl + a0 + ks * KSTEP), al1 = ld8(lay.wl + a1 + ks * KSTEP);
          c0 = Op<OT>::mma(al0, bh, c0);
          c1 = Op<OT>::mma(al1, bh, c1);
          c0 = Op<OT>::mma(ah0, bl, c0);
          c1 = Op<OT>::mma(ah1, bl, c1);
        }
      }
      c[0] = c0;
      c[1] = c1;
    } else {
      c[0] = t0 < n ? pred_tile(t0) : zero4();
      c[1] = t1 < n ? pred_tile(t1) : zero4();
    }
  }

  __device__ __forceinline__ void infer_tiles(int n, f32x4 (&c)[MAXT]) const {
    const int t0 = wave, t1 = wave + NWV;
    if (t1 < n && NWV % nbt == 0) {
      const int rt0 = qdiv(t0, inv_nbt), ct = t0 - m24(rt0, nbt), rt1 = rt0 + NWV / nbt;
      const int a0 = lay.wt + m24(rt0 * 16 + lr, lay.ldwt) + lg * KL, a1 = lay.wt + m24(rt1 * 16 + lr, lay.ldwt) + lg * KL;
      const int b0 = lay.eb + m24(ct * 16 + lr, lay.lde) + lg * KL;
      f32x4 c0 = zero4(), c1 = zero4();
      int ks = 0;
      if constexpr (!S3) {
        for (; ks + 2 <= ks_m; ks += 2) {
          V8 b[2], x0[2], x1[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            b[u] = ld8(b0 + (ks + u) * KSTEP);
            x0[u] = ld8(a0 + (ks + u) * KSTEP);
            x1[u] = ld8(a1 + (ks + u) * KSTEP);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            c0 = Op<OT>::mma(x0[u], b[u], c0);
            c1 = Op<OT>::mma(x1[u], b[u], c1);
          }
        }
      }
      for (; ks < ks_m; ++ks) {
        const V8 b = ld8(b0 + ks * KSTEP);
        c0 = Op<OT>::mma(ld8(a0 + ks * KSTEP), b, c0);
        c1 = Op<OT>::mma(ld8(a1 + ks * KSTEP), b, c1);
      }
      c[0] = c0;
      c[1] = c1;
    } else {
      c[0] = t0 < n ? infer_tile(t0) : zero4();
      c[1] = t1 < n ? infer_tile(t1) : zero4();
    }
  }

  __device__ __forceinline__ void update_tiles(int n, f32x4 (&c)[MAXT]) const {
    const int t0 = wave, t1 = wave + NWV;
    if (!p.outer && t1 < n && NWV % ktl == 0) {
      const int rt0 = urt(t0), ct = t0 - m24(rt0, ktl), rt1 = rt0 + NWV / ktl;
      const int a0 = lay.ea + m24(rt0 * 16 + lr, lay.lda) + lg * KL, a1 = lay.ea + m24(rt1 * 16 + lr, lay.lda) + lg * KL;
      const int b0 = lay.ft + m24(ct * 16 + lr, lay.ldft) + lg * KL;
      f32x4 c0 = zero4(), c1 = zero4();
      for (int ks = 0; ks < ks_b; ++ks) {
        const V8 b = ld8(b0 + ks * KSTEP);
        c0 = Op<OT>::mma(ld8(a0 + ks * KSTEP), b, c0);
        c1 = Op<OT>::mma(ld8(a1 + ks * KSTEP), b, c1);
      }
      c[0] = c0;
      c[1] = c1;
    } else {
      c[0] = t0 < n ? update_tile(t0) : zero4();
      c[1] = t1 < n ? update_tile(t1) : zero4();
    }
  }
};

// Publishes step `value` for this workgroup: every store of the workgroup
// before it becomes visible at agent scope before the flag does (the barrier
// orders the other waves' stores before thread 0's release fence, which
// writes back L2, and the fence orders them before the relaxed flag store).
__device__ __forceinline__ void publish(unsigned* flag, unsigned value) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Waits until every peer's flag reaches `value`, the last `n_prev` peers'
// flags `value - 1` (one lane of wave 0 per peer, relaxed polls, then one
// acquire fence, which invalidates L2, pairing with the publishers' release
// fences).  The flags count steps across launches, so they are compared as a
// difference, which stays right when the count wraps around.
__device__ __forceinline__ void wait_peers(const ResidentArgs& p, const int* peers, int npeers, unsigned value,
                                           int n_prev = 0, bool acquire = true) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const unsigned* f = lane < npeers ? &p.flags[peers[lane]] : nullptr;
    const unsigned want = lane < npeers - n_prev ? value : value - 1u;
    int spins = 0;
    while (true) {
      bool ok = true;
      if (f) ok = (int)(__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - want) >= 0;
      if (__all(ok)) break;
      __builtin_amdgcn_s_sleep(1);
      if (++spins > p.spin_limit) {
        if (lane == 0) __hip_atomic_store(&p.bar[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    if (acquire) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// Four exchange records (16 bytes per lane each) read coherently at agent
// scope: SC1 loads are served from the device's coherence point, never from a
// line the reader's L2 may hold from before, the same coherence the flag polls
// rely on.  The writer's release fence has written its records back before its
// flag went up, and these loads leave only after the flag was seen, so no
// acquire fence (an invalidation of the whole L2) is needed before them.  One
// block that waits for all four: no load stays in flight past it.
// (Two scalar bases, each with two 32-bit byte offsets.)
__device__ __forceinline__ void ld_rec4_sc1(const float* b0, unsigned o0, unsigned o1, const float* b1, unsigned o2,
                                            unsigned o3, f32x4& v0, f32x4& v1, f32x4& v2, f32x4& v3) {
  asm volatile(
      "global_load_dwordx4 %0, %4, %8 sc1\n\t"
      "global_load_dwordx4 %1, %5, %8 sc1\n\t"
      "global_load_dwordx4 %2, %6, %9 sc1\n\t"
      "global_load_dwordx4 %3, %7, %9 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
      : "v"(o0), "v"(o1), "v"(o2), "v"(o3), "s"(b0), "s"(b1)
      : "memory");
}

// The flags area across launches.  Step flags are never cleared: every
// workgroup publishes once per step, so at the start of a launch they all
// hold the same count, the workgroup's own flag gives it, and the launch
// publishes and waits for base + s + 1.  Word RES_MAX_WG is a generation,
// bumped when cached operands go stale (the forward initialisation, which may
// change x[L], and ipc_plan_sync); word RES_MAX_WG + 1 + wg holds generation
// + 1 once workgroup wg's cached operands (a top chunk's input image, a hidden
// workgroup's f(x[l+1]) in fx[l+1]) belong to the current generation.  Each
// workgroup reads and writes only its own slot, at its start and end, so no
// workgroup has to know that it is the last one out.
struct Epoch {
  unsigned base, gen;
  bool warm;
};
__device__ __forceinline__ Epoch load_epoch(const ResidentArgs& a, int wg) {
  Epoch e;
  e.base = __hip_atomic_load(&a.flags[wg], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  e.gen = __hip_atomic_load(&a.flags[RES_MAX_WG], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  e.warm = __hip_atomic_load(&a.flags[RES_MAX_WG + 1 + wg], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == e.gen + 1u;
  return e;
}
// At the end of a launch (read by the next one, after the kernel boundary).
__device__ __forceinline__ void mark_cached(const ResidentArgs& a, int wg, const Epoch& e) {
  if (threadIdx.x == 0 && a.steps > 0)
    __hip_atomic_store(&a.flags[RES_MAX_WG + 1 + wg], e.gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch set-up, run while the workgroup's first state and weight loads are
// in flight: zeros in the operand regions when the block does not fill them (a
// dimension off the MFMA k-step or the 16-row tile leaves padding that the
// MFMAs read), then a barrier, so the staging writes that follow land after
// the zeros.
template <typename OT, int SPLIT, int ACT>
__device__ __forceinline__ void setup(const Resident<OT, SPLIT, ACT>& k) {
  if ((k.M | k.K | k.B) & (Resident<OT, SPLIT, ACT>::KSTEP - 1)) {
    uint4* z = reinterpret_cast<uint4*>(k.lds);
    for (int i = threadIdx.x; i < k.lay.bytes / 16; i += NT) z[i] = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
  }
}

// The end of the prologue, once the staging writes are issued: the LDS copy
// of the argument block (its words were loaded at entry and have arrived with
// the prologue's own loads) and the list of workgroups this one exchanges
// with, in both directions (thread 0, while the other waves finish staging),
// then the barrier that publishes them and the staged operands.
template <typename OT, int SPLIT, int ACT>
__device__ __forceinline__ void end_prologue(const Resident<OT, SPLIT, ACT>& k, ResidentArgs& p, int aword, int* peers,
                                             int& npeers) {
  if (threadIdx.x < sizeof(ResidentArgs) / 4) reinterpret_cast<int*>(&p)[threadIdx.x] = aword;
  static_assert(offsetof(ResidentArgs, halves) / 4 < 64, "wave 0 holds the scalars of the peer list");
  // wave 0's lanes hold the argument block's first 64 words (their share of
  // the copy): the scalars come from there instead of a memory load
  const int C = __builtin_amdgcn_readlane(aword, offsetof(ResidentArgs, chunks) / 4);
  const int halves = __builtin_amdgcn_readlane(aword, offsetof(ResidentArgs, halves) / 4);
  const int nwg = __builtin_amdgcn_readlane(aword, offsetof(ResidentArgs, nwg) / 4);
  if (threadIdx.x == 0) {
    const int L = k.L, top0 = L - 1;
    int n = 0;
    if (k.hidden) {
      if (k.l >= 1) peers[n++] = k.l - 1;
      if (k.l + 1 <= L - 2) {
        peers[n++] = k.l + 1;
      } else {
        // next to the top layer: each row block's chunk-0 eps[L-1] flag (published
        // only after the block's other chunks have published, so it also covers
        // their progress)
        for (int hh = 0; hh < halves; ++hh) peers[n++] = nwg + hh;
      }
    } else {
      // the siblings in the row block, then workgroup L-2 (waited for one step behind)
      for (int c = 0; c < C; ++c)
        if (c != k.j) peers[n++] = top0 + k.h * C + c;
      peers[n++] = L - 2;
    }
    npeers = n;
  }
  __syncthreads();
}

// The states a hidden workgroup leaves after the last step: eps[l]; x[l]
// (l >= 1); f(x[l+1]) from the values staged for the weight update (workgroup
// l + 1 holds the same x[l+1], so each f(x) is written once and no activation
// is evaluated again); and, next to the top layer, x[L-1], whose last update
// the top workgroups leave to this one (they apply each step's update one step
// late).
template <typename OT, int SPLIT, int ACT>
__device__ __forceinline__ void write_states(Resident<OT, SPLIT, ACT>& k, const ResidentArgs& p,
                                             const f32x4* ea, const f32x4* xa, const f32x4* xb, const f32x4* fb) {
  // (uniform base pointers and 32-bit byte offsets, so that each store takes
  // the lane's offset and the scalar base: one offset per tile, the rows a
  // uniform stride apart; rows are checked one by one only where a tile's
  // four rows do not all exist)
  // (x[l] is written for l >= 1, x[l+1] next to the top layer; the flags are
  // uniform, the pointers always valid)
  const int l = k.l, B = k.B, wave = k.wave;
  const bool wx = l >= 1, wxu = l + 1 == k.L - 1, wfu = p.fx[l + 1] != nullptr;
  gf32* E = gbl(uniform(p.e[l]));
  gf32* X = gbl(uniform(p.x[l]));
  gf32* XU = gbl(uniform(p.x[l + 1]));
  gf32* FU = gbl(uniform(p.fx[l + 1]));
  const unsigned rs = (unsigned)B * 4u;  // bytes between rows
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    const int t = wave + NWV * i;
    if (t < k.n_pred) {
      const int b = k.tcol(t), r0 = k.trow(t, 0);
      const unsigned o = (unsigned)(r0 * B + b) * 4u;
      if (r0 + 4 <= k.M && b < B) {
        st4_rows(E, o, rs, ea[i]);
        if (wx) st4_rows(X, o, rs, xa[i]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (r0 + q < k.M && b < B) {
            st_at(E, o + q * rs, ea[i][q]);
            if (wx) st_at(X, o + q * rs, xa[i][q]);
          }
      }
    }
    if (t < k.n_inf) {
      const int b = k.tcol(t), r0 = k.trow(t, 0);
      const unsigned o = (unsigned)(r0 * B + b) * 4u;
      if (r0 + 4 <= k.K && b < B) {
        if (wfu) st4_rows(FU, o, rs, fb[i]);
        if (wxu) st4_rows(XU, o, rs, xb[i]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (r0 + q < k.K && b < B) {
            if (wfu) st_at(FU, o + q * rs, fb[i][q]);
            if (wxu) st_at(XU, o + q * rs, xb[i][q]);
          }
      }
    }
  }
}

// Hidden layer l (0 <= l <= L-2): W[l] at the update tiles, x[l] at the
// prediction tiles, x[l+1] at the inference tiles, all resident for the launch.
template <typename OT, int SPLIT, int ACT>
__device__ __forceinline__ void run_hidden(Resident<OT, SPLIT, ACT>& k, ResidentArgs& p, int* peers,
                                           int& npeers_lds, int aword) {
  constexpr int MU = 1;  // update tiles per wave: d_l x d_{l+1} <= 64 x 64 is at most 16 tiles
  // (scalars from the kernel arguments: the LDS copy p is published by setup)
  const int L = k.L, B = k.B, C = k.p.chunks, l = k.l, wave = k.wave, lg = k.lg, lr = k.lr;
  const int npr = k.n_pred, ninf = k.n_inf;
  const float gamma = k.p.gamma, alpha = k.p.alpha;
  // fb: f(x[l+1]) as staged for the MFMAs, reused for the next step's f'(x[l+1])
  f32x4 xa[MAXT], ea[MAXT], xb[MAXT], gb[MAXT], fb[MAXT], wr[MU];
  // f(x[l+1]) as this workgroup left it in fx[l+1] at the end of the previous
  // launch (the same bits as evaluating it again) is used when that belongs to
  // the current generation; it is loaded with the states either way
  const Epoch ep = load_epoch(k.p, k.wg);
  const bool warm = ep.warm;
  f32x4 fu[MAXT];
  // (a tile index past the tile count maps to rows past the matrix, which
  // the buffers' range checks return as zeros; rows 4 lg + q and column lr of
  // a tile: one 32-bit offset per lane, the tile's corner and q uniform)
  {
    const BufRead bx0(k.x_g, k.M * B * 4), bx1(k.xu_g, k.K * B * 4), bf1(k.fu_g, k.K * B * 4);
    const unsigned lane_x = (unsigned)(4 * lg * B + lr) * 4u;
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      ea[i] = zero4(); gb[i] = zero4(); fb[i] = zero4();
      const int rt = __builtin_amdgcn_readfirstlane(qdiv(t, k.inv_nbt)), ct = t - rt * k.nbt;
      const unsigned corner = (unsigned)(rt * 16 * B + ct * 16) * 4u;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned off = lane_x + corner + (unsigned)(q * B) * 4u;
        xa[i][q] = bx0.f32(off);
        xb[i][q] = bx1.f32(off);
        fu[i][q] = bf1.f32(off);
      }
      __builtin_amdgcn_sched_barrier(0);  // one batch of loads per tile (register pressure)
    }
    const BufRead bw(k.w_g, k.M * k.ldw_g * 4);
    const unsigned lane_w = (unsigned)(4 * lg * k.ldw_g + lr) * 4u;
#pragma unroll
    for (int i = 0; i < MU; ++i) {
      const int t = wave + NWV * i;
      const int ut = __builtin_amdgcn_readfirstlane(k.urt(t)), uc = t - ut * k.ktl;
      const unsigned corner = (unsigned)(ut * 16 * k.ldw_g + uc * 16) * 4u;
#pragma unroll
      for (int q = 0; q < 4; ++q) wr[i][q] = bw.f32(lane_w + corner + (unsigned)(q * k.ldw_g) * 4u);
    }
  }
  setup(k);
  if (warm) {
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < ninf) fb[i] = k.stage_fv4(k.trow(t, 0), k.tcol(t), fu[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < ninf) fb[i] = k.stage_f4(k.trow(t, 0), k.tcol(t), xb[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < MU; ++i) {
    const int t = wave + NWV * i;
    if (t < k.n_upd) k.stage_w4(k.urt(t) * 16 + 4 * lg, k.uct(t) * 16 + lr, wr[i]);
  }
  end_prologue(k, p, aword, peers, npeers_lds);
  const int npeers = npeers_lds;

  const bool from_top = l + 1 == L - 1;
  for (int s = 0; s < p.steps; ++s) {
    k.refresh();
    const int lg = k.lg, lr = k.lr;
    const int buf = s & 1;
    // ---- 1. eps[l] = x[l] - W f(x[l+1]); g = W^T eps[l]
    float* xe = l >= 1 ? p.xe[l] + (long long)buf * npr * RES_TILE : nullptr;
    f32x4 cp[MAXT];
    k.pred_tiles_h(npr, cp);
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < npr) {
        const f32x4 c = cp[i];
        const int b = k.tcol(t), r0 = k.trow(t, 0);
        if (r0 + 4 <= k.M && b < B) {  // (the lane's four rows and its column all exist)
#pragma unroll
          for (int q = 0; q < 4; ++q) ea[i][q] = xa[i][q] - c[q];
          k.stage_e4_full(r0, b, ea[i]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) ea[i][q] = r0 + q < k.M && b < B ? xa[i][q] - c[q] : 0.0f;
          k.stage_e4(r0, b, ea[i]);
        }
        if (xe) st_rec(xe + k.rec(t), ea[i]);
      }
    }
    __syncthreads();
    // gb = f'(x[l+1]) (W^T eps[l]) of the old state x[l+1], kept for this
    // workgroup's copy of x[l+1] and sent to workgroup l+1 (or the top chunks,
    // which read it one step later: three buffers)
    float* xg = p.xg[l] + (long long)(from_top ? s % 3 : buf) * ninf * RES_TILE;
    f32x4 db[MAXT];
#pragma unroll
    for (int i = 0; i < MAXT; ++i) db[i] = dact4_from<ACT>(xb[i], fb[i]);
    k.infer_tiles(ninf, gb);
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      gb[i] = mul4(db[i], gb[i]);
      if (t < ninf) st_rec(xg + k.rec(t), gb[i]);
    }
    // ---- 2. exchange
    publish(&p.flags[k.wg], ep.base + (unsigned)(s + 1));
    wait_peers(p, peers, npeers, ep.base + (unsigned)(s + 1), 0, false);
    // ---- 3. x[l] with f'(x[l]) g[l] from workgroup l-1; x[l+1] with eps[l+1] from above
    // (every exchange load of the phase is issued before the first use)
    // (f'(x[l]) g[l] of workgroup l-1, absent for l = 0; eps[l+1] from workgroup
    // l+1, or eps[L-1] as summed by the row blocks' chunk 0; through scalar
    // bases and 32-bit byte offsets.  A tile past the counts, or an absent
    // record, reads tile 0 of eps[l+1], in range; such values are never used:
    // every use of gl and eu is under the same tile test)
    f32x4 gl[MAXT], eu[MAXT];
    static_assert(MAXT == 2, "four records per wave");
    const bool xgl = l >= 1;
    {
      const float* ebase = uniform((from_top ? p.xs : p.xe[l + 1]) + (long long)buf * ninf * RES_TILE);
      const float* gbase = xgl ? uniform(p.xg[l - 1] + (long long)buf * npr * RES_TILE) : ebase;
      const int t0 = wave, t1 = wave + NWV;
      const unsigned r0 = (unsigned)k.rec(t0) * 4u, r1 = (unsigned)k.rec(t1) * 4u, f = (unsigned)k.rec(0) * 4u;
      const bool g0 = xgl && t0 < npr, g1 = xgl && t1 < npr, e0 = t0 < ninf, e1 = t1 < ninf;
      ld_rec4_sc1(gbase, g0 ? r0 : f, g1 ? r1 : f, ebase, e0 ? r0 : f, e1 ? r1 : f, gl[0], gl[1], eu[0], eu[1]);
    }
    if (xgl) {
#pragma unroll
      for (int i = 0; i < MAXT; ++i) {
        const int t = wave + NWV * i;
        if (t < npr)
#pragma unroll
          for (int q = 0; q < 4; ++q) xa[i][q] = state_update(xa[i][q], ea[i][q], gl[i][q], gamma);
      }
    }
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < ninf) {
#pragma unroll
        for (int q = 0; q < 4; ++q) xb[i][q] = state_update(xb[i][q], eu[i][q], gb[i][q], gamma);
        const int b = k.tcol(t), r0 = k.trow(t, 0);
        if (r0 + 4 <= k.K && b < B) fb[i] = k.stage_f4_full(r0, b, xb[i]);
        else fb[i] = k.stage_f4(r0, b, xb[i]);
      }
    }
    if (s + 1 == p.steps) write_states(k, p, ea, xa, xb, fb);  // overlaps the last weight update
    __syncthreads();
    // ---- 4. W[l] += alpha eps[l] f(x_new[l+1])^T
    // (after the last step W only leaves from the registers: no operand
    // copies, no barrier)
    const bool more = s + 1 < p.steps;
#pragma unroll
    for (int i = 0; i < MU; ++i) {
      const int t = wave + NWV * i;
      if (t < k.n_upd) {
        const f32x4 c = k.update_tile_h(t);
        const int col = k.uct(t) * 16 + lr, r0 = k.urt(t) * 16 + 4 * lg;
        if (r0 + 4 <= k.M && col < k.K) {  // (the lane's four rows and its column all exist)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
            wr[i][q] = wr[i][q] + alpha * c[q];
          }
          if (more) k.stage_w4_full(r0, col, wr[i]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (r0 + q < k.M && col < k.K) {
#pragma clang fp contract(off)
              wr[i][q] = wr[i][q] + alpha * c[q];
            }
          }
          if (more) k.stage_w4(r0, col, wr[i]);
        }
      }
    }
    if (more) __syncthreads();
  }

  // ---- results: W[l] (the states went out before the last weight update)
  gf32* WG = gbl(uniform(p.w[l]));
#pragma unroll
  for (int i = 0; i < MU; ++i) {
    const int t = wave + NWV * i;
    if (t < k.n_upd) {
      const int c = k.uct(t) * 16 + lr, r0 = k.urt(t) * 16 + 4 * lg;
      const unsigned o = (unsigned)(r0 * k.ldw_g + c) * 4u, rs = (unsigned)k.ldw_g * 4u;
      if (r0 + 4 <= k.M && c < k.K) {
        st4_rows(WG, o, rs, wr[i]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (r0 + q < k.M && c < k.K) st_at(WG, o + q * rs, wr[i][q]);
      }
    }
  }
  mark_cached(p, k.wg, ep);  // fx[l+1] was written in the last step
}

// Top-layer chunk j, row block h: rows [row0, row0 + M) and columns
// [k0, k0 + K) of W[L-1] at the update tiles, the same rows of x[L-1] at the
// prediction tiles, f(x[L]) of the chunk in LDS.
template <typename OT, int SPLIT, int ACT>
__device__ __forceinline__ void run_top(Resident<OT, SPLIT, ACT>& k, ResidentArgs& p, int* peers,
                                        int& npeers_lds, int aword) {
  // (scalars from the kernel arguments: the LDS copy p is published by setup)
  const int L = k.L, B = k.B, C = k.p.chunks, l = k.l, j = k.j, wave = k.wave, lg = k.lg, lr = k.lr;
  // npr: this row block's prediction tiles; nrec: the layer's, the size of every
  // exchange record of the top layer (the block's tiles start at tile k.toff)
  const int npr = k.n_pred, nrec = k.npr_full, r0 = k.row0;
  const float gamma = k.p.gamma, alpha = k.p.alpha;
  f32x4 xa[MAXT], wr[MAXT];
  {
    // the block's rows of x[L-1] and its rows and columns of W[L-1] through
    // buffers that end with the block (tile indices past the counts map to
    // rows past it: zeros; rows 4 lg + q and column lr of a tile: one 32-bit
    // offset per lane, the tile's corner and q uniform)
    const int ldw = k.ldw_g;
    const BufRead bx(k.x_g + (long long)r0 * B, k.M * B * 4);
    const BufRead bw(k.w_g + (long long)r0 * ldw + k.k0, ((k.M - 1) * ldw + k.K) * 4);
    const unsigned lane_x = (unsigned)(4 * lg * B + lr) * 4u, lane_w = (unsigned)(4 * lg * ldw + lr) * 4u;
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      const int rt = __builtin_amdgcn_readfirstlane(qdiv(t, k.inv_nbt)), ct = t - rt * k.nbt;
      const int ut = __builtin_amdgcn_readfirstlane(k.urt(t)), uc = t - ut * k.ktl;
      const unsigned cx = (unsigned)(rt * 16 * B + ct * 16) * 4u, cw = (unsigned)(ut * 16 * ldw + uc * 16) * 4u;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xa[i][q] = bx.f32(lane_x + cx + (unsigned)(q * B) * 4u);
        wr[i][q] = bw.f32(lane_w + cw + (unsigned)(q * ldw) * 4u);
      }
      __builtin_amdgcn_sched_barrier(0);  // one batch of loads per tile (register pressure)
    }
  }
  // f(x[L]) of the chunk: x[L] is clamped, so its 16-bit operand copies (the
  // LDS region fh .. ea) are cached in the workspace by the first launch after
  // the forward initialisation (which marks the cache stale) and copied back
  // into LDS by the launches after it.  The flag that says whether the cache is
  // valid and the image's first CB * NT 16-byte pieces are loaded with the
  // states, before the set-up barrier, so that the three latencies overlap (a
  // launch with a stale cache drops the pieces; the image region always exists).
  char* image = k.image_g;
  uint4* lds_image = reinterpret_cast<uint4*>(k.lds + k.lay.fh);
  const int n16 = (k.lay.ea - k.lay.fh) * (int)sizeof(OT) / 16;
  const Epoch ep = load_epoch(k.p, k.wg);
  const bool warm = ep.warm;
  constexpr int CB = 8;  // 16-byte loads in flight per thread
  const gu32x4* isrc = (const gu32x4*)image;
  u32x4 img[CB];
  {
    // (a wave whose pieces all lie past the image issues no load for them; in
    // a wave that straddles its end, those lanes read zeros and store nothing)
    const BufRead bi(image, n16 * 16);
    const int wbase = __builtin_amdgcn_readfirstlane((int)threadIdx.x & ~63);
#pragma unroll
    for (int u = 0; u < CB; ++u)
      if (wbase + u * NT < n16) img[u] = bi.u128((threadIdx.x + u * NT) * 16u);
  }
  // A warm launch's first step sums the partial products the previous launch
  // left in xn.  Those of the wave's first prediction tile are loaded here,
  // with the image, and summed once they arrive (the same loads and chunk
  // order as sum_partials), so that the first eps[L-1] does not wait for a
  // memory round trip after the prologue; a second tile loads its own in the
  // step.  A cold launch drops them.
  const int nrec_pf = k.npr_full, npr_pf = k.n_pred;
  const bool pf = C <= PBATCH && wave < npr_pf;
  f32x4 pv[PBATCH];
  if (pf) {
    const float* xn0 = k.p.xn + k.rec(k.toff + wave);
#pragma unroll
    for (int u = 0; u < PBATCH; ++u) pv[u] = u < C ? ld_rec(xn0 + (long long)u * nrec_pf * RES_TILE) : zero4();
  }
  setup(k);
  if (warm) {
    const gu32x4* src = isrc;
    u32x4* dst = reinterpret_cast<u32x4*>(lds_image);
#pragma unroll
    for (int u = 0; u < CB; ++u)
      if ((int)threadIdx.x + u * NT < n16) dst[threadIdx.x + u * NT] = img[u];
    for (int base = threadIdx.x + CB * NT; base < n16; base += CB * NT) {
      u32x4 v[CB];
#pragma unroll
      for (int u = 0; u < CB; ++u) v[u] = src[min(base + u * NT, n16 - 1)];
#pragma unroll
      for (int u = 0; u < CB; ++u)
        if (base + u * NT < n16) dst[base + u * NT] = v[u];
    }
  } else {
    // evaluate f(x[L]) of the chunk; row block 0 also writes it to fx[L] and to
    // the image (the chunk's row blocks share one)
    const float* XL = k.p.x[L];
    float* FL = k.h == 0 ? k.p.fx[L] : nullptr;
    constexpr int SB = 8;  // loads in flight per thread
    const int n = k.K * B;
    for (int base = threadIdx.x; base < n; base += SB * NT) {
      float v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int idx = base + u * NT;
        v[u] = ld_at(XL, k.k0 * B + idx, idx < n);
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int idx = base + u * NT;
        if (idx < n) {
          const int kk = qdiv(idx, k.inv_B), b = idx - kk * B;
          k.stage_f(kk, b, v[u]);
          if (FL) gbl(FL)[(long long)k.k0 * B + idx] = act_t<ACT>(v[u]);
        }
      }
    }
    __syncthreads();
    if (k.h == 0) {
      gu32x4* dst = (gu32x4*)image;
      const u32x4* src = reinterpret_cast<const u32x4*>(lds_image);
      for (int i = threadIdx.x; i < n16; i += NT) dst[i] = src[i];
    }
  }
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    const int t = wave + NWV * i;
    if (t < k.n_upd) {
      const int c = k.uct(t) * 16 + lr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = k.urt(t) * 16 + 4 * lg + q;
        if (r < k.M && c < k.K) k.stage_w(r, c, wr[i][q]);
      }
    }
  }
  end_prologue(k, p, aword, peers, npeers_lds);
  const int npeers = npeers_lds;
  f32x4 pre_sum = zero4();
  if (pf) {
    pre_sum = pv[0];
#pragma unroll
    for (int u = 1; u < PBATCH; ++u)
      if (u < C)
#pragma unroll
        for (int q = 0; q < 4; ++q) pre_sum[q] = pre_sum[q] + pv[u][q];
  }

  // The chunks apply each step's x[L-1] update one step late, just before the
  // next step's eps[L-1]: their own chain (partial product, partial sums,
  // weight update) then waits for workgroup L-2's previous step only, and
  // workgroup L-2 writes x[L-1] after the last step.
  //
  // When the cached operands are current (warm), the previous launch has
  // left the first step's partial products in xn, computed with the same W
  // and f(x[L]) bits at its end: the first step skips its partial product
  // and the exchange and sums them at once, so the first eps[L-1] reaches
  // workgroup L-2 without waiting for the whole row block's first partial
  // product (at the start of a launch the top chunks are not yet a step
  // ahead of it).
  float* xn = p.xn + (long long)j * nrec * RES_TILE;
  // ev_prev: the previous step's eps[L-1], read from the second step on; before
  // the first, tile 0's prefetched partial sum
  f32x4 ev_prev[MAXT];
#pragma unroll
  for (int i = 0; i < MAXT; ++i) ev_prev[i] = i == 0 ? pre_sum : zero4();
  for (int s = 0; s < p.steps; ++s) {
    k.refresh();
    const int lg = k.lg, lr = k.lr;
    const int buf = s & 1;
    const bool last = s + 1 == p.steps;
    const bool pre = warm && s == 0;  // the partials are the previous launch's xn
    // ---- 1. partial product of the chunk
    float* xp = pre ? p.xn : p.xp + (long long)buf * C * nrec * RES_TILE;
    if (!pre) {
      f32x4 cp[MAXT];
      k.pred_tiles(npr, cp);
#pragma unroll
      for (int i = 0; i < MAXT; ++i) {
        const int t = wave + NWV * i;
        if (t < npr) st_rec(xp + (long long)j * nrec * RES_TILE + k.rec(k.toff + t), cp[i]);
      }
    }
    // ---- 2. exchange: the siblings' partials of this step, workgroup L-2's
    // f'(x[L-1]) g of the previous one (f' of the state the late update starts
    // from; nothing to wait for in a first step from xn: its flag goes up once
    // the step has read xn, below)
    if (!pre) publish(&p.flags[k.wg], ep.base + (unsigned)(s + 1));
    if (!pre) wait_peers(p, peers, npeers, ep.base + (unsigned)(s + 1), 1);
    f32x4 g[MAXT];
#pragma unroll
    for (int i = 0; i < MAXT; ++i) g[i] = zero4();
    if (s >= 1) {
      const float* xg = p.xg[L - 2] + (long long)((s - 1) % 3) * nrec * RES_TILE;
#pragma unroll
      for (int i = 0; i < MAXT; ++i) {
        const int t = wave + NWV * i;
        if (t < npr) g[i] = ld_rec(xg + k.rec(k.toff + t));
      }
    }
    // ---- 3. x[L-1] of this step (the previous step's update), then eps[L-1] =
    // x[L-1] - (P_0 + P_1 + ...) in chunk order (this chunk's own partial read
    // back like the others); chunk 0 publishes it for workgroup L-2
    f32x4 ev4[MAXT];
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      ev4[i] = zero4();
      if (t < npr) {
        const f32x4 sum = i == 0 && pre && pf ? ev_prev[0] : sum_partials(xp, (long long)nrec * RES_TILE, C, k.rec(k.toff + t));
        const int b = k.tcol(t);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = k.trow(t, q);
          if (s >= 1) xa[i][q] = state_update(xa[i][q], ev_prev[i][q], g[i][q], gamma);
          ev4[i][q] = (r < k.M && b < B) ? xa[i][q] - sum[q] : 0.0f;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (j == 0) {
      float* xs = p.xs + (long long)buf * nrec * RES_TILE;
#pragma unroll
      for (int i = 0; i < MAXT; ++i) {
        const int t = wave + NWV * i;
        if (t < npr) st_rec(xs + k.rec(k.toff + t), ev4[i]);
      }
      publish(&p.flags[p.nwg + k.h], ep.base + (unsigned)(s + 1));
    }
    // a first step from xn raises its step flag after its reads of xn (the
    // launch's end rewrites xn once every sibling's flag has passed base + 1)
    // only when it is the launch's last step: otherwise the second step's
    // flag, base + 2, says as much, and nobody waits for base + 1
    if (pre && last) publish(&p.flags[k.wg], ep.base + 1u);
    // eps[L-1] into the weight-update A operand (and e[L-1] after the last step)
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      ev_prev[i] = ev4[i];
      if (t < npr) {
        const int b = k.tcol(t);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = k.trow(t, q);
          if (r < k.M && b < B) {
            k.lds[k.lay.ea + k.m24(r, k.lay.lda) + b] = cvt<OT>(ev4[i][q]);
            if (last && j == 0) gbl(p.e[l])[(long long)(r0 + r) * B + b] = ev4[i][q];
          }
        }
      }
    }
    __syncthreads();
    // ---- 4. W[L-1][:, chunk] += alpha eps[L-1] f(x[L])[chunk]^T
    f32x4 cu[MAXT];
    k.update_tiles(k.n_upd, cu);
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < k.n_upd) {
        const f32x4 c = cu[i];
        const int col = k.uct(t) * 16 + lr;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = k.urt(t) * 16 + 4 * lg + q;
          if (r < k.M && col < k.K) {
#pragma clang fp contract(off)
            wr[i][q] = wr[i][q] + alpha * c[q];
            k.stage_w(r, col, wr[i][q]);
          }
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    const int t = wave + NWV * i;
    if (t < k.n_upd) {
      const int c = k.uct(t) * 16 + lr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = k.urt(t) * 16 + 4 * lg + q;
        if (r < k.M && c < k.K) gbl(p.w[l])[(long long)(r0 + r) * k.ldw_g + k.k0 + c] = wr[i][q];
      }
    }
  }
  // the next launch's first partial product, with the final W (staged by the
  // last step) once every sibling has read this launch's xn (its first step's
  // flag); the same instructions and operand bits as a step's partial product
  if (p.steps > 0) {
    wait_peers(p, peers, npeers, ep.base + 1u, 1);
    f32x4 cp[MAXT];
    k.pred_tiles(npr, cp);
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int t = wave + NWV * i;
      if (t < npr) st_rec(xn + k.rec(k.toff + t), cp[i]);
    }
  }
  mark_cached(p, k.wg, ep);  // the chunk's image (row block 0 wrote it this launch or before) and xn
}

// XCD-aware placement.  Blocks are dealt to the eight XCDs round-robin by
// block index, so the top workgroups of row block h take blocks 7 - h,
// 15 - h, 23 - h, ... (one XCD per row block: each of them reads all its
// siblings' partial products every step, and those reads then share one L2)
// and the hidden workgroups the blocks of the other XCDs, the lower ones
// first: the XCDs start their first blocks in index order, and the hidden
// chain sets the pace while the top chunks may run a step ahead.  The spare
// blocks of the grid exit at once.  Placement only affects speed: every
// exchange is ordered at agent scope wherever the workgroups run.
__host__ __device__ inline int resident_role(int bid, int hidden, int chunks, int halves) {
  const int x = 7 - (bid & 7), i = bid >> 3;  // x: XCD counted from the last
  if (x < halves) return i < chunks ? hidden + x * chunks + i : -1;
  const int l = i * (8 - halves) + (x - halves);
  return l < hidden ? l : -1;
}
inline int resident_grid(int hidden, int chunks, int halves) {
  // the top chunks' blocks end at 8 * chunks - 1; the hidden workgroups fill
  // XCDs 0 .. 7 - halves row by row of eight blocks
  const int top = 8 * chunks;
  const int low = hidden > 0 ? 8 * ((hidden - 1) / (8 - halves)) + 8 : 0;
  return top > low ? top : low;
}

template <typename OT, int SPLIT, int ACT>
__global__ void __launch_bounds__(NT) resident_kernel(const ResidentArgs args) {
  using R = Resident<OT, SPLIT, ACT>;
  extern __shared__ __align__(16) char lds_raw[];
  // The argument block is indexed with run-time layer numbers; a copy in LDS
  // serves those reads at LDS latency instead of a memory round trip each.
  __shared__ ResidentArgs p;
  __shared__ int peers[RES_MAX_WG];
  __shared__ int npeers;
  static_assert(sizeof(ResidentArgs) % 4 == 0 && sizeof(ResidentArgs) / 4 <= NT, "argument block copy");
  // Each thread's word of the copy is loaded first and stored at the end of
  // the prologue (end_prologue), whose barrier publishes it; until then the
  // role and the prologue's loads are addressed from the kernel arguments
  // (k.p).
  constexpr int NARG = sizeof(ResidentArgs) / 4;
  const int aword = reinterpret_cast<const int*>(&args)[min((int)threadIdx.x, NARG - 1)];  // (no branch)
  // The argument scalars the prologue needs arrive in two batches of loads
  // with one wait each (loaded where first used, they cost a memory round
  // trip each): those that place the block, then those of its layer.
  const int L = args.L, B = args.B, chunks = args.chunks, halves = args.halves;
  asm volatile("" ::"s"(L), "s"(B), "s"(chunks), "s"(halves));
  const int role = resident_role(blockIdx.x, L - 1, chunks, halves);
  if (role < 0) return;  // a spare block of the XCD-aware grid
  R k(args, lds_raw, role);  // (loads the layer's scalars in the second batch)
  if (k.hidden) run_hidden(k, p, peers, npeers, aword);
  else run_top(k, p, peers, npeers, aword);
}

// ---------------------------------------------------------------- dispatch
template <typename OT, int SPLIT, int ACT>
struct ResLaunch {
  static hipError_t prepare(int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&resident_kernel<OT, SPLIT, ACT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  }
  static hipError_t launch(const ResidentArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((resident_kernel<OT, SPLIT, ACT>), dim3(resident_grid(a.L - 1, a.chunks, a.halves)), dim3(NT),
                       (size_t)a.lds_bytes, s, a);
    return hipGetLastError();
  }
  static hipError_t occupancy(int bytes, int* per_cu) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(
        per_cu, reinterpret_cast<const void*>(&resident_kernel<OT, SPLIT, ACT>), NT, (size_t)bytes);
  }
};

template <typename OT, int SPLIT>
hipError_t by_act(int act, bool prep, int bytes, const ResidentArgs* a, hipStream_t s, int* occ) {
#define IPC_RES_CASE(A)                                                                  \
  case A:                                                                                \
    return occ ? ResLaunch<OT, SPLIT, A>::occupancy(bytes, occ)                           \
               : prep ? ResLaunch<OT, SPLIT, A>::prepare(bytes) : ResLaunch<OT, SPLIT, A>::launch(*a, s);
  switch (act) {
    IPC_RES_CASE(ACT_RELU)
    IPC_RES_CASE(ACT_TANH)
    IPC_RES_CASE(ACT_SIGMOID)
    IPC_RES_CASE(ACT_SILU)
    IPC_RES_CASE(ACT_GELU)
    IPC_RES_CASE(ACT_IDENTITY)
    default:
      return hipErrorInvalidValue;
  }
#undef IPC_RES_CASE
}

// One of three operations on the instantiation for (operand, split, act):
// raise its LDS limit (prep), report its workgroups per CU (occ) or launch it.
hipError_t dispatch(int operand, int split, int act, bool prep, int bytes, const ResidentArgs* a, hipStream_t s,
                    int* occ = nullptr) {
  if (operand == DT_F32) return by_act<float, 1>(act, prep, bytes, a, s, occ);
  if (operand == DT_F16)
    return split >= 3 ? by_act<f16, 3>(act, prep, bytes, a, s, occ) : by_act<f16, 1>(act, prep, bytes, a, s, occ);
  if (operand == DT_BF16)
    return split >= 3 ? by_act<bf16, 3>(act, prep, bytes, a, s, occ) : by_act<bf16, 1>(act, prep, bytes, a, s, occ);
  return hipErrorInvalidValue;
}

}  // namespace

long long resident_plan(const int* dims, int L, int B, int split, int esize, bool outer, int top_rows,
                        ResidentArgs& a) {
  if (top_rows != 16 && top_rows != 32 && top_rows != 64) return -1;
  if (L < 2 || L > NARROW_MAX_L || B < 1 || B > RES_MAX_B) return -1;
  if (esize == 4 ? split >= 2 : esize != 2) return -1;
  if (outer && (esize != 4 || B > NARROW_OUTER_MAX_B)) return -1;
  for (int l = 0; l < L; ++l)
    if (dims[l] < 1 || dims[l] > RES_MAX_WIDTH) return -1;
  const bool s3 = split >= 3;
  const int limit = NARROW_LDS_LIMIT - 2048;  // static LDS: argument copy and peer list
  int need = 0;
  for (int l = 0; l + 1 < L; ++l) {
    ResidentLds o;
    resident_lds_layout(dims[l], dims[l + 1], B, true, s3, esize, o);
    need = o.bytes > need ? o.bytes : need;
  }
  // top layer: one workgroup per NARROW_KCHUNK columns (the column kernel's
  // partial-sum order)
  // and row blocks of top_rows rows (a workgroup per chunk and block; one
  // XCD per row block, at least one XCD left for the hidden workgroups)
  const int dL = dims[L], kc = NARROW_KCHUNK, C = (dL + kc - 1) / kc;
  const int halves = (dims[L - 1] + top_rows - 1) / top_rows;
  if (halves > 7) return -1;
  if ((L - 1) + halves * C + halves > RES_MAX_WG) return -1;  // flags[nwg + h]: block h's eps flags
  ResidentLds o;
  resident_lds_layout(dims[L - 1] < top_rows ? dims[L - 1] : top_rows, dL < kc ? dL : kc, B, false, s3, esize, o);
  need = o.bytes > need ? o.bytes : need;
  if (need > limit) return -1;
  a.L = L;
  a.B = B;
  a.chunks = C;
  a.kc = kc;
  a.halves = halves;
  a.top_rows = top_rows;
  a.outer = outer ? 1 : 0;
  a.nwg = (L - 1) + halves * C;
  a.lds_bytes = res_round(need, 16);
  for (int l = 0; l <= L; ++l) a.dims[l] = dims[l];
  long long bytes = RES_FLAG_BYTES;  // flags
  for (int l = 0; l + 1 < L; ++l) {
    if (l >= 1) bytes += 2LL * resident_tiles(dims[l], B) * RES_TILE * 4;
    bytes += (l + 2 == L ? 3LL : 2LL) * resident_tiles(dims[l + 1], B) * RES_TILE * 4;
  }
  bytes += (2LL * (C + 1) + C) * resident_tiles(dims[L - 1], B) * RES_TILE * 4;
  a.image_stride = res_round((o.ea - o.fh) * esize, 256);  // the fh .. ea region of the widest chunk
  bytes = res_round(bytes, 256) + C * a.image_stride;
  return bytes;
}

void resident_bind(ResidentArgs& a, char* ws) {
  const int L = a.L, B = a.B;
  a.flags = reinterpret_cast<unsigned*>(ws);
  char* at = ws + RES_FLAG_BYTES;
  for (int l = 0; l < NARROW_MAX_L; ++l) { a.xe[l] = nullptr; a.xg[l] = nullptr; }
  for (int l = 0; l + 1 < L; ++l) {
    if (l >= 1) {
      a.xe[l] = reinterpret_cast<float*>(at);
      at += 2LL * resident_tiles(a.dims[l], B) * RES_TILE * 4;
    }
    a.xg[l] = reinterpret_cast<float*>(at);
    at += (l + 2 == L ? 3LL : 2LL) * resident_tiles(a.dims[l + 1], B) * RES_TILE * 4;
  }
  a.xp = reinterpret_cast<float*>(at);
  at += 2LL * a.chunks * resident_tiles(a.dims[L - 1], B) * RES_TILE * 4;
  a.xs = reinterpret_cast<float*>(at);
  at += 2LL * resident_tiles(a.dims[L - 1], B) * RES_TILE * 4;
  a.xn = reinterpret_cast<float*>(at);
  at += (long long)a.chunks * resident_tiles(a.dims[L - 1], B) * RES_TILE * 4;
  a.image = ws + res_round((long long)(at - ws), 256);
}

__global__ void resident_invalidate_kernel(unsigned* gen) { *gen += 1u; }

hipError_t resident_invalidate(const ResidentArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(resident_invalidate_kernel, dim3(1), dim3(1), 0, s, a.flags + RES_MAX_WG);
  return hipGetLastError();
}

hipError_t resident_prepare(int operand, int split, int act, int lds_bytes) {
  return dispatch(operand, split, act, true, lds_bytes, nullptr, nullptr);
}

int resident_launch_blocks(const ResidentArgs& a) { return resident_grid(a.L - 1, a.chunks, a.halves); }

hipError_t resident_occupancy(int operand, int split, int act, int lds_bytes, int* per_cu) {
  *per_cu = 0;
  return dispatch(operand, split, act, false, lds_bytes, nullptr, nullptr, per_cu);
}

hipError_t launch_resident(const ResidentArgs& a, int operand, int split, int act, hipStream_t s) {
  return dispatch(operand, split, act, false, 0, &a, s);
}

}  // namespace ipc
