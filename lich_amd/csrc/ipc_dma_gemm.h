// ipc_dma_gemm.h - the LDS-DMA MFMA GEMM kernel template (gfx950).
//
// One workgroup = WGM x WGN waves = one BM x BN output tile; each wave owns
// (BM/WGM) x (BN/WGN) of it as 32x32 fp32 MFMA blocks
// (v_mfma_f32_32x32x16_{f16,bf16}).  Main loop, per k-step of 64:
//
//   * operands move HBM -> LDS with global_load_lds_dwordx4 (LDS DMA: no VGPR
//     staging), S stages deep; one wave instruction fills 1 KB of LDS.  An
//     operand that needs its activation applied (f(X_upper) of the
//     standalone pred / weight kernels) instead goes global -> VGPR ->
//     f -> LDS, loaded one stage ahead and stored after the current stage's
//     MFMAs;
//   * a k-contiguous operand block is EDGE rows of 128 bytes, 16-byte chunk c
//     of row r stored at chunk c ^ ((r >> 1) & 7): a 16-byte fragment read by
//     16 lanes of 16 consecutive rows touches each of the 64 LDS banks once;
//   * an m/n-contiguous block is 64 k-rows of 2*EDGE bytes, chunk c of k-row
//     r at chunk c ^ ((r & 3) << 2); its fragments come from two
//     ds_read_b64_tr_b16 (16 lanes read a 4 x 16 block, one 8-byte row piece
//     each, and get its columns back), and the swizzle spreads the 4 k-rows of
//     a half-wave over distinct banks;
//   * one workgroup barrier per k-step without the fence of __syncthreads
//     (that fence would make the compiler wait for every outstanding DMA
//     load): a wave waits for its own loads of the step it is about to read
//     (s_waitcnt vmcnt), the barrier publishes everybody's, then it refills
//     the stage everybody has finished with;
//   * fragments of the next 16-k slice are read while the current slice's
//     MFMAs run; split 2 adds the A_lo B products (error compensation);
//   * A32 (split-2 wide prediction and forward): A is the fp32 W itself, 64
//     k-values per 256-byte LDS row (chunk c of row r at c ^ (r & 15)), split
//     into its hi and lo 16-bit fragments as it is read (the values the
//     separate hi / lo copies would hold, in the same bytes per stage);
//   * workgroups are renumbered so that the tiles one XCD runs are consecutive
//     (the tiles sharing rows of A share that XCD's L2);
//   * a k-split prediction problem (last in its launch) runs each tile as
//     ksplit slices of the contraction that store raw fp32 partial products;
//     their workgroups come after every whole tile's, so the slices fill the
//     CUs that the last round of whole tiles leaves idle.
//
// Epilogue: the accumulator tile goes through LDS (the stages are free by
// then) so that every global access is a coalesced row-major 4-column group;
// the fp32 input the epilogue updates is fetched into registers before the
// main loop.  Reference semantics: src/ipc_tilelang/tilelang_kernels.py:173
// (prediction error), :227-231 (inference update), :319-320 (weight update);
// the fp32 rounding sequence is that of src/ipc_tilelang/reference.py:49-57,
// every operation rounded on its own (no FMA contraction).
#pragma once

#include "ipc_device.h"
#include "ipc_launch.h"
#include "ipc_wide.h"

namespace ipc {
namespace dma {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the fence of __syncthreads.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Operand layouts: A is m-contiguous (read transposed) for the standalone
// inference update (W_lower [K][M]), k-contiguous otherwise; B is
// n-contiguous for the standalone prediction / forward / inference kernels
// (X_upper, E_lower [K][B]), k-contiguous for the weight update and for the
// prediction / forward given f(X_upper)^T (S16_PREDT / S16_FWDT).  The wide
// path keeps k-contiguous copies of every operand (WT, FT, ET next to W, F,
// E), so all of its reads are plain 16-byte fragment reads.
constexpr bool a_mn(int mode) { return mode == S16_INFER; }
constexpr bool b_mn(int mode) { return mode == S16_PRED || mode == S16_FWD || mode == S16_INFER; }
constexpr bool is_s16(int mode) { return mode >= S16_PRED; }
// the standalone prediction / forward, with B as given or as f(X_upper)^T
constexpr bool s16_pred(int mode) { return mode == S16_PRED || mode == S16_PREDT; }
constexpr bool s16_fwd(int mode) { return mode == S16_FWD || mode == S16_FWDT; }
// the standalone inference update, with W_lower / E_lower as given or transposed
constexpr bool s16_infer(int mode) { return mode == S16_INFER || mode == S16_INFERT; }

// chunk position of chunk c in row r
__device__ __forceinline__ int kc_swz(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int mn_swz(int r, int c) { return c ^ ((r & 3) << 2); }

// Global source of LDS slot `slot` (16 bytes) of an operand block.
//   KC: rows e0 .. e0+EDGE-1 (clamped to lim-1), k0 .. k0+63
//   MN: k-rows k0 .. k0+63, columns e0 .. e0+EDGE-1 (chunk starts clamped to lim-8)
// Global source of LDS slot `slot` (16 bytes = 4 floats) of an fp32
// k-contiguous block: rows e0 .. e0+EDGE-1 (clamped to lim-1), k0 .. k0+63.
template <int EDGE>
__device__ __forceinline__ const float* slot_src32(const float* g, long long ld, int e0, int lim, int k0, int slot) {
  const int r = slot >> 4, c = (slot & 15) ^ (r & 15);
  const int row = e0 + r < lim ? e0 + r : lim - 1;
  return g + (long long)row * ld + k0 + c * 4;
}

template <typename OT, bool MN, int EDGE>
__device__ __forceinline__ const OT* slot_src(const OT* g, long long ld, int e0, int lim, int k0, int slot) {
  if (!MN) {
    const int r = slot >> 3, c = kc_swz(r, slot & 7);
    const int row = e0 + r < lim ? e0 + r : lim - 1;
    return g + (long long)row * ld + k0 + c * 8;
  } else {
    constexpr int CPR = EDGE / 8;  // chunks per k-row
    const int r = slot / CPR, c = mn_swz(r, slot % CPR);
    const int col = e0 + c * 8 <= lim - 8 ? e0 + c * 8 : lim - 8;
    return g + (long long)(k0 + r) * ld + col;
  }
}

typedef float f32x8 __attribute__((ext_vector_type(8)));

// The fp32 values of 8 packed 16-bit operands (bf16: each half of a packed
// word shifted into place, so that no value is converted a second time).
__device__ __forceinline__ f32x8 widen8(bf16x8 h) {
  const uint4 u = __builtin_bit_cast(uint4, h);
  auto lo = [](unsigned w) { return __builtin_bit_cast(float, w << 16); };
  auto hi = [](unsigned w) { return __builtin_bit_cast(float, w & 0xffff0000u); };
  return f32x8{lo(u.x), hi(u.x), lo(u.y), hi(u.y), lo(u.z), hi(u.z), lo(u.w), hi(u.w)};
}
__device__ __forceinline__ f32x8 widen8(f16x8 h) { return __builtin_convertvector(h, f32x8); }

template <typename OT>
__device__ __forceinline__ unsigned pack2(OT a, OT b) {
  return (unsigned)__builtin_bit_cast(unsigned short, a) | ((unsigned)__builtin_bit_cast(unsigned short, b) << 16);
}

template <typename OT>
__device__ __forceinline__ float lo16(unsigned v) {
  return to_f32(__builtin_bit_cast(OT, (unsigned short)(v & 0xffffu)));
}
template <typename OT>
__device__ __forceinline__ float hi16(unsigned v) {
  return to_f32(__builtin_bit_cast(OT, (unsigned short)(v >> 16)));
}

// A buffer resource over `bytes` bytes at `base`: loads and stores take a
// 32-bit per-lane offset and a uniform (scalar) one, so an epilogue can
// address an element as (its lane's row and column) + (the row step of an
// accumulator register, uniform) without a 64-bit address per element.
// Offsets at or past `bytes` load zero and store nothing.
struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Buf(const void* base, long long bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                            (int)(bytes < 0x7fffffffLL ? bytes : 0x7fffffffLL), 0x00020000)) {}
  __device__ __forceinline__ float ld32(unsigned v, unsigned s) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0));
  }
  __device__ __forceinline__ void st32(float x, unsigned v, unsigned s) const {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), r, v, s, 0);
  }
  __device__ __forceinline__ void st16(unsigned short x, unsigned v, unsigned s) const {
    __builtin_amdgcn_raw_buffer_store_b16(x, r, v, s, 0);
  }
  __device__ __forceinline__ unsigned short ld16(unsigned v, unsigned s) const {
    return __builtin_amdgcn_raw_buffer_load_b16(r, v, s, 0);
  }
};

// Dynamic LDS of a configuration: the pipeline stages, reused by the fp32
// epilogue tile (BM rows of BN + 1 floats) when that tile fits the CU's
// 160 KB; a configuration whose tile does not (256 x 256) finishes from the
// registers and stages only the wide path's 16-bit transposed copy
// (reg_epilogue).
// (LO: the A_lo block, or A stored as fp32 rows of twice the bytes.)
constexpr int stage_bytes(int BM, int BN, int S, bool LO) { return S * (BM * 128 * (LO ? 2 : 1) + BN * 128); }
constexpr bool reg_epilogue(int BM, int BN, int S, bool LO, bool s16) {
  return BM * (BN + 1) * 4 > 160 * 1024 && stage_bytes(BM, BN, S, LO) <= 160 * 1024;
}
// The split-2 prediction reading the fp32 W (A32) with 2 stages takes a third
// A stage when the LDS holds it (128 x 256: 3 x 32 + 2 x 32 KB = 160 KB): in
// the wide configuration's steady state 299-304 us per launch against
// 311-314 us, bit-identical.
constexpr bool a32_extra_stage(int BM, int BN, int S, bool a32) {
  return a32 && S == 2 && (S + 1) * BM * 256 + S * BN * 128 <= 160 * 1024;
}
constexpr int smem_bytes(int BM, int BN, int S, bool LO, bool s16 = true) {
  return reg_epilogue(BM, BN, S, LO, s16) || stage_bytes(BM, BN, S, LO) > BM * (BN + 1) * 4
             ? stage_bytes(BM, BN, S, LO)
             : BM * (BN + 1) * 4;
}

// Position (tile row mb, tile column nb) of tile `t` of a tm x tn tile grid
// walked in supertiles of ST_R x ST_C tiles: row-major inside a supertile,
// supertiles row-major, the last band and column of supertiles cut to what is
// left.  The tiles one XCD runs at once (32 CUs) then form one 8 x 4 block,
// which reads 8 row blocks of A and 4 of B, instead of 2 x 16 (the whole of
// B) in row-major order; with at most 4 tile columns the order is row-major.
constexpr int ST_R = 8, ST_C = 4;
__device__ __forceinline__ void supertile_pos(int t, int tm, int tn, int& mb, int& nb) {
  const int band = t / (ST_R * tn);
  const int rows = tm - band * ST_R < ST_R ? tm - band * ST_R : ST_R;
  const int w = t - band * ST_R * tn;
  const int cs = w / (rows * ST_C);
  const int cols = tn - cs * ST_C < ST_C ? tn - cs * ST_C : ST_C;
  const int w2 = w - cs * rows * ST_C;
  mb = band * ST_R + w2 / cols;
  nb = cs * ST_C + w2 % cols;
}

struct Batch {
  WideProblem p[WIDE_MAX_BATCH];
  int start[WIDE_MAX_BATCH + 1];  // first tile of each problem
  int count;
  int tail;                       // first k-split problem (count if none)
};

// ACT: the epilogue activation (WIDE_INFER, WIDE_FWD, S16_INFER) or the
// activation of the register-path B operand (BREG: S16_PRED, S16_FWD,
// S16_WEIGHT recompute); ACT_IDENTITY otherwise.
template <typename OT, int MODE, int SPLIT, int ACT, bool BREG, int BM, int BN, int S, int WGM, int WGN,
          bool A32 = false>
__global__ void __launch_bounds__(WGM * WGN * 64) dma_gemm_kernel(const Batch bt) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr bool LO = SPLIT == 2;
  constexpr bool AMN = a_mn(MODE), BMN = b_mn(MODE), S16 = is_s16(MODE);
  static_assert(!A32 || (LO && !AMN && !S16 && !BREG), "fp32 A: the split-2 wide prediction and forward");
  constexpr int NW = WGM * WGN, NT = NW * 64;
  // A: one 16-bit block of 128-byte rows (and its A_lo block), or one fp32
  // block of 256-byte rows (A32): the same bytes per stage
  constexpr int A_BYTES = BM * (A32 ? 256 : 128), B_BYTES = BN * 128;
  constexpr int A_BLOCKS = LO && !A32 ? 2 : 1;
  constexpr int STAGE = A_BYTES * A_BLOCKS + B_BYTES;
  constexpr int IA = A_BYTES / 1024 / NW, IB = B_BYTES / 1024 / NW;  // DMA instructions per wave and stage
  constexpr int LPS = IA * A_BLOCKS + (BREG ? 0 : IB);
  // A32 with 2 stages: the fp32 W, which each row block's few column tiles
  // read from far, takes a third stage where the LDS holds it, so its loads
  // lead by two k-steps, while the 16-bit B block (shared by every row tile,
  // an L2 hit) keeps two: the A ring first in the LDS, then the B ring.
  constexpr int AX = a32_extra_stage(BM, BN, S, A32) ? 1 : 0, SA = S + AX;
  constexpr int RB = B_BYTES / 16 / NT;                               // register-path chunks per thread
  constexpr int WTM = BM / WGM, WTN = BN / WGN, RM = WTM / 32, RN = WTN / 32;
  using MF = Mfma32<OT>;
  typedef typename MF::operand V;
  static_assert(S >= 2 && IA * 1024 * NW == A_BYTES && IB * 1024 * NW == B_BYTES && RB * 16 * NT == B_BYTES,
                "tile / wave count");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0 && BM % 128 == 0 && BN % 128 == 0, "tile");
  static_assert(!BREG || S16, "register-path operands belong to the standalone kernels");

  // XCD-aware renumbering: workgroup b runs on XCD b % 8; give every XCD a
  // contiguous range of tiles, first of the whole tiles, then (workgroups
  // numbered after all whole tiles, so dispatched last) of the k-split slices.
  const int b = blockIdx.x, n_whole = bt.start[bt.tail];
  const int gb = b < n_whole ? b : b - n_whole, gG = b < n_whole ? n_whole : (int)gridDim.x - n_whole;
  const int xcd = gb & 7, per = gG >> 3, rem = gG & 7;
  const int tile = (b < n_whole ? 0 : n_whole) + xcd * per + (xcd < rem ? xcd : rem) + (gb >> 3);
  int pi = 0;
#pragma unroll 1
  while (pi + 1 < bt.count && tile >= bt.start[pi + 1]) ++pi;
  const WideProblem& p = bt.p[pi];
  const int tn = (p.N + BN - 1) / BN;
  // k-split prediction: the tile's slice of the contraction
  const bool partial = MODE == WIDE_PRED && p.ksplit > 1;
  const int tmn = ((p.M + BM - 1) / BM) * tn;
  const int slice = partial ? (tile - bt.start[pi]) / tmn : 0;
  const int local = tile - bt.start[pi] - slice * tmn;
  const int kslice = partial ? p.K / p.ksplit : p.K;
  int mblk, nblk;
  supertile_pos(local, (p.M + BM - 1) / BM, tn, mblk, nblk);
  const int m0 = mblk * BM, n0 = nblk * BN;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w / WGN, wn = w % WGN;
  const OT* A = reinterpret_cast<const OT*>(p.a);
  const float* A32p = reinterpret_cast<const float*>(p.a);  // A32: the fp32 W
  const OT* Al = reinterpret_cast<const OT*>(p.a_lo);
  const OT* Bg = reinterpret_cast<const OT*>(p.b);
  const long long lda = p.lda, ldb = p.ldb;
  const int alim = p.a_lim, blim = p.b_lim;
  const int nk = kslice / WIDE_BK, kbase = slice * kslice;

  // stage i's A block (its A_lo block follows it) and B block
  auto a_stage = [&](int i) -> unsigned char* { return AX ? smem + i * A_BYTES : smem + i * STAGE; };
  auto b_stage = [&](int i) -> unsigned char* {
    return AX ? smem + SA * A_BYTES + i * B_BYTES : smem + i * STAGE + A_BYTES * A_BLOCKS;
  };
  auto issue_a = [&](int kt, unsigned char* st) {
    const int k0 = kbase + kt * WIDE_BK;
#pragma unroll
    for (int q = 0; q < IA; ++q) {
      const int blk = q * NW + w;
      if constexpr (A32) {
        const float* src = slot_src32<BM>(A32p, lda, m0, alim, k0, blk * 64 + lane);
        __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(st + blk * 1024), 16, 0, 0);
      } else {
        const OT* src = slot_src<OT, AMN, BM>(A, lda, m0, alim, k0, blk * 64 + lane);
        __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(st + blk * 1024), 16, 0, 0);
        if (LO) {
          const OT* srl = slot_src<OT, AMN, BM>(Al, lda, m0, alim, k0, blk * 64 + lane);
          __builtin_amdgcn_global_load_lds((glb_void*)srl, (lds_void*)(st + A_BYTES + blk * 1024), 16, 0, 0);
        }
      }
    }
  };
  auto issue_b = [&](int kt, unsigned char* st) {
    const int k0 = kbase + kt * WIDE_BK;
#pragma unroll
    for (int q = 0; q < IB; ++q) {
      const int blk = q * NW + w;
      const OT* src = slot_src<OT, BMN, BN>(Bg, ldb, n0, blim, k0, blk * 64 + lane);
      __builtin_amdgcn_global_load_lds((glb_void*)src, (lds_void*)(st + blk * 1024), 16, 0, 0);
    }
  };
  auto issue_dma = [&](int kt, int stage) {
    issue_a(kt, a_stage(stage));
    if (!BREG) issue_b(kt, b_stage(stage));
  };
  // register path of the B operand: 16-byte chunks of the stage's B block
  uint4 breg[BREG ? RB : 1];
  auto issue_breg = [&](int kt) {
    if (BREG) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
        breg[i] = *reinterpret_cast<const uint4*>(
            slot_src<OT, BMN, BN>(Bg, ldb, n0, blim, kbase + kt * WIDE_BK, i * NT + tid));
    }
  };
  auto store_breg = [&](int stage) {
    if (BREG) {
      unsigned char* sb = smem + stage * STAGE + A_BYTES * A_BLOCKS;
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const unsigned in[4] = {breg[i].x, breg[i].y, breg[i].z, breg[i].w};
        unsigned o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pack2(cvt<OT>(act_t<ACT>(lo16<OT>(in[j]))), cvt<OT>(act_t<ACT>(hi16<OT>(in[j]))));
        *reinterpret_cast<uint4*>(sb + (i * NT + tid) * 16) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  };

  // The epilogue's input (x for pred / infer, W for weight) is fetched now,
  // ahead of the main loop, in the row-major 4-column groups the epilogue
  // walks: its latency hides behind the MFMAs.
  constexpr int IT = BM * BN / 4 / NT, CH = IT < 8 ? IT : 8;
  static_assert(IT % CH == 0 && IT * 4 * NT == BM * BN, "epilogue groups");
  const int M = p.M, N = p.N;
  const bool vec = p.vec != 0;
  auto load_group = [&](const void* basev, long long ld, int u, float (&o)[4]) {
    const int idx = u * NT + tid;
    const int r = idx / (BN / 4), col = (idx % (BN / 4)) * 4;
    const int m = m0 + r, n = n0 + col;
    const int nv = (m < M && n < N) ? (N - n < 4 ? N - n : 4) : 0;
    if (S16) {
      const OT* src = reinterpret_cast<const OT*>(basev) + (long long)m * ld + n;
      if (vec && nv == 4) {
        const uint2 t2 = *reinterpret_cast<const uint2*>(src);
        o[0] = lo16<OT>(t2.x); o[1] = hi16<OT>(t2.x); o[2] = lo16<OT>(t2.y); o[3] = hi16<OT>(t2.y);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = q < nv ? to_f32(src[q]) : 0.0f;
      }
    } else {
      const float* src = reinterpret_cast<const float*>(basev) + (long long)m * ld + n;
      if (vec && nv == 4) {
        const float4 t4 = *reinterpret_cast<const float4*>(src);
        o[0] = t4.x; o[1] = t4.y; o[2] = t4.z; o[3] = t4.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = q < nv ? src[q] : 0.0f;
      }
    }
  };
  constexpr bool PRE = MODE != WIDE_FWD && !s16_fwd(MODE);
  constexpr bool REG = reg_epilogue(BM, BN, S, LO, S16);
  const bool pre_from_aux = MODE == WIDE_PRED || s16_pred(MODE);
  // the register epilogue loads its input block by block after the main loop
  // (fetched here, IT groups of 4 would take the accumulators' registers)
  constexpr bool PREF = PRE && !REG;
  float pre[PREF ? IT : 1][4];
  if (PREF && !partial) {
#pragma unroll
    for (int u = 0; u < IT; ++u)
      load_group(pre_from_aux ? p.aux : p.out, pre_from_aux ? p.ldx : p.ldo, u, pre[PREF ? u : 0]);
  }

  f32x16 acc[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

  // prologue: stages 0 .. S-2
#pragma unroll
  for (int s = 0; s < S - 1; ++s) {
    if (s < nk) {
      issue_breg(s);
      issue_dma(s, s);
      if (BREG) {
        wait_vmcnt<LPS>();
        store_breg(s);
      }
    }
  }
  if (AX && S - 1 < nk) issue_a(S - 1, a_stage(S - 1));  // the extra A stage's first fill

  // lane-constant parts of the fragment addresses
  const int lr = lane & 31, lk = lane >> 5;         // k-contiguous reads: row, 8-k half
  const int kc_sw = (lr >> 1) & 7;
  const int g4 = lane >> 4, li = lane & 15;          // transposing reads: 16-lane group, lane in group
  const int tr_row = 8 * (g4 >> 1) + (li >> 2);      // k-row within the 16-k slice (+4 for the second read)
  const int tr_low = 2 * (g4 & 1) + ((li & 3) >> 1); // chunk within the 4-chunk group of a 32-wide block
  const int tr_half = (li & 1) * 8, tr_x = li >> 2;  // byte in chunk, swizzle of the 4-chunk group
  auto frag_kc = [&](const unsigned char* blk, int row0, int kk) -> V {
    return *reinterpret_cast<const V*>(blk + (row0 + lr) * 128 + (((kk * 2 + lk) ^ kc_sw) << 4));
  };
  auto frag_mn = [&](const unsigned char* blk, int rowb, int col0, int kk) -> V {
    // col0: first column of the 32-wide block (multiple of 32)
    const int chunk = ((((col0 >> 5) ^ tr_x)) << 2) | tr_low;
    const unsigned char* p0 = blk + (kk * 16 + tr_row) * rowb + (chunk << 4) + tr_half;
    const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
    const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + 4 * rowb));
    const s16x8 v = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(V, v);
  };
  auto frag_a = [&](const unsigned char* blk, int i, int kk) -> V {
    if (AMN) return frag_mn(blk, BM * 2, wm * WTM + i * 32, kk);
    return frag_kc(blk, wm * WTM + i * 32, kk);
  };
  // A32: the 8 fp32 k-values of the lane (two 16-byte chunks of its row)
  // split into hi = cvt(w) and lo = cvt(w - hi), converted as a vector (packed
  // round-to-nearest-even conversions, the same bits as cvt of each value: the
  // values come from LDS, with no product the compiler could fold in)
  auto frag_a32 = [&](const unsigned char* blk, int i, int kk, V& hi, V& lo) {
    const unsigned char* rb = blk + (wm * WTM + i * 32 + lr) * 256;
    const int c0 = kk * 4 + lk * 2, sw = lr & 15;
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(rb + ((c0 ^ sw) << 4));
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(rb + (((c0 + 1) ^ sw) << 4));
    const f32x8 wv = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
    hi = __builtin_convertvector(wv, V);
    lo = __builtin_convertvector(wv - widen8(hi), V);  // w - hi is exact
  };
  auto frag_b = [&](const unsigned char* blk, int j, int kk) -> V {
    if (BMN) return frag_mn(blk, BN * 2, wn * WTN + j * 32, kk);
    return frag_kc(blk, wn * WTN + j * 32, kk);
  };

  int stage = 0, fill = S - 1, astage = 0;
#pragma unroll 1
  for (int kt = 0; kt < nk; ++kt) {
    if constexpr (AX) {
      // issue order per step: B(kt + 1), then A(kt + 2); step kt's A and B are
      // done once at most the last A fill, A(kt + 1), is in flight
      if (kt + 1 < nk) wait_vmcnt<IA>();
      else wait_vmcnt<0>();
    } else {
      // this wave's DMA loads of step kt are done once at most S-2 later steps are in flight
      if (kt + S - 2 < nk) wait_vmcnt<(S - 2) * LPS>();
      else wait_vmcnt<0>();
    }
    wg_barrier();
    const bool refill = kt + S - 1 < nk;
    if constexpr (AX) {
      if (refill) issue_b(kt + S - 1, b_stage(fill));
      if (kt + SA - 1 < nk) issue_a(kt + SA - 1, a_stage(astage == 0 ? SA - 1 : astage - 1));
    } else if (refill) {
      issue_breg(kt + S - 1);
      issue_dma(kt + S - 1, fill);
    }

    const unsigned char* sa = a_stage(AX ? astage : stage);
    const unsigned char* sal = sa + A_BYTES;
    const unsigned char* sb = b_stage(stage);
    V af[2][RM], bf[2][RN], alf[2][LO ? RM : 1];
    // Software pipeline over the 16-k slices of the stage: the reads of
    // slice kk+1 go out while slice kk's MFMAs run.  A scheduling barrier
    // between slices keeps the compiler from sinking the reads next to their
    // first use (which would expose the LDS latency once per MFMA pair).
#pragma unroll
    for (int j = 0; j < RN; ++j) bf[0][j] = frag_b(sb, j, 0);
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      if constexpr (A32) {
        frag_a32(sa, i, 0, af[0][i], alf[0][LO ? i : 0]);
      } else {
        af[0][i] = frag_a(sa, i, 0);
        if (LO) alf[0][i] = frag_a(sal, i, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < WIDE_BK / 16; ++kk) {
      const int cur = kk & 1, nxt = cur ^ 1;
      if (kk + 1 < WIDE_BK / 16) {
#pragma unroll
        for (int j = 0; j < RN; ++j) bf[nxt][j] = frag_b(sb, j, kk + 1);
#pragma unroll
        for (int i = 0; i < RM; ++i) {
          if constexpr (A32) {
            frag_a32(sa, i, kk + 1, af[nxt][i], alf[nxt][LO ? i : 0]);
          } else {
            af[nxt][i] = frag_a(sa, i, kk + 1);
            if (LO) alf[nxt][i] = frag_a(sal, i, kk + 1);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(af[cur][i], bf[cur][j], acc[i][j]);
      if (LO) {
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
          for (int j = 0; j < RN; ++j) acc[i][j] = MF::run(alf[cur][i], bf[cur][j], acc[i][j]);
      }
      if (kk + 1 < WIDE_BK / 16) {
        // one LDS read between consecutive MFMAs, as far as the reads go
        constexpr int NLD = RM * (LO ? 2 : 1) * (AMN ? 2 : 1) + RN * (BMN ? 2 : 1);
        constexpr int NMF = RM * RN * (LO ? 2 : 1);
#pragma unroll
        for (int q = 0; q < NMF; ++q) {
          if (q < NLD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        if (NLD > NMF) __builtin_amdgcn_sched_group_barrier(0x100, NLD > NMF ? NLD - NMF : 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (BREG && refill) {
      // the register loads were issued before this step's DMA loads
      wait_vmcnt<LPS>();
      store_breg(fill);
    }
    stage = stage + 1 == S ? 0 : stage + 1;
    fill = fill + 1 == S ? 0 : fill + 1;
    astage = astage + 1 == SA ? 0 : astage + 1;
  }

  // ------------------------------------------------------------ epilogue
  if (partial) {
    // raw partial product of this slice; lanes 0-31 of a row store 32
    // consecutive columns
    float* po = reinterpret_cast<float*>(p.out) + slice * p.part_stride;
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int m = m0 + wm * WTM + i * 32 + 8 * (q >> 2) + 4 * lk + (q & 3);
          const int n = n0 + wn * WTN + j * 32 + lr;
          if (m < M && n < N) po[(long long)m * p.ldo + n] = acc[i][j][q];
        }
    return;
  }
  if constexpr (REG) {
    // Register epilogue (wide configurations whose fp32 tile exceeds the
    // LDS): every element is finished in the accumulator layout (lane column
    // elr = lane % 32, rows 8 g + 4 elk + 0..3 of each 32 x 32 block) with
    // the rounding steps of the LDS path below; the fp32 masters and the
    // natural 16-bit copy are stored from the registers (32 lanes: 128 / 64
    // contiguous bytes of one row), through buffer resources, so that an
    // element's address is the lane's offset plus the register's uniform row
    // step.  The 16-bit transposed copy is staged in LDS as a [BN][BM] tile
    // (16-byte chunk c of row n at chunk c ^ (n % 32): conflict-free for both
    // passes, BM >= 256) and then written row by row, 16 bytes per lane.
    // The standalone kernels' inputs and outputs are 16-bit (their rounding
    // steps are those of the LDS path) and they have no transposed copy.
    static_assert(BM >= 256 && BN * BM * (int)sizeof(OT) <= stage_bytes(BM, BN, S, LO), "transposed tile");
    const int elr = lane & 31, elk = lane >> 5;
    constexpr bool EIN = MODE == WIDE_INFER || s16_infer(MODE);
    constexpr unsigned ES = S16 ? (unsigned)sizeof(OT) : 4u;  // bytes of an input, output or out2 element
    const long long xld = pre_from_aux ? p.ldx : p.ldo;
    const Buf bx(pre_from_aux ? p.aux : p.out, PRE ? (long long)M * xld * ES : 0);
    const Buf be(p.aux, EIN ? (long long)M * p.ldx * ES : 0);
    const Buf bo(p.out, (long long)M * p.ldo * ES);
    const Buf bh(p.h, !S16 && p.h ? (long long)M * p.ldh * (long long)sizeof(OT) : 0);
    const Buf bl(p.hl, !S16 && p.hl ? (long long)M * p.ldhl * (long long)sizeof(OT) : 0);
    const Buf b2(p.out2, p.out2 ? (long long)M * p.ld2 * ES : 0);
    auto ldin = [&](const Buf& b, unsigned v, unsigned s) -> float {
      if constexpr (S16) return to_f32(__builtin_bit_cast(OT, b.ld16(v, s)));
      else return b.ld32(v, s);
    };
    unsigned short* tl = reinterpret_cast<unsigned short*>(smem);
    wait_vmcnt<0>();
    __syncthreads();  // every wave is done with the pipeline stages
    auto qrow = [](int q) { return 8 * (q >> 2) + (q & 3); };
    if constexpr (S16) {
      // Standalone calls (16-bit inputs and outputs, no copies): a two-deep
      // pipeline over the wave's RM x RN accumulator blocks, the inputs of
      // block b + 1 in flight while block b is finished (256 x 256 tiles at
      // 8192^3: 5-10 % faster than loading each block just before it, the
      // form the wide path below keeps: its fp32 epilogues are bound by HBM
      // traffic and measured 2-4 us slower pipelined).  A lane whose column
      // is past N loads its row's first element instead (in range exactly
      // when the row's other elements are) and never stores the result, so
      // the loads need no branch.
      constexpr int NBK = RM * RN;
      const long long s_ldo = p.ldo, s_ld2 = p.ld2;
      const float s_scal = p.scal;
      const bool s_out2 = s16_infer(MODE) && p.out2 != nullptr;
      float xin[2][PRE ? 16 : 1], ein[2][EIN ? 16 : 1];
      auto load_block = [&](int bk, float (&xo)[PRE ? 16 : 1], float (&eo)[EIN ? 16 : 1]) {
        const int n = n0 + wn * WTN + (bk % RN) * 32 + elr, nn = n < N ? n : 0;
        const int mb = m0 + wm * WTM + (bk / RN) * 32 + 4 * elk;
        const unsigned vx = (unsigned)(mb * xld + nn) * ES, ve = (unsigned)(mb * p.ldx + nn) * ES;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          if constexpr (PRE) xo[PRE ? q : 0] = ldin(bx, vx, (unsigned)(qrow(q) * xld) * ES);
          if constexpr (EIN) eo[EIN ? q : 0] = ldin(be, ve, (unsigned)(qrow(q) * p.ldx) * ES);
        }
      };
      load_block(0, xin[0], ein[0]);
#pragma unroll
      for (int bk = 0; bk < NBK; ++bk) {
        if (bk + 1 < NBK) load_block(bk + 1, xin[(bk + 1) & 1], ein[(bk + 1) & 1]);
        const int i = bk / RN, j = bk % RN, cur = bk & 1;
        const int n = n0 + wn * WTN + j * 32 + elr, mb = m0 + wm * WTM + i * 32 + 4 * elk;
        if (n >= N) continue;
        const unsigned vo = (unsigned)(mb * s_ldo + n) * ES, v2 = (unsigned)(mb * s_ld2 + n) * ES;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
#pragma clang fp contract(off)
          const float a = acc[i][j][q];
          const float x = PRE ? xin[cur][PRE ? q : 0] : 0.0f;
          OT hv, lv;
          if (s16_pred(MODE)) {
            // tilelang_kernels.py:173: E = cast(X_lower) - cast(acc) in storage precision
            hv = cvt<OT>(x - to_f32(cvt<OT>(a)));
          } else if (s16_fwd(MODE)) {
            hv = cvt<OT>(a);
          } else if (s16_infer(MODE)) {
            const float xn = x + s_scal * (-ein[cur][EIN ? q : 0] + dact_t<ACT>(x) * a);
            hv = cvt<OT>(xn);
            lv = cvt<OT>(act_t<ACT>(xn));                              // A_out
          } else {
            // tilelang_kernels.py:319-320: W = cast(float(W) + alpha * acc)
            hv = cvt<OT>(x + s_scal * a);
          }
          const unsigned r = (unsigned)qrow(q);
          bo.st16(__builtin_bit_cast(unsigned short, hv), vo, r * (unsigned)s_ldo * ES);
          if (s_out2) b2.st16(__builtin_bit_cast(unsigned short, lv), v2, r * (unsigned)s_ld2 * ES);
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j) {
        const int nl = wn * WTN + j * 32 + elr, n = n0 + nl;
        const int ml0 = wm * WTM + i * 32 + 4 * elk, mb = m0 + ml0;
        const bool ncol = n < N;
        float xin[PRE ? 16 : 1], ein[EIN ? 16 : 1];
        const unsigned vx = (unsigned)(mb * xld + n) * ES, ve = (unsigned)(mb * p.ldx + n) * ES;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          if constexpr (PRE) xin[PRE ? q : 0] = ncol ? ldin(bx, vx, (unsigned)(qrow(q) * xld) * ES) : 0.0f;
          if constexpr (EIN) ein[EIN ? q : 0] = ncol ? ldin(be, ve, (unsigned)(qrow(q) * p.ldx) * ES) : 0.0f;
        }
        const unsigned vo = (unsigned)(mb * p.ldo + n) * ES, vh = (unsigned)(mb * p.ldh + n) * (unsigned)sizeof(OT),
                       vl = (unsigned)(mb * p.ldhl + n) * (unsigned)sizeof(OT), v2 = (unsigned)(mb * p.ld2 + n) * ES;
        unsigned short hs[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
#pragma clang fp contract(off)
          const float a = acc[i][j][q];
          const float x = PRE ? xin[PRE ? q : 0] : 0.0f;
          float v, fv = 0.0f;
          OT hv, lv;
          if (MODE == WIDE_PRED) {
            v = x - a;                                                // eps
            hv = cvt<OT>(v);
          } else if (MODE == WIDE_INFER) {
            v = x + p.scal * (-ein[EIN ? q : 0] + dact_t<ACT>(x) * a);  // x_new
            fv = act_t<ACT>(v);
            hv = cvt<OT>(fv);
          } else if (MODE == WIDE_FWD) {
            v = a;                                                    // x = W f(x_upper)
            fv = act_t<ACT>(v);
            hv = cvt<OT>(fv);
          } else if (MODE == WIDE_WEIGHT) {
            v = x + p.scal * a;                                       // W_new
            hv = cvt<OT>(v);
            lv = cvt<OT>(v - to_f32(hv));
          } else if (s16_pred(MODE)) {
            // tilelang_kernels.py:173: E = cast(X_lower) - cast(acc) in storage precision
            hv = cvt<OT>(x - to_f32(cvt<OT>(a)));
          } else if (s16_fwd(MODE)) {
            hv = cvt<OT>(a);
          } else if (s16_infer(MODE)) {
            const float xn = x + p.scal * (-ein[EIN ? q : 0] + dact_t<ACT>(x) * a);
            hv = cvt<OT>(xn);
            lv = cvt<OT>(act_t<ACT>(xn));                              // A_out
          } else {
            // tilelang_kernels.py:319-320: W = cast(float(W) + alpha * acc)
            hv = cvt<OT>(x + p.scal * a);
          }
          const unsigned r = (unsigned)qrow(q);
          if (ncol) {
            if constexpr (S16) {
              bo.st16(__builtin_bit_cast(unsigned short, hv), vo, r * (unsigned)p.ldo * ES);
              if (s16_infer(MODE) && p.out2) b2.st16(__builtin_bit_cast(unsigned short, lv), v2, r * (unsigned)p.ld2 * ES);
            } else {
              bo.st32(v, vo, r * (unsigned)p.ldo * 4u);
              if (MODE != WIDE_WEIGHT || p.h) bh.st16(__builtin_bit_cast(unsigned short, hv), vh, r * (unsigned)p.ldh * (unsigned)sizeof(OT));
              if (MODE == WIDE_WEIGHT && p.hl) bl.st16(__builtin_bit_cast(unsigned short, lv), vl, r * (unsigned)p.ldhl * (unsigned)sizeof(OT));
              if (MODE == WIDE_INFER && p.out2) b2.st32(fv, v2, r * (unsigned)p.ld2 * 4u);
            }
          }
          hs[q] = mb + (int)r < M ? __builtin_bit_cast(unsigned short, hv) : (unsigned short)0;  // padding stays zero
        }
        if constexpr (S16) continue;
        // rows 8 g + 4 elk + (0, 1) and (2, 3): two 4-byte LDS stores per group
#pragma unroll
        for (int q = 0; q < 16; q += 2) {
          const int ml = ml0 + qrow(q);
          *reinterpret_cast<unsigned*>(tl + nl * BM + ((((ml >> 3) ^ (nl & 31))) << 3) + (ml & 7)) =
              (unsigned)hs[q] | ((unsigned)hs[q + 1] << 16);
        }
      }
    if (S16 || !p.t) return;
    __syncthreads();
    OT* tcopy = reinterpret_cast<OT*>(p.t);
#pragma unroll 4
    for (int idx = tid; idx < BN * BM / 8; idx += NT) {
      const int nl = idx / (BM / 8), c = idx % (BM / 8);
      const int n = n0 + nl, m = m0 + c * 8;
      if (n < N && m < M)  // the chunk's rows at or past M hold zeros (the copy's padding)
        *reinterpret_cast<uint4*>(tcopy + (long long)n * p.ldt + m) =
            *reinterpret_cast<const uint4*>(tl + nl * BM + ((c ^ (nl & 31)) << 3));
    }
    return;
  }
  // The accumulator tile goes through LDS (the pipeline stages are free now)
  // so that every global access of the epilogue is coalesced: pass 1 walks
  // the tile row-major, 4 columns per thread (fp32 master, natural 16-bit
  // copy), pass 2 column-major (the transposed 16-bit copy of the wide path).
  constexpr int CS = BN + 1;  // fp32 row stride: conflict-free column walk in pass 2
  static_assert(REG || BM * CS * 4 <= smem_bytes(BM, BN, S, LO), "epilogue tile exceeds the LDS");
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

#pragma unroll
  for (int c0 = 0; c0 < IT; c0 += CH) {
    float ein[CH][4];
    if (MODE == WIDE_INFER || s16_infer(MODE)) {
#pragma unroll
      for (int u = 0; u < CH; ++u) load_group(p.aux, p.ldx, c0 + u, ein[u]);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int idx = (c0 + u) * NT + tid;
      const int r = idx / (BN / 4), col = (idx % (BN / 4)) * 4;
      const int m = m0 + r, n = n0 + col;
      if (m >= M || n >= N) continue;
      const int nv = N - n < 4 ? N - n : 4;
      float* cr = cs + r * CS + col;
      float v[4], fv[4];
      OT hv[4], lv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
        const float a = cr[q];
        const float x = PREF ? pre[PREF ? c0 + u : 0][q] : 0.0f;
        if (MODE == WIDE_PRED) {
          v[q] = x - a;                                              // eps
          hv[q] = cvt<OT>(v[q]);
        } else if (MODE == WIDE_INFER) {
          v[q] = x + p.scal * (-ein[u][q] + dact_t<ACT>(x) * a);    // x_new
          fv[q] = act_t<ACT>(v[q]);
          hv[q] = cvt<OT>(fv[q]);
        } else if (MODE == WIDE_FWD) {
          v[q] = a;                                                  // x = W f(x_upper)
          fv[q] = act_t<ACT>(v[q]);
          hv[q] = cvt<OT>(fv[q]);
        } else if (MODE == WIDE_WEIGHT) {
          v[q] = x + p.scal * a;                                     // W_new
          hv[q] = cvt<OT>(v[q]);
          lv[q] = cvt<OT>(v[q] - to_f32(hv[q]));
        } else if (s16_pred(MODE)) {
          // tilelang_kernels.py:173: E = cast(X_lower) - cast(acc) in storage precision
          hv[q] = cvt<OT>(x - to_f32(cvt<OT>(a)));
        } else if (s16_fwd(MODE)) {
          hv[q] = cvt<OT>(a);
        } else if (s16_infer(MODE)) {
          const float xn = x + p.scal * (-ein[u][q] + dact_t<ACT>(x) * a);
          hv[q] = cvt<OT>(xn);
          lv[q] = cvt<OT>(act_t<ACT>(xn));                            // A_out
        } else {
          // tilelang_kernels.py:319-320: W = cast(float(W) + alpha * acc)
          hv[q] = cvt<OT>(x + p.scal * a);
        }
        if (!S16) cr[q] = to_f32(hv[q]);  // the value the transposed copy takes
      }
      if (!S16) {
        float* op = reinterpret_cast<float*>(p.out) + (long long)m * p.ldo + n;
        OT* hp = reinterpret_cast<OT*>(p.h) + (long long)m * p.ldh + n;
        if (vec && nv == 4) {
          *reinterpret_cast<float4*>(op) = make_float4(v[0], v[1], v[2], v[3]);
          uint2 hh; hh.x = pack2(hv[0], hv[1]); hh.y = pack2(hv[2], hv[3]);
          if (MODE != WIDE_WEIGHT || p.h) *reinterpret_cast<uint2*>(hp) = hh;
          if (MODE == WIDE_WEIGHT && p.hl) {
            uint2 ll; ll.x = pack2(lv[0], lv[1]); ll.y = pack2(lv[2], lv[3]);
            *reinterpret_cast<uint2*>(reinterpret_cast<OT*>(p.hl) + (long long)m * p.ldhl + n) = ll;
          }
          if (MODE == WIDE_INFER && p.out2)
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out2) + (long long)m * p.ld2 + n) =
                make_float4(fv[0], fv[1], fv[2], fv[3]);
        } else {
          for (int q = 0; q < nv; ++q) {
            op[q] = v[q];
            if (MODE != WIDE_WEIGHT || p.h) hp[q] = hv[q];
            if (MODE == WIDE_WEIGHT && p.hl) reinterpret_cast<OT*>(p.hl)[(long long)m * p.ldhl + n + q] = lv[q];
            if (MODE == WIDE_INFER && p.out2) reinterpret_cast<float*>(p.out2)[(long long)m * p.ld2 + n + q] = fv[q];
          }
        }
      } else {
        OT* op = reinterpret_cast<OT*>(p.out) + (long long)m * p.ldo + n;
        OT* o2 = s16_infer(MODE) && p.out2 ? reinterpret_cast<OT*>(p.out2) + (long long)m * p.ld2 + n : nullptr;
        if (vec && nv == 4) {
          uint2 hh; hh.x = pack2(hv[0], hv[1]); hh.y = pack2(hv[2], hv[3]);
          *reinterpret_cast<uint2*>(op) = hh;
          if (o2) {
            uint2 ll; ll.x = pack2(lv[0], lv[1]); ll.y = pack2(lv[2], lv[3]);
            *reinterpret_cast<uint2*>(o2) = ll;
          }
        } else {
          for (int q = 0; q < nv; ++q) {
            op[q] = hv[q];
            if (o2) o2[q] = lv[q];
          }
        }
      }
    }
  }
  if (S16 || !p.t) return;
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

// Host-side check of one problem, made for every problem of a launch before
// any HIP call.  A split-2 kernel that does not split the fp32 W itself (A32)
// DMA-loads an A_lo block next to every A block (prediction and forward
// alike), so a problem without A_lo would make every workgroup read through a
// null pointer: a GPU memory fault, not an error code.  A k-split prediction
// slice must be a whole number of k-steps.
inline bool problem_ok(int mode, int split, bool a32, const WideProblem& q) {
  if (split == 2 && !a32 && !q.a_lo) return false;
  const int ks = mode == WIDE_PRED && q.ksplit > 1 ? q.ksplit : 1;
  if (ks > 1 && q.K % (ks * WIDE_BK) != 0) return false;
  return true;
}

// One kernel configuration: LDS limit set once per process, launch over a
// ragged batch of up to WIDE_MAX_BATCH problems.
template <typename OT, int MODE, int SPLIT, int ACT, bool BREG, int BM, int BN, int S, int WGM, int WGN,
          bool A32 = false>
struct Cfg {
  static constexpr int smem = a32_extra_stage(BM, BN, S, A32)
                                  ? (S + 1) * BM * 256 + S * BN * 128 > smem_bytes(BM, BN, S, true, false)
                                        ? (S + 1) * BM * 256 + S * BN * 128
                                        : smem_bytes(BM, BN, S, true, false)
                                  : smem_bytes(BM, BN, S, SPLIT == 2, is_s16(MODE));
  static_assert(smem <= 160 * 1024, "a configuration's LDS exceeds the CU's 160 KB");
  static constexpr int BM_ = BM, BN_ = BN;
  static const void* fn() {
    return reinterpret_cast<const void*>(&dma_gemm_kernel<OT, MODE, SPLIT, ACT, BREG, BM, BN, S, WGM, WGN, A32>);
  }
  static hipError_t prepare() {
    static const hipError_t e = hipFuncSetAttribute(fn(), hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    return e;
  }
  static hipError_t launch(const WideProblem* probs, int count, hipStream_t s) {
    for (int i = 0; i < count; ++i)
      if (!problem_ok(MODE, SPLIT, A32, probs[i])) return hipErrorInvalidValue;
    const hipError_t pe = prepare();
    if (pe != hipSuccess) return pe;
    Batch bt;
    bt.count = count;
    bt.tail = count;
    int total = 0;
    for (int i = 0; i < count; ++i) {
      const int ks = MODE == WIDE_PRED && probs[i].ksplit > 1 ? probs[i].ksplit : 1;
      if (ks > 1) {
        if (bt.tail == count) bt.tail = i;
      } else if (bt.tail != count) {
        return hipErrorInvalidValue;  // k-split problems must come last
      }
      bt.p[i] = probs[i];
      bt.start[i] = total;
      total += ((probs[i].M + BM - 1) / BM) * ((probs[i].N + BN - 1) / BN) * ks;
    }
    for (int i = count; i <= WIDE_MAX_BATCH; ++i) bt.start[i] = total;
    if (total == 0) return hipSuccess;
    void* args[] = {&bt};
    return hipLaunchKernel(fn(), dim3(total), dim3(WGM * WGN * 64), args, smem, s);
  }
};

// Calls F<ACT>::run(args...) for the runtime activation code.
template <template <int> class F, typename... Args>
hipError_t by_act(int act, Args... a) {
  switch (act) {
    case ACT_RELU: return F<ACT_RELU>::run(a...);
    case ACT_TANH: return F<ACT_TANH>::run(a...);
    case ACT_SIGMOID: return F<ACT_SIGMOID>::run(a...);
    case ACT_SILU: return F<ACT_SILU>::run(a...);
    case ACT_GELU: return F<ACT_GELU>::run(a...);
    default: return F<ACT_IDENTITY>::run(a...);
  }
}

}  // namespace dma
}  // namespace ipc
