// ipc_narrow.h - host interface of the whole-step kernel for narrow nets.
#pragma once

#include <hip/hip_runtime.h>

namespace ipc {

constexpr int NARROW_MAX_L = 16;        // weight matrices
constexpr int NARROW_MAX_WIDTH = 128;   // every output width d_0 .. d_{L-1}
constexpr int NARROW_OUTER_MAX_B = 16;  // batch limit of the rank-B outer-product phase B
constexpr int NARROW_NC = 16;           // batch columns per column block
constexpr int NARROW_MAX_UNITS = NARROW_MAX_L * (NARROW_MAX_WIDTH / 16);
constexpr int NARROW_LDS_LIMIT = 160 * 1024;
// Both whole-step kernels accumulate a prediction contraction in partials of
// this many columns, summed in order (one layer-resident workgroup per
// partial of the top layer).
constexpr int NARROW_KCHUNK = 128;

enum { NMODE_STEPS = 0, NMODE_PHASE_A = 1, NMODE_PHASE_B = 2, NMODE_FORWARD = 3 };

struct NarrowArgs {
  int L, B, act, mode, steps, nblocks, spin_limit, outer;
  float alpha, gamma;
  int lds_bytes;
  int n_units;                                  // prediction units (layer, row tile)
  int dims[NARROW_MAX_L + 1];
  int wtile_start[NARROW_MAX_L + 1];            // prefix sums of 64x64 weight tiles per layer
  unsigned char unit_l[NARROW_MAX_UNITS];       // prediction units, longest first
  unsigned char unit_rt[NARROW_MAX_UNITS];
  float* x[NARROW_MAX_L + 1];
  float* e[NARROW_MAX_L + 1];
  float* w[NARROW_MAX_L];
  float* a[NARROW_MAX_L + 1];  // saved activations (save mode) or nullptr
  float* fx[NARROW_MAX_L + 1]; // f(x[l]) as read by phase B: a[l] in save mode, else workspace
  unsigned* bar;               // workspace: [0] arrivals, [1] exits, [2] barrier timeout flag
  unsigned* res_image_flag;    // layer-resident plans: the cache generation every launch bumps, else nullptr
};

// Workspace bytes of a plan: 256 bytes of barrier counters, then (recompute
// mode) one fp32 [d_l, B] buffer per l = 1..L for the pre-evaluated f(x[l]).
inline long long narrow_workspace_bytes(const int* dims, int L, int B, bool recompute) {
  long long total = 256;
  if (recompute)
    for (int l = 1; l <= L; ++l) total += ((long long)dims[l] * B * 4 + 255) / 256 * 256;
  return total;
}

// Offsets (in bytes from the dynamic LDS base) of the phase-A buffers of one
// column block.  KS / PAD / esize are those of the operand type (fp32: 16, 4,
// 4; fp16/bf16: 32, 8, 2); split3 doubles the staged f(x) for its lo terms.
//   xr  fp32 [row][NC]  raw x[l], l < L              (row = offset + r)
//   ef  fp32 [row][NC]  eps[l], 1 <= l < L
//   fs  OT   [NC][ldk(d_l)] f(x[l]) hi (and lo) per l = 1..L
//   es  OT   [NC][ldk(d_l)] eps[l] per l = 0..L-2 (B operand of inference)
//   outer fp32 2 x [64][NC+1]  phase-B rank-B staging
struct NarrowLds {
  int xr_row[NARROW_MAX_L + 1];   // row offset of layer l in xr
  int ef_row[NARROW_MAX_L + 1];
  int fs_off[NARROW_MAX_L + 2];   // element offset of layer l's hi block (lo follows it)
  int es_off[NARROW_MAX_L + 1];
  int xr_bytes, ef_base, fs_base, es_base, outer_base, total;
};

__host__ __device__ inline int narrow_ldk(int d, int KS, int PAD) { return (d + KS - 1) / KS * KS + PAD; }

__host__ __device__ inline void narrow_lds_layout(const int* dims, int L, int KS, int PAD, int esize, bool split3,
                                                  NarrowLds& o) {
  int r = 0;
  for (int l = 0; l < L; ++l) { o.xr_row[l] = r; r += dims[l]; }
  o.xr_bytes = r * NARROW_NC * 4;
  int er = 0;
  for (int l = 1; l < L; ++l) { o.ef_row[l] = er; er += dims[l]; }
  o.ef_base = o.xr_bytes;
  o.fs_base = o.ef_base + er * NARROW_NC * 4;
  int f = 0;
  for (int l = 1; l <= L; ++l) {
    o.fs_off[l] = f;
    f += NARROW_NC * narrow_ldk(dims[l], KS, PAD) * (split3 ? 2 : 1);
  }
  o.es_base = o.fs_base + ((f * esize + 15) / 16) * 16;
  int e = 0;
  for (int l = 0; l + 1 < L; ++l) { o.es_off[l] = e; e += NARROW_NC * narrow_ldk(dims[l], KS, PAD); }
  // phase-B outer-product staging gets its own region: in a multi-step launch
  // the phase-A buffers above stay resident across steps
  o.outer_base = o.es_base + ((e * esize + 15) / 16) * 16;
  o.total = o.outer_base + 2 * 64 * (NARROW_NC + 1) * 4;
}

// ---------------------------------------------------------------- layer-resident kernel
// Multi-step launches of nets whose hidden widths are <= 64 run a second
// whole-step kernel in which every workgroup owns one layer's W for all steps
// (the top layer's W, with its long input-width contraction, is split into
// column chunks owned by one workgroup each) and exchanges only eps and
// f'(x) W^T eps with its neighbours: 16-bit operands with the GEMM weight update
// (B <= 128), and fp32 operands with either weight update while the operand
// blocks fit the LDS (B <= 64 at width 64).
constexpr int RES_MAX_WIDTH = 64;   // d_0 .. d_{L-1}
constexpr int RES_MAX_B = 128;
constexpr int RES_MAX_WG = 63;      // word 63 of the flag area is the cache generation
constexpr int RES_FLAG_BYTES = 512;  // flag area: step flags, generation, per-workgroup cache slots
constexpr int RES_TILE = 256;       // floats per exchanged 16x16 tile (64 lanes x 4)
constexpr int RES_TOP_ROWS = 32;    // default rows of W[L-1] per top workgroup (a 64-row layer takes two)

struct ResidentArgs {
  int L, B, steps, nwg, chunks, kc, spin_limit, lds_bytes;
  int halves;                   // top-layer row blocks of top_rows (one workgroup per chunk and block)
  int top_rows;                 // rows of W[L-1] per top workgroup: 16, 32 (default) or 64
  int outer;                    // weight update as a rank-B outer product on the VALU (fp32 operands, B <= 16)
  float alpha, gamma;
  int dims[NARROW_MAX_L + 1];
  float* x[NARROW_MAX_L + 1];
  float* e[NARROW_MAX_L + 1];
  float* w[NARROW_MAX_L];
  float* fx[NARROW_MAX_L + 1];  // f(x[l]) written at the end (a[l] in save mode)
  float* xe[NARROW_MAX_L];      // eps[l], l = 1..L-2:        [2][tiles(d_l)][RES_TILE]
  float* xg[NARROW_MAX_L];      // f'(x[l+1]) W[l]^T eps[l], l = 0..L-2: [2][tiles(d_{l+1})][RES_TILE]
  float* xp;                    // top-layer partial products: [2][chunks][tiles(d_{L-1})][RES_TILE]
  float* xs;                    // eps[L-1] as summed by each row block's chunk 0: [2][tiles(d_{L-1})][RES_TILE]
  float* xn;                    // the top-layer partial products of the next launch's first step, computed
                                // with the final W at the end of a launch: [chunks][tiles(d_{L-1})][RES_TILE]
  char* image;                  // per top chunk: its f(x[L]) operand LDS image, image_stride bytes apart
  long long image_stride;
  unsigned* flags;              // [nwg] steps each workgroup has published (counted across launches),
                                // [nwg + h] those whose eps[L-1] rows top chunk 0 of row block h has
                                // published; [RES_MAX_WG] cache generation, [RES_MAX_WG + 1 + w]
                                // generation + 1 once workgroup w's cached operands are current
  unsigned* bar;                // [2] wait timeout flag (shared with the column kernel)
};

// LDS layout of one workgroup (element offsets, in operand elements of
// `esize` bytes).  M x K is the workgroup's block of W; `hidden` workgroups
// also hold W^T and eps in the inference operand layout.  Contraction extents
// are padded to the MFMA k-step (KP: 32 for 16-bit operands, 16 for fp32) and
// output extents to 16; every row is padded by KP / 4 elements (16 bytes).
//   wh, wl  [M16][KkP+pad]  W hi / lo          (prediction A)
//   wt      [K16][MkP+pad]  W^T hi             (inference A, hidden only)
// (16-bit hidden workgroups: no wh; wt holds KkP rows and is read transposed
// as the prediction A as well; wl is W^T lo in wt's layout; no ft or ea, below)
//   fh, fl  [B16][KkP+pad]  f(x upper) hi / lo (prediction B)
//   ft      [K16][BkP+pad]  f(x upper) hi      (weight-update B)
//   eb      [B16][MkP+pad]  eps                (inference B, hidden only)
//   ea      [M16][BkP+pad]  eps                (weight-update A)
struct ResidentLds {
  int ldw, ldwt, ldf, ldft, lde, lda;
  int wh, wl, wt, fh, fl, ft, eb, ea, bytes;
};

__host__ __device__ inline int res_round(int v, int m) { return (v + m - 1) / m * m; }

__host__ __device__ inline void resident_lds_layout(int M, int K, int B, bool hidden, bool split3, int esize,
                                                    ResidentLds& o) {
  const int KP = esize == 4 ? 16 : 32, pad = KP / 4;
  const int M16 = res_round(M, 16), MP = res_round(M, KP), K16 = res_round(K, 16), KK = res_round(K, KP);
  const int B16 = res_round(B, 16), BP = res_round(B, KP);
  o.ldw = KK + pad; o.ldwt = MP + pad; o.ldf = KK + pad; o.ldft = BP + pad; o.lde = MP + pad; o.lda = BP + pad;
  // 16-bit hidden workgroups read the prediction's W operand from wt and the
  // weight update's operands from fh and eb with transposing LDS loads, and
  // keep no wh, ft or ea; wt (and wl, W^T lo in wt's layout) then hold the
  // prediction's KK contraction rows, fh and eb the update's BP (rows past
  // the matrix zero)
  const bool trh = hidden && esize == 2;
  int at = 0;
  o.wh = at; if (!trh) at += M16 * o.ldw;
  o.wl = at; if (split3) at += trh ? KK * o.ldwt : M16 * o.ldw;
  o.wt = at; if (hidden) at += (trh ? KK : K16) * o.ldwt;
  o.fh = at; at += (trh ? BP : B16) * o.ldf;
  o.fl = at; if (split3) at += B16 * o.ldf;
  o.ft = at; if (!trh) at += K16 * o.ldft;
  o.eb = at; if (hidden) at += (trh ? BP : B16) * o.lde;
  o.ea = at; if (!trh) at += M16 * o.lda;
  o.bytes = at * esize;
}

// Exchanged 16x16 tiles of a [d][B] matrix.
inline int resident_tiles(int d, int B) { return ((d + 15) / 16) * ((B + 15) / 16); }

// Plan of the layer-resident kernel for dims / B (operands of `esize` bytes:
// 2 with split 1 or 3, 4 with split 1; `outer`: the rank-B weight update,
// fp32 operands and B <= NARROW_OUTER_MAX_B only): fills chunks
// (NARROW_KCHUNK columns of the top layer each), kc, nwg, outer and
// lds_bytes of `a` and returns the workspace bytes its flags and exchange
// buffers need, or -1 when the net is not eligible.
long long resident_plan(const int* dims, int L, int B, int split, int esize, bool outer, int top_rows,
                        ResidentArgs& a);

// Lays the flags, exchange buffers and input images out in `ws` (resident_plan's bytes).
void resident_bind(ResidentArgs& a, char* ws);

// Marks the top chunks' cached f(x[L]) images stale (x[L] was rewritten).
hipError_t resident_invalidate(const ResidentArgs& a, hipStream_t s);

hipError_t resident_prepare(int operand, int split, int act, int lds_bytes);
// Workgroups one launch of the layer-resident kernel starts (the working
// ones and the spare blocks of its XCD-aware grid): all of them must be able
// to run at once.
int resident_launch_blocks(const ResidentArgs& a);
// Workgroups of the plan's instantiation that one CU can hold at once.
hipError_t resident_occupancy(int operand, int split, int act, int lds_bytes, int* per_cu);
hipError_t launch_resident(const ResidentArgs& a, int operand, int split, int act, hipStream_t s);

// Number of 64x64 weight-update tiles of all layers.
int narrow_tiles(const int* dims, int L);

// Dynamic LDS bytes of the whole-step kernel for this operand type / split.
int narrow_lds_bytes(const int* dims, int L, int operand, int split);

// Raises the dynamic-LDS limit of the kernel instantiation a plan uses.
hipError_t narrow_prepare(int operand, int split, int act, int lds_bytes);
// Workgroups of that instantiation that one CU can hold at once.
hipError_t narrow_occupancy(int operand, int split, int act, int lds_bytes, int* per_cu);

// `operand` is a DT_* code, `split` 1 or 3 (16-bit operands only).
hipError_t launch_narrow(const NarrowArgs& p, int operand, int split, hipStream_t s);

}  // namespace ipc
