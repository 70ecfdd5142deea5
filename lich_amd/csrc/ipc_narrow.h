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

// Number of 64x64 weight-update tiles of all layers.
int narrow_tiles(const int* dims, int L);

// Dynamic LDS bytes of the whole-step kernel for this operand type / split.
int narrow_lds_bytes(const int* dims, int L, int operand, int split);

// Raises the dynamic-LDS limit of the kernel instantiation a plan uses.
hipError_t narrow_prepare(int operand, int split, int act, int lds_bytes);

// `operand` is a DT_* code, `split` 1 or 3 (16-bit operands only).
hipError_t launch_narrow(const NarrowArgs& p, int operand, int split, hipStream_t s);

}  // namespace ipc
