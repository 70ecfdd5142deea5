// ipc_launch.h - host-side launch interface between the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace ipc {

// Which fused epilogue (and operand layout) a GEMM launch uses.
enum GemmKind {
  KIND_PRED = 0,    // E = X_lower - W f(X_upper)        A = W [M][K],  B = X_upper [K][N]
  KIND_FWD = 1,     // OUT = W f(X_upper)                 same operands as KIND_PRED
  KIND_INFER = 2,   // X += g(-E + f'(X) W_lo^T E_lo)     A = W_lower [K][M] (read transposed), B = E_lower [K][N]
  KIND_WEIGHT = 3,  // W += a E A^T                       A = E [M][Bt], B = X_upper [N][Bt] (contraction over batch)
};

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// One (possibly grouped) GEMM with fused prologue/epilogue.  Output is M x N,
// contraction K.  Group g offsets every pointer by g * <its group stride>.
// All strides are in elements.
struct GemmProblem {
  int kind;
  int M, N, K, groups;
  const void* a; long long lda, a_gs;
  const void* b; long long ldb, b_gs;
  void* out; long long ldo, o_gs;        // E (pred) / OUT (fwd) / X (infer) / W (weight)
  const void* aux; long long ldx, x_gs;  // X_lower (pred) / E (infer); unused otherwise
  void* out2; long long ld2, o2_gs;      // A_out (infer, save mode) or nullptr
  float scal;                            // gamma (infer) / alpha (weight)
  int act_b;                             // activation applied to the B operand in its loader
  int act_epi;                           // activation of the infer epilogue
  int vec_a, vec_b;                      // 1 if the operand allows 4-element vector loads
};

// A ragged batch of independent GEMMs of one layout launched as ONE kernel:
// workgroup w belongs to problem i when start[i] <= w < start[i+1].  All
// problems of a batch share the tile configuration and the layout (kinds
// PRED/FWD, INFER or WEIGHT), not their shapes.
constexpr int MAX_BATCH = 12;
struct GemmBatch {
  GemmProblem p[MAX_BATCH];
  int start[MAX_BATCH + 1];
  int count;
};

// Launches `count` problems (split into several launches if count > MAX_BATCH);
// `storage`/`operand` are DT_* codes, `tile` a tile id.
// `split` (1, 2 or 3) selects the error-compensated 16-bit prediction
// operands of the PF layout; other layouts ignore it.
hipError_t launch_gemm(const GemmProblem* probs, int count, int storage, int operand, int split, int tile,
                       hipStream_t s);

struct OuterProblem {
  int M, K, B, groups;
  void* w; long long w_gs;
  const void* e; long long e_gs;
  const void* x; long long x_gs;
  float alpha;
  int act;  // ACT_IDENTITY for a saved activation
};

hipError_t launch_outer(const OuterProblem& p, int storage, hipStream_t s);

// dst[i] = f(src[i]) for i < n (same storage type).
hipError_t launch_act(const void* src, void* dst, long long n, int act, int storage, hipStream_t s);

// Tile geometry per tile id (shared with the host heuristics).
struct TileShape { int bm, bn, bk, threads; };
TileShape tile_shape(int tile);

}  // namespace ipc
