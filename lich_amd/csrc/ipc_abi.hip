// ipc_abi.hip - the extern "C" boundary of libipc_hip.so (declared in include/ipc_hip.h).
//
// Every entry point validates its arguments on the host before any HIP call
// (so the error paths are testable without a GPU), converts them to
// GemmProblem / OuterProblem records and enqueues on the caller's stream.
// No entry point allocates device memory; only ipc_plan_check synchronises
// (it reads the whole-step kernels' timeout word).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <new>
#include <queue>
#include <string>
#include <vector>

#include "../../include/ipc_hip.h"
#include "ipc_launch.h"
#include "ipc_narrow.h"
#include "ipc_wide.h"

using namespace ipc;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() { return IPC_OK; }

const long long kMaxElems = (1LL << 31) - 1;  // per-matrix element count (32-bit tile indices)

int elem_size(int dt) { return dt == IPC_DT_F32 ? 4 : 2; }

int check_dtypes(int storage, int operand) {
  if (storage < IPC_DT_F32 || storage > IPC_DT_BF16)
    return fail(IPC_ERR_DTYPE, "unknown storage dtype %d", storage);
  if (operand < IPC_DT_F32 || operand > IPC_DT_BF16)
    return fail(IPC_ERR_DTYPE, "unknown operand dtype %d", operand);
  if (storage != IPC_DT_F32 && operand != storage)
    return fail(IPC_ERR_DTYPE, "16-bit storage (%d) requires operand dtype == storage (got %d)",
                storage, operand);
  return ok();
}

int check_act(int act) {
  if (act < IPC_ACT_IDENTITY || act > IPC_ACT_GELU)
    return fail(IPC_ERR_ACT, "unknown activation %d", act);
  return ok();
}

int check_dims(int M, int K, int B, int groups) {
  if (M < 1 || K < 1 || B < 1 || groups < 1)
    return fail(IPC_ERR_SHAPE, "dimensions must be >= 1 (M=%d K=%d B=%d groups=%d)", M, K, B, groups);
  if ((long long)M * K > kMaxElems || (long long)M * B > kMaxElems || (long long)K * B > kMaxElems)
    return fail(IPC_ERR_SHAPE, "matrix too large (M=%d K=%d B=%d)", M, K, B);
  return ok();
}

int check_ptr(const void* p, const char* name, int esize) {
  if (!p) return fail(IPC_ERR_NULL, "%s is NULL", name);
  if (reinterpret_cast<uintptr_t>(p) % esize)
    return fail(IPC_ERR_ALIGN, "%s is not aligned to its %d-byte element", name, esize);
  return ok();
}

int check_split(int split) {
  if (split < IPC_SPLIT_NONE || split > IPC_SPLIT_WX) return fail(IPC_ERR_CONFIG, "unknown split %d", split);
  return ok();
}

// Splitting only changes anything for fp32 data feeding 16-bit operands.
int effective_split(int storage, int operand, int split) {
  return (storage == IPC_DT_F32 && operand != IPC_DT_F32) ? split : IPC_SPLIT_NONE;
}

int check_tile(int tile) {
  if (tile < IPC_TILE_AUTO || tile >= IPC_TILE_COUNT)
    return fail(IPC_ERR_CONFIG, "unknown tile config %d", tile);
  return ok();
}

#define TRY(x)                  \
  do {                          \
    const int _rc = (x);        \
    if (_rc != IPC_OK) return _rc; \
  } while (0)

// 4-element vector loads need the contiguous length and the base aligned to 4 elements.
int vec_ok(const void* p, long long contiguous, int esize) {
  return (contiguous % 4 == 0) && (reinterpret_cast<uintptr_t>(p) % (4 * esize) == 0);
}

// Auto tile: the largest tile that still yields at least ~2 workgroups per CU
// (256 CUs), falling back to smaller tiles for the latency-bound shapes.
int pick_tile(long long M, long long N, long long groups) {
  const long long t128 = ((M + 127) / 128) * ((N + 127) / 128) * groups;
  const long long t64 = ((M + 63) / 64) * ((N + 63) / 64) * groups;
  if (t128 >= 512) return IPC_TILE_128x128;
  if (t64 >= 256) return IPC_TILE_64x64;
  if (M >= 64 && N >= 64 && t64 >= 64) return IPC_TILE_64x64;
  return IPC_TILE_32x32;
}

int launch_rc(hipError_t err, const char* what) {
  if (err != hipSuccess) return fail(IPC_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
  return ok();
}

GemmProblem make_pf(int kind, const void* xu, const void* w, const void* xl, void* out, int M, int K,
                    int B, int groups, int act, int esize) {
  GemmProblem p{};
  p.kind = kind;
  p.M = M; p.N = B; p.K = K; p.groups = groups;
  p.a = w; p.lda = K; p.a_gs = (long long)M * K;
  p.b = xu; p.ldb = B; p.b_gs = (long long)K * B;
  p.out = out; p.ldo = B; p.o_gs = (long long)M * B;
  p.aux = xl; p.ldx = B; p.x_gs = (long long)M * B;
  p.out2 = nullptr;
  p.act_b = act; p.act_epi = act;
  p.vec_a = vec_ok(w, K, esize);
  p.vec_b = vec_ok(xu, B, esize);
  return p;
}

GemmProblem make_inf(void* x, const void* e, const void* wl, const void* el, void* aout, int M, int K,
                     int B, int groups, float gamma, int act, int esize) {
  GemmProblem p{};
  p.kind = KIND_INFER;
  p.M = M; p.N = B; p.K = K; p.groups = groups;
  p.a = wl; p.lda = M; p.a_gs = (long long)K * M;
  p.b = el; p.ldb = B; p.b_gs = (long long)K * B;
  p.out = x; p.ldo = B; p.o_gs = (long long)M * B;
  p.aux = e; p.ldx = B; p.x_gs = (long long)M * B;
  p.out2 = aout; p.ld2 = B; p.o2_gs = (long long)M * B;
  p.scal = gamma;
  p.act_b = IPC_ACT_IDENTITY; p.act_epi = act;
  p.vec_a = vec_ok(wl, M, esize);
  p.vec_b = vec_ok(el, B, esize);
  return p;
}

GemmProblem make_wgt(void* w, const void* e, const void* xu, int M, int K, int B, int groups,
                     float alpha, int recompute, int act, int esize) {
  GemmProblem p{};
  p.kind = KIND_WEIGHT;
  p.M = M; p.N = K; p.K = B; p.groups = groups;
  p.a = e; p.lda = B; p.a_gs = (long long)M * B;
  p.b = xu; p.ldb = B; p.b_gs = (long long)K * B;
  p.out = w; p.ldo = K; p.o_gs = (long long)M * K;
  p.aux = nullptr;
  p.out2 = nullptr;
  p.scal = alpha;
  p.act_b = recompute ? act : IPC_ACT_IDENTITY; p.act_epi = act;
  p.vec_a = vec_ok(e, B, esize);
  p.vec_b = vec_ok(xu, B, esize);
  return p;
}

OuterProblem make_outer(void* w, const void* e, const void* xu, int M, int K, int B, int groups,
                        float alpha, int recompute, int act) {
  OuterProblem p{};
  p.M = M; p.K = K; p.B = B; p.groups = groups;
  p.w = w; p.w_gs = (long long)M * K;
  p.e = e; p.e_gs = (long long)M * B;
  p.x = xu; p.x_gs = (long long)K * B;
  p.alpha = alpha;
  p.act = recompute ? act : IPC_ACT_IDENTITY;
  return p;
}

constexpr int kOuterMaxB = 32;

bool al16(const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; }
bool al8(const void* q) { return q == nullptr || reinterpret_cast<uintptr_t>(q) % 8 == 0; }

// The LDS-DMA kernel serves 16-bit storage whose contraction is a multiple of
// WIDE_BK and whose operands stream in 16-byte chunks: aligned bases, row
// strides (in elements) that are multiples of 8.
bool dma_eligible(int storage, int contraction, std::initializer_list<const void*> operands,
                  std::initializer_list<long long> strides) {
  if (storage == IPC_DT_F32 || contraction % WIDE_BK != 0) return false;
  for (const void* q : operands)
    if (!al16(q)) return false;
  for (long long ld : strides)
    if (ld % 8 != 0) return false;
  return true;
}

// Tile selection of a standalone call: returns 1 + the LDS-DMA configuration
// (0: 256 x 128, 1: 128 x 256, 2: 128 x 128, 3: 256 x 256) if that kernel runs it, 0 for
// the generic kernel (tile resolved), or an error.
int select_tile(int& tile, bool eligible, long long M, long long N, long long groups) {
  const bool dma_tile = tile >= IPC_TILE_DMA_256x128;
  if (dma_tile && !eligible)
    return fail(IPC_ERR_CONFIG,
                "tile %d (LDS-DMA) needs 16-bit storage, a contraction that is a multiple of %d, 16-byte "
                "aligned tensors and row lengths that are multiples of 8", tile, WIDE_BK);
  if (eligible && tile == IPC_TILE_AUTO) {
    // 256 x 256 tiles (half the LDS reads per MFMA) once they fill every CU
    // (256) at least once, else 256 x 128: per-kernel sweep on MI355X, e.g.
    // M = K = 8192: prediction 0.26 -> 0.34, inference 0.31 -> 0.37, weight
    // update 0.40 -> 0.43 of the bf16 peak; at 128 tiles of 256 x 256 half the
    // CUs idle and the smaller tile wins
    const long long t256 = ((M + 255) / 256) * ((N + 255) / 256) * groups;
    return t256 >= 256 ? 1 + IPC_TILE_DMA_256x256 - IPC_TILE_DMA_256x128 : 1;
  }
  if (dma_tile) return 1 + tile - IPC_TILE_DMA_256x128;
  if (tile == IPC_TILE_AUTO) tile = pick_tile(M, N, groups);
  return 0;
}

// One WideProblem per group of a standalone 16-bit call.
std::vector<WideProblem> s16_groups(const WideProblem& q, int groups, long long a_gs, long long b_gs,
                                    long long o_gs, long long x_gs, long long o2_gs) {
  std::vector<WideProblem> v((size_t)groups, q);
  for (int g = 0; g < groups; ++g) {
    WideProblem& r = v[(size_t)g];
    r.a = static_cast<const char*>(q.a) + 2 * g * a_gs;
    r.b = static_cast<const char*>(q.b) + 2 * g * b_gs;
    r.out = static_cast<char*>(q.out) + 2 * g * o_gs;
    if (q.aux) r.aux = static_cast<const char*>(q.aux) + 2 * g * x_gs;
    if (q.out2) r.out2 = static_cast<char*>(q.out2) + 2 * g * o2_gs;
  }
  return v;
}

// Pre-activation of a standalone call's B operand (ipc_set_s16_preactivate):
// -1 automatic, 0 never, 1 always.
int g_s16_preact = -1;

// Whether a call evaluates its B operand f(X_upper) once instead of in the
// loader of every row tile (the same bits: f of the stored value, one
// rounding; then the GEMM reads the result through LDS DMA like every other
// operand).  The automatic rule, from the per-kernel sweep on MI355X: the
// exponential activations pay for the extra pass from 4 row tiles of 256
// (M >= 1024) and a 2^20-element operand; relu, cheap in the loader, from 16
// row tiles and 2^22 elements.  The inference update has no activated
// operand; given a workspace it stores W_lower and E_lower transposed
// instead, which pays only for the largest calls (W and E_lower of at least
// 2^26 elements each): at 8192^3 3-8 % faster, at 8192 x 8192 x 2048 and
// 4096^2 x 8192 3-9 % slower, the two copying passes outweighing the GEMM's
// gain.
bool s16_preact_rule(int mode, int act, int M, int K, long long kb) {
  if (g_s16_preact == 0) return false;
  if (mode == S16_INFER) return g_s16_preact > 0 || ((long long)M * K >= (1LL << 26) && kb >= (1LL << 26));
  if (act == IPC_ACT_IDENTITY) return false;
  if (g_s16_preact > 0) return true;
  if (act == IPC_ACT_RELU) return M >= 4096 && kb >= (1LL << 22);
  return M >= 1024 && kb >= (1LL << 20);
}

// Bytes of caller workspace a call uses (0 when the rule says it does not
// use one): the groups' activated B operands, 16-bit, contiguous; for the
// inference update the groups' W_lower^T blocks [M][K], then their
// E_lower^T blocks [B][K].
long long s16_workspace_need(int mode, int act, int M, int K, long long kb, int groups) {
  if (!s16_preact_rule(mode, act, M, K, kb)) return 0;
  return mode == S16_INFER ? (long long)groups * ((long long)M * K + kb) * 2 : (long long)groups * kb * 2;
}

// A standalone call on the LDS-DMA kernel.  With a caller workspace of at
// least s16_workspace_need bytes the B operand is activated once into it
// (an elementwise launch) and the GEMM reads it like the other operands, or,
// for the inference update, both operands are copied transposed into it;
// otherwise every row tile activates its B block in its loader and the
// inference update reads its operands transposed from LDS.  The library
// allocates nothing either way.
int run_s16(int mode, const WideProblem& q, int groups, long long a_gs, long long b_gs, long long o_gs,
            long long x_gs, long long o2_gs, int operand, int act, int cfg, void* workspace, long long ws_bytes,
            void* stream, const char* what) {
  hipStream_t s = (hipStream_t)stream;
  const long long need = s16_workspace_need(mode, act, q.M, q.K, b_gs, groups);
  if (need > 0 && workspace && ws_bytes >= need) {
    WideProblem qa = q;
    if (mode == S16_INFER) {
      // W_lower [K][M] -> [M][K] and E_lower [K][B] -> [B][K] (identity
      // "activation"): both GEMM operands k-contiguous, the same values in
      // the same k order
      char* wt = static_cast<char*>(workspace);
      char* et = wt + (long long)groups * a_gs * 2;
      qa.a = wt; qa.lda = q.K; qa.a_lim = q.M;
      qa.b = et; qa.ldb = q.K; qa.b_lim = q.N;
      const std::vector<WideProblem> v = s16_groups(qa, groups, a_gs, b_gs, o_gs, x_gs, o2_gs);
      TRY(launch_rc(launch_s16_activate_t(q.a, wt, q.K, q.M, groups, a_gs, operand, IPC_ACT_IDENTITY, s), what));
      TRY(launch_rc(launch_s16_activate_t(q.b, et, q.K, q.N, groups, b_gs, operand, IPC_ACT_IDENTITY, s), what));
      return launch_rc(launch_s16(S16_INFERT, v.data(), groups, operand, act, cfg, s), what);
    }
    qa.b = workspace;
    if (mode == S16_PRED || mode == S16_FWD) {
      // f(X_upper [K][B])^T into the workspace: the GEMM then reads both
      // operands k-contiguous (plain 16-byte fragment reads instead of the
      // transposing ones), with the same values in the same k order
      qa.ldb = q.K;
      qa.b_lim = q.N;
      const std::vector<WideProblem> v = s16_groups(qa, groups, a_gs, b_gs, o_gs, x_gs, o2_gs);
      TRY(launch_rc(launch_s16_activate_t(q.b, workspace, q.K, q.N, groups, b_gs, operand, act, s), what));
      return launch_rc(launch_s16(mode == S16_PRED ? S16_PREDT : S16_FWDT, v.data(), groups, operand,
                                  IPC_ACT_IDENTITY, cfg, s), what);
    }
    const long long n = (long long)groups * b_gs;  // the groups' B operands are contiguous, b_gs apart
    const std::vector<WideProblem> v = s16_groups(qa, groups, a_gs, b_gs, o_gs, x_gs, o2_gs);
    TRY(launch_rc(launch_s16_activate(q.b, workspace, n, operand, act, s), what));
    return launch_rc(launch_s16(mode, v.data(), groups, operand, IPC_ACT_IDENTITY, cfg, s), what);
  }
  const std::vector<WideProblem> v = s16_groups(q, groups, a_gs, b_gs, o_gs, x_gs, o2_gs);
  return launch_rc(launch_s16(mode, v.data(), groups, operand, act, cfg, s), what);
}

int check_workspace(const void* workspace, long long ws_bytes) {
  if (ws_bytes < 0) return fail(IPC_ERR_SHAPE, "workspace_bytes must be >= 0");
  if (workspace && reinterpret_cast<uintptr_t>(workspace) % 16)
    return fail(IPC_ERR_ALIGN, "workspace must be 16-byte aligned");
  return ok();
}

}  // namespace

// =========================================================================== C ABI
extern "C" {

int ipc_abi_version(void) { return IPC_ABI_VERSION; }

const char* ipc_last_error(void) { return g_last_error.c_str(); }

int ipc_device_check(int device, char* buf, int buflen) {
  hipDeviceProp_t prop;
  const hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return fail(IPC_ERR_DEVICE, "no HIP device %d: %s", device, hipGetErrorString(err));
  if (buf && buflen > 0) {
    std::strncpy(buf, prop.gcnArchName, (size_t)buflen - 1);
    buf[buflen - 1] = '\0';
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(IPC_ERR_DEVICE, "device %d is %s; this library is built for gfx950 (MI355X) only",
                device, prop.gcnArchName);
  return ok();
}

int ipc_pred_err(const void* x_upper, const void* w, const void* x_lower, void* e, int M, int K, int B,
                 int groups, int storage, int operand, int split, int act, int tile, void* stream) {
  return ipc_pred_err_ws(x_upper, w, x_lower, e, M, K, B, groups, storage, operand, split, act, tile, nullptr, 0,
                         stream);
}

int ipc_pred_err_ws(const void* x_upper, const void* w, const void* x_lower, void* e, int M, int K, int B,
                    int groups, int storage, int operand, int split, int act, int tile, void* workspace,
                    long long workspace_bytes, void* stream) {
  TRY(check_workspace(workspace, workspace_bytes));
  TRY(check_dtypes(storage, operand));
  TRY(check_split(split));
  TRY(check_act(act));
  TRY(check_dims(M, K, B, groups));
  TRY(check_tile(tile));
  const int es = elem_size(storage);
  TRY(check_ptr(x_upper, "x_upper", es));
  TRY(check_ptr(w, "w", es));
  TRY(check_ptr(x_lower, "x_lower", es));
  TRY(check_ptr(e, "e", es));
  const int use_dma = select_tile(tile, dma_eligible(storage, K, {x_upper, w}, {K, B}), M, B, groups);
  if (use_dma < 0) return use_dma;
  if (use_dma) {
    WideProblem q{};
    q.M = M; q.N = B; q.K = K;
    q.a = w; q.lda = K; q.a_lim = M;
    q.b = x_upper; q.ldb = B; q.b_lim = B;
    q.out = e; q.ldo = B; q.aux = x_lower; q.ldx = B;
    q.vec = B % 4 == 0 && al8(e) && al8(x_lower);
    return run_s16(S16_PRED, q, groups, (long long)M * K, (long long)K * B, (long long)M * B, (long long)M * B, 0,
                   operand, act, use_dma - 1, workspace, workspace_bytes, stream, "ipc_pred_err");
  }
  GemmProblem p = make_pf(KIND_PRED, x_upper, w, x_lower, e, M, K, B, groups, act, es);
  return launch_rc(launch_gemm(&p, 1, storage, operand, effective_split(storage, operand, split), tile,
                               (hipStream_t)stream), "ipc_pred_err");
}

int ipc_forward(const void* x_upper, const void* w, void* out, int M, int K, int B, int groups, int storage,
                int operand, int split, int act, int tile, void* stream) {
  return ipc_forward_ws(x_upper, w, out, M, K, B, groups, storage, operand, split, act, tile, nullptr, 0, stream);
}

int ipc_forward_ws(const void* x_upper, const void* w, void* out, int M, int K, int B, int groups, int storage,
                   int operand, int split, int act, int tile, void* workspace, long long workspace_bytes,
                   void* stream) {
  TRY(check_workspace(workspace, workspace_bytes));
  TRY(check_dtypes(storage, operand));
  TRY(check_split(split));
  TRY(check_act(act));
  TRY(check_dims(M, K, B, groups));
  TRY(check_tile(tile));
  const int es = elem_size(storage);
  TRY(check_ptr(x_upper, "x_upper", es));
  TRY(check_ptr(w, "w", es));
  TRY(check_ptr(out, "out", es));
  const int use_dma = select_tile(tile, dma_eligible(storage, K, {x_upper, w}, {K, B}), M, B, groups);
  if (use_dma < 0) return use_dma;
  if (use_dma) {
    WideProblem q{};
    q.M = M; q.N = B; q.K = K;
    q.a = w; q.lda = K; q.a_lim = M;
    q.b = x_upper; q.ldb = B; q.b_lim = B;
    q.out = out; q.ldo = B;
    q.vec = B % 4 == 0 && al8(out);
    return run_s16(S16_FWD, q, groups, (long long)M * K, (long long)K * B, (long long)M * B, 0, 0, operand, act,
                   use_dma - 1, workspace, workspace_bytes, stream, "ipc_forward");
  }
  GemmProblem p = make_pf(KIND_FWD, x_upper, w, nullptr, out, M, K, B, groups, act, es);
  return launch_rc(launch_gemm(&p, 1, storage, operand, effective_split(storage, operand, split), tile,
                               (hipStream_t)stream), "ipc_forward");
}

int ipc_infer_update(void* x, const void* e, const void* w_lower, const void* e_lower, void* a_out, int M,
                     int K, int B, int groups, float gamma, int storage, int operand, int act, int tile,
                     void* stream) {
  return ipc_infer_update_ws(x, e, w_lower, e_lower, a_out, M, K, B, groups, gamma, storage, operand, act, tile,
                             nullptr, 0, stream);
}

int ipc_infer_update_ws(void* x, const void* e, const void* w_lower, const void* e_lower, void* a_out, int M,
                        int K, int B, int groups, float gamma, int storage, int operand, int act, int tile,
                        void* workspace, long long workspace_bytes, void* stream) {
  TRY(check_workspace(workspace, workspace_bytes));
  TRY(check_dtypes(storage, operand));
  TRY(check_act(act));
  TRY(check_dims(M, K, B, groups));
  TRY(check_tile(tile));
  const int es = elem_size(storage);
  TRY(check_ptr(x, "x", es));
  TRY(check_ptr(e, "e", es));
  TRY(check_ptr(w_lower, "w_lower", es));
  TRY(check_ptr(e_lower, "e_lower", es));
  if (a_out) TRY(check_ptr(a_out, "a_out", es));
  const int use_dma = select_tile(tile, dma_eligible(storage, K, {w_lower, e_lower}, {M, B}), M, B, groups);
  if (use_dma < 0) return use_dma;
  if (use_dma) {
    WideProblem q{};
    q.M = M; q.N = B; q.K = K;
    q.a = w_lower; q.lda = M; q.a_lim = M;
    q.b = e_lower; q.ldb = B; q.b_lim = B;
    q.out = x; q.ldo = B; q.aux = e; q.ldx = B;
    q.out2 = a_out; q.ld2 = B;
    q.scal = gamma;
    q.vec = B % 4 == 0 && al8(x) && al8(e) && al8(a_out);
    return run_s16(S16_INFER, q, groups, (long long)K * M, (long long)K * B, (long long)M * B, (long long)M * B,
                   (long long)M * B, operand, act, use_dma - 1, workspace, workspace_bytes, stream,
                   "ipc_infer_update");
  }
  GemmProblem p = make_inf(x, e, w_lower, e_lower, a_out, M, K, B, groups, gamma, act, es);
  return launch_rc(launch_gemm(&p, 1, storage, operand, IPC_SPLIT_NONE, tile, (hipStream_t)stream),
                   "ipc_infer_update");
}

int ipc_weight_update(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                      float alpha, int recompute, int storage, int operand, int act, int tile, void* stream) {
  return ipc_weight_update_ws(w, e, x_upper, M, K, B, groups, alpha, recompute, storage, operand, act, tile, nullptr,
                              0, stream);
}

int ipc_weight_update_ws(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                         float alpha, int recompute, int storage, int operand, int act, int tile, void* workspace,
                         long long workspace_bytes, void* stream) {
  TRY(check_workspace(workspace, workspace_bytes));
  TRY(check_dtypes(storage, operand));
  TRY(check_act(act));
  TRY(check_dims(M, K, B, groups));
  TRY(check_tile(tile));
  const int es = elem_size(storage);
  TRY(check_ptr(w, "w", es));
  TRY(check_ptr(e, "e", es));
  TRY(check_ptr(x_upper, "x_upper", es));
  const int use_dma = select_tile(tile, dma_eligible(storage, B, {e, x_upper}, {B}), M, K, groups);
  if (use_dma < 0) return use_dma;
  if (use_dma) {
    WideProblem q{};
    q.M = M; q.N = K; q.K = B;
    q.a = e; q.lda = B; q.a_lim = M;
    q.b = x_upper; q.ldb = B; q.b_lim = K;
    q.out = w; q.ldo = K;
    q.scal = alpha;
    q.vec = K % 4 == 0 && al8(w);
    return run_s16(S16_WEIGHT, q, groups, (long long)M * B, (long long)K * B, (long long)M * K, 0, 0, operand,
                   recompute ? act : IPC_ACT_IDENTITY, use_dma - 1, workspace, workspace_bytes, stream,
                   "ipc_weight_update");
  }
  GemmProblem p = make_wgt(w, e, x_upper, M, K, B, groups, alpha, recompute, act, es);
  return launch_rc(launch_gemm(&p, 1, storage, operand, IPC_SPLIT_NONE, tile, (hipStream_t)stream),
                   "ipc_weight_update");
}

int ipc_weight_update_outer(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                            float alpha, int recompute, int storage, int act, void* stream) {
  TRY(check_dtypes(storage, storage));
  TRY(check_act(act));
  TRY(check_dims(M, K, B, groups));
  if (B > kOuterMaxB) return fail(IPC_ERR_SHAPE, "outer-product update supports B <= %d (got %d)", kOuterMaxB, B);
  const int es = elem_size(storage);
  TRY(check_ptr(w, "w", es));
  TRY(check_ptr(e, "e", es));
  TRY(check_ptr(x_upper, "x_upper", es));
  OuterProblem p = make_outer(w, e, x_upper, M, K, B, groups, alpha, recompute, act);
  return launch_rc(launch_outer(p, storage, (hipStream_t)stream), "ipc_weight_update_outer");
}

}  // extern "C"

// =========================================================================== plan
struct ipc_plan {
  int L = 0, B = 0, storage = 0, operand = 0, split = 1, act = 0, recompute = 1, wmode = 0;
  float alpha = 0.f, gamma = 0.f;
  std::vector<int> dims;
  bool bound = false;
  // prepared launches of one step
  std::vector<GemmProblem> pred, infer, weight;
  std::vector<OuterProblem> outer;
  int tile_pred = 0, tile_infer = 0, tile_weight = 0;
  int tile_override[3] = {IPC_TILE_AUTO, IPC_TILE_AUTO, IPC_TILE_AUTO};  // ipc_plan_set_tiles
  // forward initialisation launches (l = L-1 .. 1, sequential)
  std::vector<GemmProblem> fwd;
  const void* act_src = nullptr;  // x[L]
  void* act_dst = nullptr;        // a[L] in save mode
  int launches = 0;
  // whole-step kernels for narrow nets (column-block; layer-resident for multi-step launches)
  bool narrow = false;
  NarrowArgs nargs{};
  bool resident = false;
  bool res_stale = false;  // bound since the last layer-resident launch: invalidate its caches first
  ResidentArgs rargs{};
  long long res_ws_off = 0;
  // wide GEMM path
  bool wide = false;
  bool wdirect = false;  // wide, split 2: the prediction reads W itself (no Wh / Wl copies)
  std::vector<WideProblem> wpred, winfer, wweight, wfwd;  // wfwd: l = L-1 .. 1
  int pred_ksplit = 1;                                    // > 1: layer 0's prediction is k-split (last in wpred)
  int wcfg[3] = {0, 0, 0};                                // tile configuration of the pred / infer / weight launches
  int ksplit_request = 0;                                 // > 0: layer 0's k-split as set by the caller (1 = none)
  WideReduce wreduce{};                                   // its epilogue
  std::vector<WideCopy> wsync, wsync_init;               // wsync_init: W and x[L] only
  long long ws_bytes = 0;
  void* workspace = nullptr;
  // whole-step kernels: polls before a wait gives up (and raises the timeout
  // word), and the most workgroups of the column kernel that can run at once
  int spin_limit = 0;
  int narrow_cap = 256;
  // captured steps (ipc_plan_graph_capture): the graph, its executable and
  // the private stream it was captured on
  hipStream_t cap_stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  int graph_steps = 0;
  bool graph_direct = false;  // the captured steps are one whole-step launch, replayed as such

  void release_graph() {
    if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
    if (graph) (void)hipGraphDestroy(graph);
    graph_exec = nullptr;
    graph = nullptr;
    graph_steps = 0;
    graph_direct = false;
  }
  ~ipc_plan() {
    release_graph();
    if (cap_stream) (void)hipStreamDestroy(cap_stream);
  }
};

namespace {

constexpr int kNarrowSpinLimit = 1 << 22;

// > 0: the co-resident workgroup capacity used instead of the device's
// (ipc_set_coresident_limit, a test hook).
int g_coresident_limit = 0;

// >= 0: the spin limit of ipc_steps_noalloc's waits instead of the default
// (ipc_noalloc_set_spin_limit, a test hook).
int g_noalloc_spin_limit = -1;

// Static device scratch of the no-allocation entry point (ipc_steps_noalloc):
// every GPU the library runs on holds its own copy for the life of the
// process.  Host code never uses the array's name as an address (on the host
// it is a stand-in symbol): scratch_address looks up the device copy with
// hipGetSymbolAddress once per device and keeps it.
constexpr long long kScratchBytes = 8LL << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};

// Address of the current device's copy of `scratch`.
int scratch_address(char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(IPC_ERR_DEVICE, "no current device");
  if (dev < 0 || dev >= kMaxDevices) return fail(IPC_ERR_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(IPC_ERR_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

// Zeroes the column kernel's barrier words and, when given, the resident
// kernel's flag words (64 words each) before a launch on the scratch.
// Word 2 (the timeout word) is left alone: it stays set until
// ipc_noalloc_check reads and clears it, so a call whose waits gave up is
// reported even after later calls.
__global__ void scratch_clear_kernel(unsigned* bar, unsigned* flags) {
  if (threadIdx.x < 64 && threadIdx.x != 2) bar[threadIdx.x] = 0u;
  if (flags) flags[threadIdx.x] = 0u;  // the layer-resident flag area, RES_FLAG_BYTES / 4 words
}

// Workgroups of a whole-step kernel instantiation that the current device
// can run at once (workgroups per CU x CUs), or -1 when it cannot be
// determined (no device).  `occupancy` reports the workgroups per CU after
// the instantiation's LDS limit has been raised by `prepare`.
template <typename Prepare, typename Occupancy>
int coresident_capacity(const Prepare& prepare, const Occupancy& occupancy) {
  if (g_coresident_limit > 0) return g_coresident_limit;
  int dev = 0, ncu = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0) return -1;
  if (prepare() != hipSuccess || occupancy(&per_cu) != hipSuccess) return -1;
  return per_cu * ncu;
}

bool narrow_eligible(int L, const int* dims, int storage, int operand, int split) {
  if (storage != IPC_DT_F32 || L > NARROW_MAX_L) return false;
  if (split == IPC_SPLIT_W) return false;  // the whole-step kernel carries split 1 or 3
  for (int l = 0; l < L; ++l)
    if (dims[l] > NARROW_MAX_WIDTH) return false;
  // one column block's states, errors and staged activations must fit in LDS
  return narrow_lds_bytes(dims, L, operand, split) <= NARROW_LDS_LIMIT - 1024;
}

bool wide_eligible(int storage, int operand, int split, int wmode, int B) {
  if (storage != IPC_DT_F32 || operand == IPC_DT_F32) return false;
  if (split != IPC_SPLIT_NONE && split != IPC_SPLIT_W) return false;
  return wmode == IPC_WMODE_GEMM || (wmode == IPC_WMODE_AUTO && B > 16);
}

// Workspace layout of the wide path: after the 256 bytes every plan reserves,
// one 256-byte aligned buffer per 16-bit operand copy, rows and columns
// padded to WIDE_PAD with zeros; every operand has a k-contiguous copy for
// each GEMM that reads it.
struct WideLayout {
  struct Buf { long long off = -1, ld = 0, rows = 0; };
  std::vector<Buf> wh, wl, wt, f, ft, e, et;
  long long total = 256;
  // fp32 partial products of a k-split layer-0 prediction: up to part_smax
  // slices of [d_0][B], part_stride floats apart
  int part_smax = 1;
  long long part_off = -1, part_stride = 0;

  Buf add(long long rows, long long cols) {
    Buf b;
    b.ld = wide_pad(cols, WIDE_PAD);
    b.rows = wide_pad(rows, WIDE_PAD);
    b.off = total;
    total += wide_pad(b.rows * b.ld * 2, 256);
    return b;
  }
  // direct: the split-2 prediction reads the fp32 W (ld = d_{l+1}, a multiple
  // of WIDE_BK) in place of Wh / Wl, which then get no storage (their ld and
  // rows still give the contraction lengths and row counts)
  WideLayout(const std::vector<int>& d, int L, int B, bool split2, int pred_cfg, bool direct = false) {
    wh.resize(L); wl.resize(L); wt.resize(L); f.resize(L + 1); ft.resize(L + 1); e.resize(L); et.resize(L);
    for (int l = 0; l < L; ++l) {
      if (direct) {
        wh[l].ld = d[l + 1];
        wh[l].rows = d[l];
      } else {
        wh[l] = add(d[l], d[l + 1]);                // [d_l][d_{l+1}]  pred A
        if (split2) wl[l] = add(d[l], d[l + 1]);    //                 pred A_lo
      }
      if (l <= L - 2) wt[l] = add(d[l + 1], d[l]);  // [d_{l+1}][d_l]  infer A (layer l+1)
    }
    for (int l = 1; l <= L; ++l) {
      f[l] = add(d[l], B);                      // [d_l][B]        weight B (layer l-1)
      ft[l] = add(B, d[l]);                     // [B][d_l]        pred B (layer l-1)
    }
    for (int l = 0; l < L; ++l) {
      e[l] = add(d[l], B);                      // [d_l][B]        weight A
      if (l <= L - 2) et[l] = add(B, d[l]);     // [B][d_l]        infer B (layer l+1)
    }
    // the k-split prediction cuts layer 0's tiles into at most 512 slices in all
    int bm = 0, bn = 0;
    wide_pred_tile(split2 ? 2 : 1, pred_cfg, &bm, &bn);
    const long long t0 = ((d[0] + bm - 1) / bm) * (long long)((B + bn - 1) / bn);
    for (int sl = 16; sl >= 2; sl /= 2)
      if (sl * t0 <= 512 && wh[0].ld % (sl * WIDE_BK) == 0) { part_smax = sl; break; }
    if (part_smax > 1) {
      part_stride = (long long)d[0] * B;
      part_off = total;
      total += wide_pad(part_smax * part_stride * 4, 256);
    }
  }
};

// Slices of layer 0's prediction (1 = not split): the count, up to
// part_smax, with the shortest estimated launch when the tiles are handed to
// `ncu` CUs in dispatch order (every whole tile of layers 1..L-1, then the
// slices), one workgroup per CU, each tile costing its k-steps and each slice
// two more (prologue and partial-product store); a split pays four k-steps
// for the reduce launch.
int wide_pred_ksplit(const std::vector<int>& d, int L, int B, bool split2, int pred_cfg, const WideLayout& lay,
                     int ncu) {
  int bm = 0, bn = 0;
  wide_pred_tile(split2 ? 2 : 1, pred_cfg, &bm, &bn);
  auto tiles = [&](int l) { return ((d[l] + bm - 1) / bm) * (long long)((B + bn - 1) / bn); };
  auto makespan = [&](int sl) {
    std::priority_queue<double, std::vector<double>, std::greater<double>> cu;
    for (int i = 0; i < ncu; ++i) cu.push(0.0);
    auto run = [&](double cost) { const double t = cu.top() + cost; cu.pop(); cu.push(t); };
    for (int l = 1; l < L; ++l)
      for (long long t = 0; t < tiles(l); ++t) run((double)(lay.wh[l].ld / WIDE_BK));
    const double c0 = (double)(lay.wh[0].ld / WIDE_BK) / sl + (sl > 1 ? 2.0 : 0.0);
    for (long long t = 0; t < tiles(0) * sl; ++t) run(c0);
    double end = 0.0;
    while (!cu.empty()) { end = cu.top(); cu.pop(); }
    return end + (sl > 1 ? 4.0 : 0.0);
  };
  int best = 1;
  double best_t = makespan(1);
  for (int sl = 2; sl <= lay.part_smax; sl *= 2) {
    if (lay.wh[0].ld % (sl * WIDE_BK) != 0) continue;
    const double t = makespan(sl);
    if (t < best_t) { best = sl; best_t = t; }
  }
  return best;
}

bool narrow_outer(int B, int wmode) {
  return B <= NARROW_OUTER_MAX_B && (wmode == IPC_WMODE_OUTER || (wmode == IPC_WMODE_AUTO && B <= 16));
}

// Layer-resident kernel eligibility; fills `ra` and returns its workspace bytes, or -1.
// fp32 operands run it with either weight update (the rank-B one as the column
// kernel computes it); 16-bit operands with the GEMM update only.
long long resident_eligible(int L, const int* dims, int B, int operand, int split, int wmode, bool narrow,
                            ResidentArgs& ra, int top_rows = RES_TOP_ROWS) {
  if (!narrow) return -1;
  const bool outer = narrow_outer(B, wmode);
  if (operand == IPC_DT_F32)
    return split == IPC_SPLIT_NONE ? resident_plan(dims, L, B, 1, 4, outer, top_rows, ra) : -1;
  if (outer || (split != IPC_SPLIT_NONE && split != IPC_SPLIT_WX)) return -1;
  return resident_plan(dims, L, B, split == IPC_SPLIT_WX ? 3 : 1, 2, false, top_rows, ra);
}

int launch_narrow_mode(ipc_plan* plan, int mode, int steps, hipStream_t s) {
  if (mode == NMODE_STEPS && plan->resident) {
    // The caches a resident launch keeps in the workspace (f(x[L]) images,
    // hidden f(x), the next launch's first-step partials) belong to the
    // buffers bound when they were written: after a (re)bind, start cold.
    if (plan->res_stale) {
      TRY(launch_rc(resident_invalidate(plan->rargs, s), "layer-resident cache invalidation"));
      plan->res_stale = false;
    }
    ResidentArgs a = plan->rargs;
    a.steps = steps;
    return launch_rc(launch_resident(a, plan->operand, plan->split, plan->act, s), "layer-resident whole-step kernel");
  }
  NarrowArgs a = plan->nargs;
  a.mode = mode;
  a.steps = steps;
  if (mode == NMODE_PHASE_A || mode == NMODE_FORWARD) a.nblocks = (plan->B + NARROW_NC - 1) / NARROW_NC;
  if (mode == NMODE_PHASE_B) a.nblocks = a.wtile_start[plan->L];
  // the grid barriers of a multi-step launch need every workgroup running at
  // once; the phases' loops stride by the grid, so fewer workgroups only serialise
  if (a.nblocks > plan->narrow_cap) a.nblocks = plan->narrow_cap;
  return launch_rc(launch_narrow(a, plan->operand, plan->split, s), "whole-step kernel");
}

// Arguments of the whole-step kernels for bound buffers: the column kernel's
// `na` and, when `ra` is given (already laid out by resident_plan), the
// layer-resident kernel's.  `a` is NULL in recompute mode; `ws` is the
// workspace (barrier words, then the f(x) buffers of recompute mode, the
// resident exchange at `res_ws_off`).  Builds everything in place without
// heap allocation, so the no-allocation entry point shares it.
int bind_whole_step(NarrowArgs& na, ResidentArgs* ra, int L, const int* d, int B, void* const* x, void* const* e,
                    void* const* w, void* const* a, int act, int operand, int split, float alpha, float gamma,
                    bool outer, int spin_limit, int cap, char* ws, long long res_ws_off) {
  na = NarrowArgs{};
  na.L = L; na.B = B; na.act = act;
  na.alpha = alpha; na.gamma = gamma;
  na.spin_limit = spin_limit;
  na.outer = outer;
  int tiles = 0;
  for (int l = 0; l <= L; ++l) {
    na.dims[l] = d[l];
    na.x[l] = static_cast<float*>(x[l]);
    na.e[l] = l < L ? static_cast<float*>(e[l]) : nullptr;
    na.a[l] = (a && l >= 1) ? static_cast<float*>(a[l]) : nullptr;
    na.fx[l] = na.a[l];
    if (l < L) na.w[l] = static_cast<float*>(w[l]);
    na.wtile_start[l] = tiles;
    if (l < L) tiles += narrow_tiles(&d[l], 1);
  }
  // prediction/inference units (layer, 16-row tile), the longest contraction
  // first; insertion keeps units of equal contraction in (layer, tile) order
  int n = 0;
  for (int l = 0; l < L; ++l)
    for (int rt = 0; rt * 16 < d[l]; ++rt) {
      if (n >= NARROW_MAX_UNITS) return fail(IPC_ERR_SHAPE, "too many prediction units for the whole-step kernel");
      int i = n++;
      while (i > 0 && d[na.unit_l[i - 1] + 1] < d[l + 1]) {
        na.unit_l[i] = na.unit_l[i - 1];
        na.unit_rt[i] = na.unit_rt[i - 1];
        --i;
      }
      na.unit_l[i] = (unsigned char)l;
      na.unit_rt[i] = (unsigned char)rt;
    }
  na.n_units = n;
  na.lds_bytes = narrow_lds_bytes(d, L, operand, split);
  const int ncb = (B + NARROW_NC - 1) / NARROW_NC;
  na.nblocks = std::min(cap, std::max(ncb, tiles));
  na.bar = reinterpret_cast<unsigned*>(ws);
  if (!a) {
    // pre-evaluated f(x[l]) buffers follow the barrier counters in the workspace
    char* at = ws + 256;
    for (int l = 1; l <= L; ++l) {
      na.fx[l] = reinterpret_cast<float*>(at);
      at += ((long long)d[l] * B * 4 + 255) / 256 * 256;
    }
  }
  TRY(launch_rc(narrow_prepare(operand, split, act, na.lds_bytes), "whole-step kernel LDS limit"));
  if (ra) {
    ra->alpha = alpha; ra->gamma = gamma;
    ra->spin_limit = spin_limit;
    for (int l = 0; l <= L; ++l) {
      ra->x[l] = na.x[l];
      ra->e[l] = na.e[l];
      ra->fx[l] = na.fx[l];
      if (l < L) ra->w[l] = na.w[l];
    }
    ra->bar = na.bar;
    resident_bind(*ra, ws + res_ws_off);
    na.res_image_flag = ra->flags + RES_MAX_WG;
    TRY(launch_rc(resident_prepare(operand, split, act, ra->lds_bytes), "layer-resident kernel LDS limit"));
  }
  return ok();
}

}  // namespace

extern "C" {

int ipc_plan_create(ipc_plan** out, int L, const int* dims, int B, int storage, int operand, int split, int act,
                    float alpha, float gamma, int recompute, int weight_mode, int path) {
  if (!out) return fail(IPC_ERR_NULL, "out is NULL");
  *out = nullptr;
  if (!dims) return fail(IPC_ERR_NULL, "dims is NULL");
  if (L < 1 || L > 4096) return fail(IPC_ERR_SHAPE, "L must be in [1, 4096] (got %d)", L);
  TRY(check_dtypes(storage, operand));
  TRY(check_split(split));
  TRY(check_act(act));
  if (weight_mode < IPC_WMODE_GEMM || weight_mode > IPC_WMODE_AUTO)
    return fail(IPC_ERR_CONFIG, "unknown weight mode %d", weight_mode);
  for (int l = 0; l < L; ++l) TRY(check_dims(dims[l], dims[l + 1], B, 1));
  if (weight_mode == IPC_WMODE_OUTER && B > kOuterMaxB)
    return fail(IPC_ERR_SHAPE, "outer weight mode supports B <= %d (got %d)", kOuterMaxB, B);
  if (path < IPC_PATH_AUTO || path > IPC_PATH_RESIDENT) return fail(IPC_ERR_CONFIG, "unknown path %d", path);
  const int esplit = effective_split(storage, operand, split);
  const bool eligible = narrow_eligible(L, dims, storage, operand, esplit);
  ResidentArgs ra{};
  long long res_bytes = resident_eligible(L, dims, B, operand, esplit, weight_mode, eligible, ra);
  if (path == IPC_PATH_RESIDENT && res_bytes < 0)
    return fail(IPC_ERR_CONFIG,
                "the layer-resident kernel needs a narrow net with L >= 2, widths d_0..d_{L-1} <= %d, B <= %d, "
                "operand blocks that fit the LDS, and fp16/bf16 operands with split 1 or 3 and the GEMM weight "
                "update, or fp32 operands", RES_MAX_WIDTH, RES_MAX_B);
  // Every workgroup of a layer-resident launch waits for others, so all of
  // them must be able to run at once on this device (a compute-partitioned
  // device, or a smaller part, may hold fewer); otherwise an AUTO plan takes
  // the column kernel, whose grid is capped at the capacity below.
  if (res_bytes >= 0 && (path == IPC_PATH_RESIDENT || path == IPC_PATH_AUTO)) {
    const int cap = coresident_capacity(
        [&] { return resident_prepare(operand, esplit, act, ra.lds_bytes); },
        [&](int* n) { return resident_occupancy(operand, esplit, act, ra.lds_bytes, n); });
    const int need = resident_launch_blocks(ra);
    if (cap >= 0 && need > cap) {
      if (path == IPC_PATH_RESIDENT)
        return fail(IPC_ERR_CONFIG,
                    "the layer-resident kernel needs %d co-resident workgroups; this device holds %d of them",
                    need, cap);
      res_bytes = -1;
    }
  }
  int narrow_cap = 256;
  if (eligible && (path == IPC_PATH_AUTO || path == IPC_PATH_NARROW || path == IPC_PATH_RESIDENT)) {
    const int lds = narrow_lds_bytes(dims, L, operand, esplit);
    const int cap = coresident_capacity([&] { return narrow_prepare(operand, esplit, act, lds); },
                                        [&](int* n) { return narrow_occupancy(operand, esplit, act, lds, n); });
    if (cap == 0) return fail(IPC_ERR_CONFIG, "the whole-step kernel cannot run on this device (capacity 0)");
    if (cap > 0 && cap < narrow_cap) narrow_cap = cap;
  }
  if (path == IPC_PATH_NARROW && !eligible)
    return fail(IPC_ERR_CONFIG,
                "the whole-step kernel needs fp32 storage, L <= %d, widths d_0..d_{L-1} <= %d and a column "
                "block that fits in LDS", NARROW_MAX_L, NARROW_MAX_WIDTH);
  const bool weligible = wide_eligible(storage, operand, esplit, weight_mode, B);
  if (path == IPC_PATH_WIDE && !weligible)
    return fail(IPC_ERR_CONFIG,
                "the wide path needs fp32 storage, fp16/bf16 operands, split 1 or 2 and the GEMM weight update");
  ipc_plan* p = new (std::nothrow) ipc_plan();
  if (!p) return fail(IPC_ERR_CONFIG, "out of host memory");
  p->L = L; p->B = B; p->storage = storage; p->operand = operand; p->act = act;
  p->split = esplit;
  p->alpha = alpha; p->gamma = gamma; p->recompute = recompute ? 1 : 0;
  p->wmode = weight_mode;
  p->dims.assign(dims, dims + L + 1);
  p->spin_limit = kNarrowSpinLimit;
  p->narrow_cap = narrow_cap;
  p->resident = path == IPC_PATH_RESIDENT || (path == IPC_PATH_AUTO && res_bytes >= 0);
  p->narrow = p->resident || path == IPC_PATH_NARROW || (path == IPC_PATH_AUTO && eligible);
  p->wide = !p->narrow && (path == IPC_PATH_WIDE || (path == IPC_PATH_AUTO && weligible));
  if (p->narrow) p->ws_bytes = narrow_workspace_bytes(dims, L, B, p->recompute != 0);
  if (p->resident) {
    p->rargs = ra;
    p->res_ws_off = (p->ws_bytes + 255) / 256 * 256;
    p->ws_bytes = p->res_ws_off + res_bytes;
  }
  if (p->wide) {
    // the split-2 prediction reads W itself when every contraction is whole k-steps
    p->wdirect = p->split == IPC_SPLIT_W;
    for (int l = 0; l < L; ++l) p->wdirect = p->wdirect && dims[l + 1] % WIDE_BK == 0;
    p->ws_bytes = WideLayout(p->dims, L, B, p->split == IPC_SPLIT_W, 0, p->wdirect).total;
  }
  *out = p;
  return ok();
}

int ipc_plan_fused(const ipc_plan* plan) { return plan && plan->narrow ? 1 : 0; }

int ipc_plan_path(const ipc_plan* plan) {
  if (!plan) return -1;
  if (plan->resident) return IPC_PATH_RESIDENT;
  return plan->narrow ? IPC_PATH_NARROW : plan->wide ? IPC_PATH_WIDE : IPC_PATH_PHASED;
}

long long ipc_plan_workspace_bytes(const ipc_plan* plan) { return plan ? plan->ws_bytes : 0; }

int ipc_plan_bind(ipc_plan* plan, void* const* x, void* const* e, void* const* w, void* const* a,
                  void* workspace) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  plan->release_graph();  // a captured graph holds the previous buffers' addresses
  if (plan->ws_bytes) {
    TRY(check_ptr(workspace, "workspace", 4));
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(IPC_ERR_ALIGN, "workspace must be 256-byte aligned");
  }
  if (!x || !e || !w) return fail(IPC_ERR_NULL, "x, e and w pointer arrays are required");
  if (!plan->recompute && !a) return fail(IPC_ERR_NULL, "save-activation plan needs the a[] array");
  const int L = plan->L, B = plan->B, es = elem_size(plan->storage);
  char name[32];
  for (int l = 0; l <= L; ++l) {
    snprintf(name, sizeof(name), "x[%d]", l);
    TRY(check_ptr(x[l], name, es));
    if (l < L) {
      snprintf(name, sizeof(name), "e[%d]", l);
      TRY(check_ptr(e[l], name, es));
      snprintf(name, sizeof(name), "w[%d]", l);
      TRY(check_ptr(w[l], name, es));
    }
    if (!plan->recompute && l >= 1) {
      snprintf(name, sizeof(name), "a[%d]", l);
      TRY(check_ptr(a[l], name, es));
    }
  }
  const std::vector<int>& d = plan->dims;
  plan->pred.clear(); plan->infer.clear(); plan->weight.clear(); plan->outer.clear(); plan->fwd.clear();
  // Prediction always applies f to x[l+1] in its loader (trainer.py:617-618);
  // only the weight update consumes the saved activation.
  for (int l = 0; l < L; ++l)
    plan->pred.push_back(make_pf(KIND_PRED, x[l + 1], w[l], x[l], e[l], d[l], d[l + 1], B, 1, plan->act, es));
  for (int l = 1; l < L; ++l) {
    plan->infer.push_back(make_inf(x[l], e[l], w[l - 1], e[l - 1], plan->recompute ? nullptr : a[l], d[l],
                                   d[l - 1], B, 1, plan->gamma, plan->act, es));
  }
  for (int l = 0; l < L; ++l) {
    const bool use_outer = plan->wmode == IPC_WMODE_OUTER || (plan->wmode == IPC_WMODE_AUTO && B <= 16);
    const void* src = plan->recompute ? x[l + 1] : a[l + 1];
    if (use_outer)
      plan->outer.push_back(make_outer(w[l], e[l], src, d[l], d[l + 1], B, 1, plan->alpha, plan->recompute, plan->act));
    else
      plan->weight.push_back(make_wgt(w[l], e[l], src, d[l], d[l + 1], B, 1, plan->alpha, plan->recompute, plan->act, es));
  }
  plan->act_src = x[L];
  plan->act_dst = plan->recompute ? nullptr : a[L];
  for (int l = L - 1; l >= 1; --l)
    plan->fwd.push_back(make_pf(KIND_FWD, x[l + 1], w[l], nullptr, x[l], d[l], d[l + 1], B, 1, plan->act, es));
  // One tile configuration per phase, chosen from the phase's total work.
  long long rows_p = 0, rows_i = 0, rows_w = 0, cols_w = 0;
  for (auto& q : plan->pred) rows_p += q.M;
  for (auto& q : plan->infer) rows_i += q.M;
  for (auto& q : plan->weight) { rows_w += q.M; cols_w = std::max(cols_w, (long long)q.N); }
  plan->tile_pred = pick_tile(rows_p, B, 1);
  plan->tile_infer = rows_i ? pick_tile(rows_i, B, 1) : 0;
  plan->tile_weight = rows_w ? pick_tile(rows_w, cols_w, 1) : 0;
  if (plan->tile_override[0] != IPC_TILE_AUTO) plan->tile_pred = plan->tile_override[0];
  if (plan->tile_override[1] != IPC_TILE_AUTO) plan->tile_infer = plan->tile_override[1];
  if (plan->tile_override[2] != IPC_TILE_AUTO) plan->tile_weight = plan->tile_override[2];
  plan->launches = 1 + (plan->infer.empty() ? 0 : 1) + (plan->weight.empty() ? 0 : 1) + (int)plan->outer.size();
  if (plan->narrow) {
    TRY(bind_whole_step(plan->nargs, plan->resident ? &plan->rargs : nullptr, L, d.data(), B, x, e, w,
                        plan->recompute ? nullptr : a, plan->act, plan->operand, plan->split, plan->alpha,
                        plan->gamma, narrow_outer(B, plan->wmode), plan->spin_limit, plan->narrow_cap,
                        static_cast<char*>(workspace), plan->res_ws_off));
    plan->launches = 1;
  }
  if (plan->wide) {
    const WideLayout lay(d, L, B, plan->split == IPC_SPLIT_W, plan->wcfg[0], plan->wdirect);
    if (plan->wdirect)
      for (int l = 0; l < L; ++l)
        if (reinterpret_cast<uintptr_t>(w[l]) % 16 != 0)
          return fail(IPC_ERR_ALIGN, "W[%d] must be 16-byte aligned: the wide prediction reads it directly", l);
    char* ws = static_cast<char*>(workspace);
    auto buf = [&](const WideLayout::Buf& b) -> void* { return b.off < 0 ? nullptr : ws + b.off; };
    auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    plan->wpred.clear(); plan->winfer.clear(); plan->wweight.clear(); plan->wsync.clear();
    std::vector<WideProblem> pred_layer;
    for (int l = 0; l < L; ++l) {
      WideProblem q{};
      q.M = d[l]; q.N = B; q.K = (int)lay.wh[l].ld;
      q.a = buf(lay.wh[l]); q.a_lo = buf(lay.wl[l]); q.lda = lay.wh[l].ld; q.a_lim = (int)lay.wh[l].rows;
      if (plan->wdirect) { q.a = w[l]; q.a_lo = nullptr; q.lda = d[l + 1]; q.a_lim = d[l]; }
      q.b = buf(lay.ft[l + 1]); q.ldb = lay.ft[l + 1].ld; q.b_lim = (int)lay.ft[l + 1].rows;
      q.out = e[l]; q.ldo = B;
      q.aux = x[l]; q.ldx = B;
      q.h = buf(lay.e[l]); q.ldh = lay.e[l].ld;
      q.t = buf(lay.et[l]); q.ldt = lay.et[l].ld;
      q.vec = B % 4 == 0 && a16(e[l]) && a16(x[l]);
      pred_layer.push_back(q);
    }
    int ncu = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
      ncu = 256;
    plan->pred_ksplit = wide_pred_ksplit(d, L, B, plan->split == IPC_SPLIT_W, plan->wcfg[0], lay, ncu);
    if (plan->ksplit_request > 0) {
      const int k = plan->ksplit_request;
      if (k > lay.part_smax || (k > 1 && lay.wh[0].ld % ((long long)k * WIDE_BK) != 0))
        return fail(IPC_ERR_CONFIG, "k-split %d is not available for this net (at most %d slices of whole k-steps)",
                    k, lay.part_smax);
      plan->pred_ksplit = k;
    }
    if (plan->pred_ksplit > 1) {
      // layer 0 last, as slices writing partial products; the reduce launch writes eps[0], E, ET
      for (int l = 1; l < L; ++l) plan->wpred.push_back(pred_layer[l]);
      WideProblem q = pred_layer[0];
      q.ksplit = plan->pred_ksplit;
      q.out = ws + lay.part_off; q.ldo = B;
      q.part_stride = lay.part_stride;
      q.aux = nullptr; q.h = nullptr; q.t = nullptr;
      plan->wpred.push_back(q);
      WideReduce& r = plan->wreduce;
      r = WideReduce{};
      r.part = reinterpret_cast<const float*>(ws + lay.part_off); r.part_stride = lay.part_stride; r.ldp = B;
      r.slices = plan->pred_ksplit; r.M = d[0]; r.N = B;
      r.x = static_cast<const float*>(x[0]); r.ldx = B;
      r.eps = static_cast<float*>(e[0]); r.lde = B;
      r.h = buf(lay.e[0]); r.ldh = lay.e[0].ld;
      r.t = buf(lay.et[0]); r.ldt = lay.et[0].ld;
      r.vec = pred_layer[0].vec;
    } else {
      plan->wpred = pred_layer;
    }
    for (int l = 1; l < L; ++l) {
      WideProblem q{};
      q.M = d[l]; q.N = B; q.K = (int)lay.wt[l - 1].ld;
      q.a = buf(lay.wt[l - 1]); q.lda = lay.wt[l - 1].ld; q.a_lim = (int)lay.wt[l - 1].rows;
      q.b = buf(lay.et[l - 1]); q.ldb = lay.et[l - 1].ld; q.b_lim = (int)lay.et[l - 1].rows;
      q.out = x[l]; q.ldo = B;
      q.aux = e[l]; q.ldx = B;
      q.h = buf(lay.f[l]); q.ldh = lay.f[l].ld;
      q.t = buf(lay.ft[l]); q.ldt = lay.ft[l].ld;
      q.out2 = plan->recompute ? nullptr : a[l]; q.ld2 = B;
      q.scal = plan->gamma;
      q.vec = B % 4 == 0 && a16(x[l]) && a16(e[l]) && (!q.out2 || a16(q.out2));
      plan->winfer.push_back(q);
    }
    for (int l = 0; l < L; ++l) {
      WideProblem q{};
      q.M = d[l]; q.N = d[l + 1]; q.K = (int)lay.e[l].ld;
      q.a = buf(lay.e[l]); q.lda = lay.e[l].ld; q.a_lim = (int)lay.e[l].rows;
      q.b = buf(lay.f[l + 1]); q.ldb = lay.f[l + 1].ld; q.b_lim = (int)lay.f[l + 1].rows;
      q.out = w[l]; q.ldo = d[l + 1];
      q.h = buf(lay.wh[l]); q.ldh = lay.wh[l].ld;  // null with wdirect: only W and WT are stored
      q.hl = buf(lay.wl[l]); q.ldhl = lay.wl[l].ld;
      q.t = buf(lay.wt[l]); q.ldt = lay.wt[l].ld;
      q.scal = plan->alpha;
      q.vec = d[l + 1] % 4 == 0 && a16(w[l]);
      plan->wweight.push_back(q);
    }
    for (int l = 0; l < L; ++l) {
      WideCopy c{};
      c.src = static_cast<const float*>(w[l]); c.lds = d[l + 1];
      c.rows = d[l]; c.cols = d[l + 1]; c.act = IPC_ACT_IDENTITY;
      c.dst = buf(lay.wh[l]); c.ldd = lay.wh[l].ld;
      c.dst_lo = buf(lay.wl[l]); c.ldl = lay.wl[l].ld;
      c.dst_t = buf(lay.wt[l]); c.ldt = lay.wt[l].ld;
      plan->wsync.push_back(c);
    }
    for (int l = 1; l <= L; ++l) {
      WideCopy c{};
      c.src = static_cast<const float*>(x[l]); c.lds = B;
      c.rows = d[l]; c.cols = B; c.act = plan->act;
      c.dst = buf(lay.f[l]); c.ldd = lay.f[l].ld;
      c.dst_t = buf(lay.ft[l]); c.ldt = lay.ft[l].ld;
      plan->wsync.push_back(c);
    }
    plan->wsync_init.assign(plan->wsync.begin(), plan->wsync.begin() + L);  // W copies
    plan->wsync_init.push_back(plan->wsync.back());                         // x[L] copies
    plan->wfwd.clear();
    for (int l = L - 1; l >= 1; --l) {
      WideProblem q = pred_layer[l];
      q.out = x[l]; q.ldo = B;
      q.aux = nullptr; q.ldx = 0;
      q.h = buf(lay.f[l]); q.ldh = lay.f[l].ld;
      q.t = buf(lay.ft[l]); q.ldt = lay.ft[l].ld;
      q.vec = B % 4 == 0 && a16(x[l]);
      plan->wfwd.push_back(q);
    }
    TRY(launch_rc(wide_prepare(), "wide path LDS limit"));
    auto chunks = [](int n) { return (n + WIDE_MAX_BATCH - 1) / WIDE_MAX_BATCH; };
    plan->launches = 2 * chunks(L) + chunks(L - 1) + (plan->pred_ksplit > 1 ? 1 : 0);
  }
  plan->workspace = workspace;
  plan->bound = true;
  plan->res_stale = plan->resident;
  return ok();
}

}  // extern "C"

namespace {

int run_phase(ipc_plan* plan, int phase, hipStream_t s) {
  if (plan->wide) {
    switch (phase) {
      case IPC_PHASE_PRED:
        TRY(launch_rc(launch_wide(WIDE_PRED, plan->wpred.data(), (int)plan->wpred.size(), plan->operand,
                                  plan->split == IPC_SPLIT_W ? 2 : 1, plan->act, s, plan->wcfg[0], plan->wdirect),
                      "wide prediction phase"));
        if (plan->pred_ksplit > 1)
          return launch_rc(launch_wide_reduce(plan->wreduce, plan->operand, s), "wide prediction reduce");
        return ok();
      case IPC_PHASE_INFER:
        return launch_rc(launch_wide(WIDE_INFER, plan->winfer.data(), (int)plan->winfer.size(), plan->operand, 1,
                                     plan->act, s, plan->wcfg[1]), "wide inference phase");
      default:
        return launch_rc(launch_wide(WIDE_WEIGHT, plan->wweight.data(), (int)plan->wweight.size(), plan->operand, 1,
                                     plan->act, s, plan->wcfg[2]), "wide weight phase");
    }
  }
  switch (phase) {
    case IPC_PHASE_PRED:
      return launch_rc(launch_gemm(plan->pred.data(), (int)plan->pred.size(), plan->storage, plan->operand,
                                   plan->split, plan->tile_pred, s), "plan prediction phase");
    case IPC_PHASE_INFER:
      if (plan->infer.empty()) return ok();
      return launch_rc(launch_gemm(plan->infer.data(), (int)plan->infer.size(), plan->storage, plan->operand,
                                   IPC_SPLIT_NONE, plan->tile_infer, s), "plan inference phase");
    default:
      if (!plan->weight.empty())
        TRY(launch_rc(launch_gemm(plan->weight.data(), (int)plan->weight.size(), plan->storage, plan->operand,
                                  IPC_SPLIT_NONE, plan->tile_weight, s), "plan weight phase"));
      for (auto& q : plan->outer) TRY(launch_rc(launch_outer(q, plan->storage, s), "plan outer weight update"));
      return ok();
  }
}

}  // namespace

extern "C" {

int ipc_plan_step(ipc_plan* plan, int steps, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  if (steps < 0) return fail(IPC_ERR_SHAPE, "steps must be >= 0");
  hipStream_t s = (hipStream_t)stream;
  if (plan->narrow) return steps > 0 ? launch_narrow_mode(plan, NMODE_STEPS, steps, s) : ok();
  for (int t = 0; t < steps; ++t)
    for (int phase = IPC_PHASE_PRED; phase <= IPC_PHASE_WEIGHT; ++phase) TRY(run_phase(plan, phase, s));
  return ok();
}

int ipc_plan_phase(ipc_plan* plan, int phase, int reps, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  if (phase < IPC_PHASE_PRED || phase > IPC_PHASE_WEIGHT) return fail(IPC_ERR_CONFIG, "unknown phase %d", phase);
  if (reps < 0) return fail(IPC_ERR_SHAPE, "reps must be >= 0");
  if (plan->narrow) {
    if (phase == IPC_PHASE_INFER) return ok();
    const int mode = phase == IPC_PHASE_PRED ? NMODE_PHASE_A : NMODE_PHASE_B;
    for (int r = 0; r < reps; ++r) TRY(launch_narrow_mode(plan, mode, 1, (hipStream_t)stream));
    return ok();
  }
  for (int r = 0; r < reps; ++r) TRY(run_phase(plan, phase, (hipStream_t)stream));
  return ok();
}

int ipc_plan_forward_init(ipc_plan* plan, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  hipStream_t s = (hipStream_t)stream;
  if (plan->narrow) return launch_narrow_mode(plan, NMODE_FORWARD, 1, s);
  if (plan->act_dst) {
    const long long n = (long long)plan->dims[plan->L] * plan->B;
    TRY(launch_rc(launch_act(plan->act_src, plan->act_dst, n, plan->act, plan->storage, s), "plan a[L] = f(x[L])"));
  }
  if (plan->wide) {
    // W and f(x[L]) copies, then the layers top-down with the prediction
    // kernel (its epilogue writes x[l] and the f(x[l]) copies the next layer reads)
    TRY(launch_rc(launch_wide_copy(plan->wsync_init.data(), (int)plan->wsync_init.size(), plan->operand, s),
                  "wide operand copies"));
    for (auto& q : plan->wfwd)
      TRY(launch_rc(launch_wide(WIDE_FWD, &q, 1, plan->operand, plan->split == IPC_SPLIT_W ? 2 : 1, plan->act, s, 0,
                                plan->wdirect),
                    "wide forward init"));
    return ok();
  }
  for (auto& q : plan->fwd) {
    const int tile = pick_tile(q.M, q.N, 1);
    TRY(launch_rc(launch_gemm(&q, 1, plan->storage, plan->operand, plan->split, tile, s), "plan forward init"));
  }
  return ok();
}

int ipc_plan_sync(ipc_plan* plan, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  if (plan->resident)
    return launch_rc(resident_invalidate(plan->rargs, (hipStream_t)stream), "layer-resident input images");
  if (!plan->wide) return ok();
  return launch_rc(launch_wide_copy(plan->wsync.data(), (int)plan->wsync.size(), plan->operand, (hipStream_t)stream),
                   "wide operand copies");
}

int ipc_plan_set_tiles(ipc_plan* plan, int tile_pred, int tile_infer, int tile_weight) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  const int t[3] = {tile_pred, tile_infer, tile_weight};
  for (int i = 0; i < 3; ++i)
    if (t[i] != IPC_TILE_AUTO && (t[i] < IPC_TILE_32x32 || t[i] > IPC_TILE_128x128))
      return fail(IPC_ERR_CONFIG, "plan tile %d must be IPC_TILE_AUTO or a generic tile 0-2", t[i]);
  for (int i = 0; i < 3; ++i) plan->tile_override[i] = t[i];
  if (plan->bound) {
    if (t[0] != IPC_TILE_AUTO) plan->tile_pred = t[0];
    if (t[1] != IPC_TILE_AUTO) plan->tile_infer = t[1];
    if (t[2] != IPC_TILE_AUTO) plan->tile_weight = t[2];
  }
  return ok();
}

int ipc_plan_launch_count(const ipc_plan* plan) { return plan ? plan->launches : 0; }

int ipc_plan_wide_config_count(int phase, int split) {
  if (phase == IPC_PHASE_PRED) return split == IPC_SPLIT_W ? wide_config_count(WIDE_PRED, 2)
                                                           : split == IPC_SPLIT_NONE ? wide_config_count(WIDE_PRED, 1) : 0;
  if (phase == IPC_PHASE_INFER) return wide_config_count(WIDE_INFER, 1);
  if (phase == IPC_PHASE_WEIGHT) return wide_config_count(WIDE_WEIGHT, 1);
  return 0;
}

int ipc_plan_set_wide_config(ipc_plan* plan, int pred_cfg, int infer_cfg, int weight_cfg, int ksplit) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->wide) return fail(IPC_ERR_CONFIG, "the plan does not run the wide path");
  if (plan->bound) return fail(IPC_ERR_STATE, "set the wide configuration before ipc_plan_bind");
  const int c[3] = {pred_cfg, infer_cfg, weight_cfg};
  for (int ph = 0; ph < 3; ++ph) {
    const int n = ipc_plan_wide_config_count(ph, plan->split);
    if (c[ph] < -1 || c[ph] >= n)
      return fail(IPC_ERR_CONFIG, "phase %d has tile configurations 0..%d (-1 = default); got %d", ph, n - 1, c[ph]);
  }
  if (ksplit < -1 || ksplit == 0 || ksplit > 16 || (ksplit > 0 && (ksplit & (ksplit - 1))))
    return fail(IPC_ERR_CONFIG, "k-split must be -1 (automatic) or a power of two in [1, 16]; got %d", ksplit);
  for (int ph = 0; ph < 3; ++ph) plan->wcfg[ph] = c[ph] < 0 ? 0 : c[ph];
  plan->ksplit_request = ksplit < 0 ? 0 : ksplit;
  // the prediction tile sets how many k-split slices the workspace holds
  plan->ws_bytes =
      WideLayout(plan->dims, plan->L, plan->B, plan->split == IPC_SPLIT_W, plan->wcfg[0], plan->wdirect).total;
  return ok();
}

int ipc_plan_set_resident_rows(ipc_plan* plan, int rows) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->resident) return fail(IPC_ERR_CONFIG, "the plan does not run the layer-resident kernel");
  if (plan->bound) return fail(IPC_ERR_STATE, "set the row-block size before ipc_plan_bind");
  if (rows == -1) rows = RES_TOP_ROWS;
  if (rows != 16 && rows != 32 && rows != 64)
    return fail(IPC_ERR_CONFIG, "the top layer's row blocks are 16, 32 or 64 rows (-1 = default %d); got %d",
                RES_TOP_ROWS, rows);
  ResidentArgs ra{};
  const long long res_bytes = resident_eligible(plan->L, plan->dims.data(), plan->B, plan->operand, plan->split,
                                                plan->wmode, true, ra, rows);
  if (res_bytes < 0)
    return fail(IPC_ERR_CONFIG, "row blocks of %d rows do not fit this net's layer-resident launch (LDS or flags)",
                rows);
  const int cap = coresident_capacity(
      [&] { return resident_prepare(plan->operand, plan->split, plan->act, ra.lds_bytes); },
      [&](int* n) { return resident_occupancy(plan->operand, plan->split, plan->act, ra.lds_bytes, n); });
  if (cap >= 0 && resident_launch_blocks(ra) > cap)
    return fail(IPC_ERR_CONFIG, "row blocks of %d rows need %d co-resident workgroups; this device holds %d", rows,
                resident_launch_blocks(ra), cap);
  plan->rargs = ra;
  plan->ws_bytes = plan->res_ws_off + res_bytes;
  return ok();
}

int ipc_plan_resident_rows(const ipc_plan* plan) { return plan && plan->resident ? plan->rargs.top_rows : 0; }

int ipc_plan_set_spin_limit(ipc_plan* plan, int limit) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  plan->spin_limit = limit < 0 ? kNarrowSpinLimit : limit;
  plan->nargs.spin_limit = plan->spin_limit;
  plan->rargs.spin_limit = plan->spin_limit;
  return ok();
}

int ipc_plan_check(ipc_plan* plan, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  hipStream_t s = (hipStream_t)stream;
  if (!plan->narrow || !plan->workspace) {
    if (hipStreamSynchronize(s) != hipSuccess) return fail(IPC_ERR_LAUNCH, "stream synchronisation failed");
    return ok();
  }
  unsigned* word = static_cast<unsigned*>(plan->workspace) + 2;
  unsigned flag = 0;
  if (hipMemcpyAsync(&flag, word, sizeof(flag), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(IPC_ERR_LAUNCH, "reading the whole-step kernel's timeout word failed");
  if (flag == 0) return ok();
  const unsigned zero = 0;
  if (hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(IPC_ERR_LAUNCH, "clearing the whole-step kernel's timeout word failed");
  return fail(IPC_ERR_TIMEOUT,
              "a wait of the whole-step kernel ran past its spin limit: the workgroups of a launch were not all "
              "running at once (another kernel held CUs), and the outputs of the steps since the last check are "
              "invalid");
}

int ipc_plan_graph_capture(ipc_plan* plan, int steps) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->bound) return fail(IPC_ERR_STATE, "plan has no bound buffers");
  if (steps < 1) return fail(IPC_ERR_SHAPE, "steps must be >= 1 (got %d)", steps);
  plan->release_graph();
  if (plan->narrow) {
    // `steps` steps of a whole-step plan are one kernel launch with fixed
    // arguments: replaying that launch is what a one-node graph would do,
    // without the graph launch's own cost (measured on MI355X: 49.1 us per
    // replay of a one-node hipGraph of the d6 layer-resident launch against
    // 44.3 us per direct launch, back to back)
    plan->graph_steps = steps;
    plan->graph_direct = true;
    return ok();
  }
  if (!plan->cap_stream && hipStreamCreateWithFlags(&plan->cap_stream, hipStreamNonBlocking) != hipSuccess) {
    plan->cap_stream = nullptr;
    return fail(IPC_ERR_LAUNCH, "creating the capture stream failed");
  }
  if (hipStreamBeginCapture(plan->cap_stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return fail(IPC_ERR_LAUNCH, "hipStreamBeginCapture failed");
  const int rc = ipc_plan_step(plan, steps, plan->cap_stream);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(plan->cap_stream, &g);
  if (rc != IPC_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (ec != hipSuccess || !g) return fail(IPC_ERR_LAUNCH, "hipStreamEndCapture failed: %s", hipGetErrorString(ec));
  const hipError_t ei = hipGraphInstantiate(&plan->graph_exec, g, nullptr, nullptr, 0);
  if (ei != hipSuccess) {
    plan->graph_exec = nullptr;
    (void)hipGraphDestroy(g);
    return fail(IPC_ERR_LAUNCH, "hipGraphInstantiate failed: %s", hipGetErrorString(ei));
  }
  plan->graph = g;
  plan->graph_steps = steps;
  return ok();
}

int ipc_plan_graph_launch(ipc_plan* plan, int repeats, void* stream) {
  if (!plan) return fail(IPC_ERR_NULL, "plan is NULL");
  if (!plan->graph_exec && !plan->graph_direct)
    return fail(IPC_ERR_STATE, "the plan has no captured graph (ipc_plan_graph_capture)");
  if (repeats < 0) return fail(IPC_ERR_SHAPE, "repeats must be >= 0");
  if (plan->graph_direct) {
    for (int r = 0; r < repeats; ++r)
      TRY(launch_narrow_mode(plan, NMODE_STEPS, plan->graph_steps, (hipStream_t)stream));
    return ok();
  }
  for (int r = 0; r < repeats; ++r) {
    const hipError_t e = hipGraphLaunch(plan->graph_exec, (hipStream_t)stream);
    if (e != hipSuccess) return fail(IPC_ERR_LAUNCH, "hipGraphLaunch failed: %s", hipGetErrorString(e));
  }
  return ok();
}

int ipc_plan_graph_steps(const ipc_plan* plan) {
  return plan && (plan->graph_exec || plan->graph_direct) ? plan->graph_steps : 0;
}

int ipc_steps_noalloc(int L, const int* dims, int B, void* const* x, void* const* e, void* const* w, int operand,
                      int split, int act, float alpha, float gamma, int weight_mode, int steps, void* stream) {
  if (!dims) return fail(IPC_ERR_NULL, "dims is NULL");
  if (!x || !e || !w) return fail(IPC_ERR_NULL, "x, e and w pointer arrays are required");
  if (L < 1 || L > NARROW_MAX_L) return fail(IPC_ERR_SHAPE, "L must be in [1, %d] (got %d)", NARROW_MAX_L, L);
  TRY(check_dtypes(IPC_DT_F32, operand));
  TRY(check_split(split));
  TRY(check_act(act));
  if (weight_mode < IPC_WMODE_GEMM || weight_mode > IPC_WMODE_AUTO)
    return fail(IPC_ERR_CONFIG, "unknown weight mode %d", weight_mode);
  for (int l = 0; l < L; ++l) TRY(check_dims(dims[l], dims[l + 1], B, 1));
  if (weight_mode == IPC_WMODE_OUTER && B > kOuterMaxB)
    return fail(IPC_ERR_SHAPE, "outer weight mode supports B <= %d (got %d)", kOuterMaxB, B);
  if (steps < 0) return fail(IPC_ERR_SHAPE, "steps must be >= 0");
  const int esplit = effective_split(IPC_DT_F32, operand, split);
  if (!narrow_eligible(L, dims, IPC_DT_F32, operand, esplit))
    return fail(IPC_ERR_CONFIG,
                "ipc_steps_noalloc runs the whole-step kernels only: widths d_0..d_{L-1} <= %d, L <= %d, split 1 "
                "or 3 and a column block that fits in LDS", NARROW_MAX_WIDTH, NARROW_MAX_L);
  char name[32];
  for (int l = 0; l <= L; ++l) {
    snprintf(name, sizeof(name), "x[%d]", l);
    TRY(check_ptr(x[l], name, 4));
    if (l < L) {
      snprintf(name, sizeof(name), "e[%d]", l);
      TRY(check_ptr(e[l], name, 4));
      snprintf(name, sizeof(name), "w[%d]", l);
      TRY(check_ptr(w[l], name, 4));
    }
  }
  // scratch the launch needs: the column kernel's barrier words and f(x)
  // buffers, then the layer-resident kernel's flags and exchange records
  ResidentArgs ra{};
  long long res_bytes = resident_eligible(L, dims, B, operand, esplit, weight_mode, true, ra);
  long long need = narrow_workspace_bytes(dims, L, B, true), res_off = 0;
  if (res_bytes >= 0) {
    res_off = (need + 255) / 256 * 256;
    need = res_off + res_bytes;
  }
  if (need > kScratchBytes)
    return fail(IPC_ERR_SHAPE,
                "this net needs %lld bytes of scratch; the library's static scratch holds %lld (use a plan with a "
                "caller workspace)", need, kScratchBytes);
  if (steps == 0) return ok();
  char* ws = nullptr;
  TRY(scratch_address(&ws));
  if (res_bytes >= 0) {
    const int cap = coresident_capacity([&] { return resident_prepare(operand, esplit, act, ra.lds_bytes); },
                                        [&](int* n) { return resident_occupancy(operand, esplit, act, ra.lds_bytes, n); });
    if (cap >= 0 && resident_launch_blocks(ra) > cap) res_bytes = -1;
  }
  const int lds = narrow_lds_bytes(dims, L, operand, esplit);
  int cap = coresident_capacity([&] { return narrow_prepare(operand, esplit, act, lds); },
                                [&](int* n) { return narrow_occupancy(operand, esplit, act, lds, n); });
  if (cap == 0) return fail(IPC_ERR_CONFIG, "the whole-step kernel cannot run on this device (capacity 0)");
  cap = cap < 0 || cap > 256 ? 256 : cap;
  NarrowArgs na{};
  TRY(bind_whole_step(na, res_bytes >= 0 ? &ra : nullptr, L, dims, B, x, e, w, nullptr, act, operand, esplit, alpha,
                      gamma, narrow_outer(B, weight_mode),
                      g_noalloc_spin_limit >= 0 ? g_noalloc_spin_limit : kNarrowSpinLimit, cap, ws, res_off));
  hipStream_t s = (hipStream_t)stream;
  // the scratch keeps the previous call's contents: the barrier words and the
  // resident flag area (step flags, cache generation and the workgroups'
  // cache slots: zeros mark every cache stale) must start at zero; everything
  // else is written before it is read
  hipLaunchKernelGGL(scratch_clear_kernel, dim3(1), dim3(RES_FLAG_BYTES / 4), 0, s, reinterpret_cast<unsigned*>(ws),
                     res_bytes >= 0 ? reinterpret_cast<unsigned*>(ws + res_off) : nullptr);
  TRY(launch_rc(hipGetLastError(), "scratch clear"));
  if (res_bytes >= 0) {
    ra.steps = steps;
    return launch_rc(launch_resident(ra, operand, esplit, act, s), "layer-resident whole-step kernel");
  }
  na.mode = NMODE_STEPS;
  na.steps = steps;
  return launch_rc(launch_narrow(na, operand, esplit, s), "whole-step kernel");
}

int ipc_noalloc_check(void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (hipStreamSynchronize(s) != hipSuccess) return fail(IPC_ERR_LAUNCH, "stream synchronisation failed");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(IPC_ERR_DEVICE, "no current device");
  char* ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ws = g_scratch_ptr[dev];
  }
  if (!ws) return ok();  // no call has run on this device yet
  unsigned* word = reinterpret_cast<unsigned*>(ws) + 2;
  unsigned flag = 0;
  if (hipMemcpyAsync(&flag, word, sizeof(flag), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(IPC_ERR_LAUNCH, "reading the scratch's timeout word failed");
  if (flag == 0) return ok();
  const unsigned zero = 0;
  if (hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail(IPC_ERR_LAUNCH, "clearing the scratch's timeout word failed");
  return fail(IPC_ERR_TIMEOUT,
              "a wait of an ipc_steps_noalloc call ran past its spin limit: the outputs of the calls on this device "
              "since the last check are invalid");
}

int ipc_noalloc_set_spin_limit(int limit) {
  g_noalloc_spin_limit = limit < 0 ? -1 : limit;
  return ok();
}

int ipc_set_coresident_limit(int blocks) {
  if (blocks < 0) return fail(IPC_ERR_CONFIG, "the co-resident limit must be >= 0 (got %d)", blocks);
  g_coresident_limit = blocks;
  return ok();
}

int ipc_wide_problem_check(int phase, int split, int fp32_w, int has_lo, int K, int ksplit) {
  int mode;
  switch (phase) {
    case IPC_PHASE_PRED: mode = WIDE_PRED; break;
    case IPC_PHASE_INFER: mode = WIDE_INFER; break;
    case IPC_PHASE_WEIGHT: mode = WIDE_WEIGHT; break;
    case IPC_PHASE_FORWARD: mode = WIDE_FWD; break;
    default: return fail(IPC_ERR_CONFIG, "unknown phase %d", phase);
  }
  WideProblem q{};
  static const unsigned char dummy[16] = {};
  q.M = q.N = 64;
  q.K = K;
  q.a = q.b = dummy;
  q.a_lo = has_lo ? dummy : nullptr;
  q.ksplit = ksplit;
  if (!wide_problem_ok(mode, split, fp32_w != 0, q))
    return fail(IPC_ERR_CONFIG, "LDS-DMA GEMM problem refused on the host (phase %d, split %d, fp32 W %d, lo %d, "
                "K %d, k-split %d)", phase, split, fp32_w, has_lo, K, ksplit);
  return ok();
}

int ipc_s16_preactivates(int kind, int act, int M, int K, int B) {
  const int mode = kind == IPC_PHASE_PRED ? S16_PRED : kind == IPC_PHASE_WEIGHT ? S16_WEIGHT : S16_INFER;
  return s16_preact_rule(mode, act, M, K, (long long)K * B) ? 1 : 0;
}

long long ipc_s16_workspace_bytes(int kind, int act, int M, int K, int B, int groups) {
  if (M < 1 || K < 1 || B < 1 || groups < 1) return 0;
  const int mode = kind == IPC_PHASE_PRED ? S16_PRED : kind == IPC_PHASE_WEIGHT ? S16_WEIGHT : S16_INFER;
  return s16_workspace_need(mode, act, M, K, (long long)K * B, groups);
}

int ipc_set_s16_preactivate(int mode) {
  if (mode < -1 || mode > 1) return fail(IPC_ERR_CONFIG, "pre-activation mode must be -1, 0 or 1 (got %d)", mode);
  g_s16_preact = mode;
  return ok();
}

void ipc_plan_destroy(ipc_plan* plan) { delete plan; }

}  // extern "C"
