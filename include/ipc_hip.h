/*
 * ipc_hip.h - C ABI of the MI355X (gfx950) iPC training-step library.
 *
 * The library replaces the reference's TileLang kernel builders
 * (src/ipc_tilelang/tilelang_kernels.py, src/ipc_tilelang/layer_batching.py,
 * src/ipc_tilelang/weight_update_specialization.py) and the per-layer launch
 * loop of TileLangIPC.step_initialized (src/ipc_tilelang/trainer.py:601-679).
 *
 * Conventions (reference README.md:41-50, reference.py:35-59):
 *   x[0] = fixed one-hot target, x[L] = fixed input, W[l] is [d_l, d_{l+1}]
 *   and maps f(x[l+1]) -> x[l]; every tensor is contiguous, row-major and
 *   feature-major ([features, batch]).  Grouped ("batched", grid.z) calls take
 *   contiguous [groups, rows, cols] tensors.
 *
 * Ownership: the caller owns every buffer.  Kernels mutate their outputs in
 * place, allocate nothing and never synchronise the stream (ipc_plan_check
 * is the one entry point that synchronises).  Every call is
 * enqueued on the hipStream_t passed as `stream` (NULL = the null stream), so
 * calls can be captured into a hipGraph.
 *
 * Errors: every entry point returns IPC_OK (0) or a negative IPC_ERR_* code
 * and never throws; ipc_last_error() returns the calling thread's message.
 * Argument validation happens on the host before any HIP call.
 */
#ifndef IPC_HIP_H
#define IPC_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

#define IPC_ABI_VERSION 6

/* status codes */
#define IPC_OK 0
#define IPC_ERR_NULL (-1)     /* a required pointer is NULL                  */
#define IPC_ERR_SHAPE (-2)    /* a dimension is < 1 or too large              */
#define IPC_ERR_DTYPE (-3)    /* unknown dtype or unsupported combination     */
#define IPC_ERR_ACT (-4)      /* unknown activation                           */
#define IPC_ERR_ALIGN (-5)    /* pointer not aligned to its element size      */
#define IPC_ERR_DEVICE (-6)   /* no device, or the device is not gfx950       */
#define IPC_ERR_LAUNCH (-7)   /* the HIP launch failed                        */
#define IPC_ERR_CONFIG (-8)   /* unknown tile config or plan option           */
#define IPC_ERR_STATE (-9)    /* plan used before its buffers were bound      */
#define IPC_ERR_TIMEOUT (-10) /* a whole-step kernel's wait ran past its spin
                                 limit: that launch's outputs are invalid     */

/* element types (storage and GEMM operand) */
#define IPC_DT_F32 0
#define IPC_DT_F16 1
#define IPC_DT_BF16 2

/* activations: activations.py:9-29 and tilelang_kernels.py:61-96;
 * IPC_ACT_IDENTITY is the linear case of weight_update_specialization.py:96-102 */
#define IPC_ACT_IDENTITY 0
#define IPC_ACT_RELU 1
#define IPC_ACT_TANH 2
#define IPC_ACT_SIGMOID 3
#define IPC_ACT_SILU 4
#define IPC_ACT_GELU 5

/* tile configurations of the MFMA GEMM family; IPC_TILE_AUTO picks by shape.
 * IPC_TILE_DMA_* are the LDS-DMA kernel (operands streamed HBM -> LDS without
 * VGPR staging, transposed operands read with the LDS transpose read) in
 * four tile configurations: 256 x 128, 128 x 256,
 * 128 x 128 (more tiles for small shapes) and 256 x 256 (8 waves of 128 x 64,
 * half the LDS reads per MFMA, an epilogue from the registers; for large
 * shapes).  They give bit-identical results
 * (the same k order) and serve 16-bit storage (storage == operand ==
 * fp16/bf16) with a contraction that is a multiple of 64, 16-byte aligned
 * tensors and, for operands read transposed, a contiguous extent that is a
 * multiple of 8; IPC_TILE_AUTO picks the 256 x 256 one whenever those hold
 * and its tiles fill every CU at least once (256 tiles or more over the
 * groups), the 256 x 128 one when they hold otherwise; asking for a DMA tile
 * where they do not hold is IPC_ERR_CONFIG.  The autotuner
 * searches all of them per shape. */
#define IPC_TILE_AUTO (-1)
#define IPC_TILE_32x32 0
#define IPC_TILE_64x64 1
#define IPC_TILE_128x128 2
#define IPC_TILE_DMA_256x128 3
#define IPC_TILE_DMA_128x256 4
#define IPC_TILE_DMA_128x128 5
#define IPC_TILE_DMA_256x256 6
#define IPC_TILE_COUNT 7

/* weight-update backends of a plan */
#define IPC_WMODE_GEMM 0
#define IPC_WMODE_OUTER 1
#define IPC_WMODE_AUTO 2

/* Library version of this header's ABI. */
int ipc_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ipc_last_error(void);

/* Writes the gcnArchName of `device` into buf (NUL-terminated) and returns
 * IPC_OK if it is a gfx950 part, IPC_ERR_DEVICE otherwise.  Replaces the
 * SM86 gate of trainer.py:58-63. */
int ipc_device_check(int device, char* buf, int buflen);

/*
 * Prediction + error, E[g] = X_lower[g] - W[g] @ f(X_upper[g]).
 * Replaces build_prediction_error(M,K,B,act,dtype,cfg)(X_upper,W,X_lower,E)
 * (tilelang_kernels.py:114-177) and, for groups > 1,
 * build_prediction_error_batched (layer_batching.py:89-150).
 * X_upper [G,K,B], W [G,M,K], X_lower/E [G,M,B].  f is applied in the operand
 * loader; out-of-range tail elements are zero after f.  With 16-bit storage
 * the subtraction is rounded like tilelang_kernels.py:173.
 * storage: element type of all four tensors; operand: type the GEMM operands
 * are rounded to (must equal storage when storage is 16-bit); accumulation is
 * always fp32.  split (fp32 storage with 16-bit operands only, else 1):
 * 1 = one MFMA per block; 2 = W carried as hi + lo 16-bit terms (2 MFMAs);
 * 3 = W and f(X_upper) both split, hi*hi + lo*hi + hi*lo (3 MFMAs).  The
 * prediction error is a cancelling difference, and the split keeps its error
 * near fp32 level.
 */
#define IPC_SPLIT_NONE 1
#define IPC_SPLIT_W 2
#define IPC_SPLIT_WX 3
int ipc_pred_err(const void* x_upper, const void* w, const void* x_lower, void* e,
                 int M, int K, int B, int groups,
                 int storage, int operand, int split, int act, int tile, void* stream);

/*
 * Forward prediction OUT[g] = W[g] @ f(X_upper[g]).  Used for the hidden-state
 * forward initialisation (trainer.py:512-515) and predict() (trainer.py:828-833).
 */
int ipc_forward(const void* x_upper, const void* w, void* out,
                int M, int K, int B, int groups,
                int storage, int operand, int split, int act, int tile, void* stream);

/*
 * Inference update X[g] += gamma * (-E[g] + f'(X[g]) * W_lower[g]^T @ E_lower[g]),
 * optionally writing A_out[g] = f(X_new).  Replaces
 * build_inference_update(M,K,B,act,dtype,cfg,gamma,save)(X,E,W_lower,E_lower[,A_out])
 * (tilelang_kernels.py:180-265) and build_inference_update_batched
 * (layer_batching.py:153-248).  X/E/A_out [G,M,B], W_lower [G,K,M] read
 * transposed without a global transpose, E_lower [G,K,B].  a_out may be NULL.
 */
int ipc_infer_update(void* x, const void* e, const void* w_lower, const void* e_lower, void* a_out,
                     int M, int K, int B, int groups, float gamma,
                     int storage, int operand, int act, int tile, void* stream);

/*
 * Weight update W[g] += alpha * E[g] @ A[g]^T with A = f(X_upper) when
 * recompute != 0, else A = the saved activation passed as x_upper.  Replaces
 * build_weight_update(M,K,B,act,dtype,cfg,alpha,recompute)(W,E,X_upper_or_A)
 * (tilelang_kernels.py:268-349) and build_weight_update_batched
 * (layer_batching.py:251-346).  W [G,M,K], E [G,M,B], X_upper/A [G,K,B].
 * The epilogue is W = cast(float(W) + alpha*acc) (tilelang_kernels.py:319-320).
 */
int ipc_weight_update(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                      float alpha, int recompute, int storage, int operand, int act, int tile,
                      void* stream);

/*
 * Rank-B outer-product weight update for small batches (B <= 32):
 * W[g] += alpha * sum_b E[g][:,b] f(X_upper[g][:,b])^T, accumulated in fp32.
 * Replaces SmallBWeightUpdater (weight_update_specialization.py:63-128) with
 * the +alpha sign of the GEMM path and of reference.py:57 (the reference's
 * -alpha there is a sign error) and with every activation, not only relu.
 */
int ipc_weight_update_outer(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                            float alpha, int recompute, int storage, int act, void* stream);

/*
 * Whole-step plan: one call enqueues a complete iPC step (all prediction
 * errors, then the inference updates l = 1..L-1, then all weight updates),
 * replacing the Python launch loop of TileLangIPC.step_initialized
 * (trainer.py:601-679) and, when captured, IPCGraphRunner (cuda_graph.py:6-36).
 * dims has L+1 entries (dims[0] = classes, dims[L] = input features).
 */
typedef struct ipc_plan ipc_plan;

/* split applies to the prediction phase and the forward initialisation.
 * path selects the kernels a plan runs:
 *   IPC_PATH_AUTO    the layer-resident whole-step kernel when eligible (see
 *                    IPC_PATH_RESIDENT), else the column-block whole-step
 *                    kernel when the net is narrow (fp32 storage, every output
 *                    width d_0..d_{L-1} <= 128, L <= 16, split 1 or 3, one
 *                    column block's buffers fit in LDS), else the wide GEMM
 *                    path when eligible, else the phased path;
 *   IPC_PATH_PHASED  one generic multi-layer launch per phase (any config);
 *   IPC_PATH_NARROW  the column-block whole-step kernel (IPC_ERR_CONFIG if
 *                    not narrow);
 *   IPC_PATH_RESIDENT  multi-step launches on the layer-resident whole-step
 *                    kernel (every workgroup keeps one layer's W, or a column
 *                    chunk of the top layer's, on chip for all steps and
 *                    exchanges only eps and f'(x) W^T eps with its neighbours): a
 *                    narrow net with fp16/bf16 operands, split 1 or 3, L >= 2,
 *                    d_0..d_{L-1} <= 64, B <= 128 and the GEMM weight update
 *                    (weight mode GEMM, or AUTO with B > 16); IPC_ERR_CONFIG
 *                    otherwise.  Single-phase launches and the forward
 *                    initialisation of such a plan run on the column kernel;
 *   IPC_PATH_WIDE    one LDS-DMA MFMA launch per phase over 16-bit operand
 *                    copies kept in the workspace: fp32 storage, fp16/bf16
 *                    operands, split 1 or 2, GEMM weight update (weight mode
 *                    GEMM, or AUTO with B > 16); IPC_ERR_CONFIG otherwise.
 * The IPC_FUSED_* names are the same values (AUTO, OFF = PHASED, ON = NARROW). */
#define IPC_PATH_AUTO (-1)
#define IPC_PATH_PHASED 0
#define IPC_PATH_NARROW 1
#define IPC_PATH_WIDE 2
#define IPC_PATH_RESIDENT 3
#define IPC_FUSED_AUTO IPC_PATH_AUTO
#define IPC_FUSED_OFF IPC_PATH_PHASED
#define IPC_FUSED_ON IPC_PATH_NARROW
int ipc_plan_create(ipc_plan** out, int L, const int* dims, int B,
                    int storage, int operand, int split, int act, float alpha, float gamma,
                    int recompute, int weight_mode, int path);

/* 1 if the plan runs a whole-step kernel (column-block or layer-resident), 0 otherwise. */
int ipc_plan_fused(const ipc_plan* plan);

/* The path the plan runs (IPC_PATH_PHASED, _NARROW, _WIDE or _RESIDENT), -1 for NULL. */
int ipc_plan_path(const ipc_plan* plan);

/* Bytes of zero-initialised device workspace ipc_plan_bind needs (0 for the
 * phased path).  The first 256 bytes hold the column-block whole-step
 * kernel's grid-barrier counters, which it leaves zero after every launch
 * (word 2 becomes non-zero if a wait ever ran past its spin limit); in
 * recompute mode that kernel keeps the f(x[l]) values phase A evaluates for
 * the weight update after them.  A layer-resident plan then keeps, after
 * those: its per-workgroup step flags, which count steps across launches
 * (they are never cleared), the cache generation and one cache slot per
 * workgroup; the double-buffered eps / f'(x) W^T eps exchange; and caches tied to
 * the bound buffers (the top chunks' 16-bit images of f(x[L]), the hidden
 * f(x) values and the next launch's first-step partial products), which a
 * launch reuses while their generation is current.  ipc_plan_bind and
 * ipc_plan_sync make them stale, so a rebound plan starts cold.  A workspace
 * belongs to one bound plan at a time: binding another plan to it hands it
 * over, and the first plan must be bound again before it runs again.  The
 * wide path keeps its 16-bit operand copies there (W as hi and lo terms,
 * W^T, f(x) and eps in both layouts, zero padded; their padding must stay
 * zero), then the fp32 partial products of a k-split output-layer
 * prediction. */
long long ipc_plan_workspace_bytes(const ipc_plan* plan);

/* Binds the caller's buffers: x and e hold L+1 pointers ([d_l, B] each; e[L]
 * is unused and may be NULL), w holds L pointers ([d_l, d_{l+1}]), a holds
 * L+1 pointers for save-activation mode (recompute == 0) or is NULL;
 * workspace as above (may be NULL when ipc_plan_workspace_bytes is 0). */
int ipc_plan_bind(ipc_plan* plan, void* const* x, void* const* e, void* const* w, void* const* a,
                  void* workspace);

/* Enqueues `steps` iPC steps on `stream`. */
int ipc_plan_step(ipc_plan* plan, int steps, void* stream);

/* Enqueues the forward initialisation of the bound states: a[L] = f(x[L]) in
 * save mode, hidden x[l] = W[l] f(x[l+1]) for l = L-1..1 (trainer.py:509-515),
 * then (wide path) the refresh of the 16-bit operand copies.
 * x[0] and x[L] are left to the caller; x[L] must be written before. */
int ipc_plan_forward_init(ipc_plan* plan, void* stream);

/* Wide path: re-derives the 16-bit operand copies from the fp32 masters x
 * and W.  Needed only after the caller wrote x[1..L] or W outside
 * ipc_plan_step / ipc_plan_forward_init.  Layer-resident plan: marks the
 * operands it caches between launches stale (the 16-bit copies of f(x[L]),
 * the f(x) of the hidden states, the next launch's first partial products of
 * the top layer): needed after the caller wrote x or W other than through
 * this library's entry points.  A no-op for the other paths. */
int ipc_plan_sync(ipc_plan* plan, void* stream);

/* Enqueues only one phase of the step `reps` times (0 = prediction+error,
 * 1 = inference update, 2 = weight update), so that each phase's kernel can
 * be timed on its own.  Mirrors the per-kernel timing of the reference's
 * harnesses (scripts/autotune.py:200-215).  A fused plan runs prediction and
 * inference in one phase: phase 0 launches both and phase 1 launches nothing. */
#define IPC_PHASE_PRED 0
#define IPC_PHASE_INFER 1
#define IPC_PHASE_WEIGHT 2
int ipc_plan_phase(ipc_plan* plan, int phase, int reps, void* stream);

/* Tile ids of the phased path's three launches (IPC_TILE_AUTO = -1 keeps the
 * automatic choice; the generic tiles 0-2 otherwise).  This is how a tuning
 * table's per-shape kernel configuration reaches a plan, as
 * TileLangIPC._tuned_or_default does for the reference's per-layer kernels
 * (trainer.py:183-216); the whole-step and wide paths run fixed kernels and
 * ignore it.  Valid before or after ipc_plan_bind. */
int ipc_plan_set_tiles(ipc_plan* plan, int tile_pred, int tile_infer, int tile_weight);

/* Tile configurations of the wide path (the tuning surface of
 * IPC_PATH_WIDE plans, the counterpart of the reference's per-shape
 * KernelConfig search, scripts/autotune.py:51-131).  ipc_plan_wide_config_count
 * gives the configurations a phase offers (IPC_PHASE_PRED with split
 * IPC_SPLIT_NONE or IPC_SPLIT_W, IPC_PHASE_INFER, IPC_PHASE_WEIGHT); 0 is the
 * default, and every configuration of a phase gives bit-identical results.
 * ipc_plan_set_wide_config selects one per phase (-1 = default) and the
 * number of k-slices of the output layer's prediction (-1 = chosen at bind
 * from the device's CU count; 1 = none; else a power of two up to 16).  It is
 * called after ipc_plan_create and before ipc_plan_workspace_bytes /
 * ipc_plan_bind (the prediction tile sets the workspace size); a k-split the
 * net cannot take fails at bind with IPC_ERR_CONFIG. */
int ipc_plan_wide_config_count(int phase, int split);
int ipc_plan_set_wide_config(ipc_plan* plan, int pred_cfg, int infer_cfg, int weight_cfg, int ksplit);

/* Row-block size of a layer-resident plan (the tuning surface of
 * IPC_PATH_RESIDENT plans): the top layer W[L-1] is cut into blocks of
 * `rows` rows (16, 32 or 64; -1 = the default 32) times column chunks of 128,
 * one workgroup each; smaller blocks give more, shorter top workgroups.
 * Results are bit-identical for every size (each block adds its chunks'
 * partial products in chunk order).  Called after ipc_plan_create and before
 * ipc_plan_workspace_bytes / ipc_plan_bind (the size sets the workspace);
 * IPC_ERR_CONFIG when the plan is not layer-resident or the net's blocks of
 * that size do not fit the LDS, the flag area or the device's co-resident
 * capacity (the plan is then unchanged).  ipc_plan_resident_rows reports the
 * current size (0 for other plans). */
int ipc_plan_set_resident_rows(ipc_plan* plan, int rows);
int ipc_plan_resident_rows(const ipc_plan* plan);

/* Kernel launches one ipc_plan_step(steps=1) enqueues. */
int ipc_plan_launch_count(const ipc_plan* plan);

/*
 * Health of the whole-step kernels.  Their workgroups wait for each other
 * (grid barriers, per-workgroup step flags), which needs every workgroup of a
 * launch running at once: ipc_plan_create takes the co-resident capacity of
 * the device into account (an AUTO plan falls back from the layer-resident to
 * the column kernel, an explicit IPC_PATH_RESIDENT plan fails with
 * IPC_ERR_CONFIG, the column kernel's grid is capped), but a kernel on
 * another stream or in another process can still hold CUs the launch needs.
 * Every wait is therefore bounded: after `spin limit` polls it gives up, sets
 * word 2 of the workspace (non-zero word 2 = the outputs of the steps since it
 * was last cleared are invalid) and the kernel runs to its end.
 *
 * ipc_plan_check synchronises `stream`, then returns IPC_ERR_TIMEOUT (and
 * clears word 2) if a wait gave up since the last check, IPC_OK otherwise;
 * for plans without a whole-step kernel it only synchronises.  This is
 * TileLangIPC's own addition: the reference's per-layer launches never wait
 * for each other.
 *
 * ipc_plan_set_spin_limit sets the polls per wait (< 0: the default,
 * 4194304 polls of ~64 clocks); 0 gives up at the first unsatisfied poll,
 * which lets a host test force the timeout path while every kernel still
 * exits normally.
 */
int ipc_plan_check(ipc_plan* plan, void* stream);
int ipc_plan_set_spin_limit(ipc_plan* plan, int limit);

/*
 * Captured steps: the native counterpart of IPCGraphRunner
 * (cuda_graph.py:6-36) and of the steady-state graph of
 * TileLangIPC.prepare_steady_state / run_prepared_steady_state
 * (trainer.py:693-781).  ipc_plan_graph_capture records `steps` steps of the
 * bound plan (what ipc_plan_step(plan, steps, ...) enqueues) into a hipGraph
 * on a private stream of default priority and instantiates it; it enqueues
 * no work.  ipc_plan_graph_launch replays it `repeats` times on `stream` (any
 * stream, the null stream included) with one hipGraphLaunch each.  A plan
 * whose `steps` steps are one launch of a whole-step kernel records that
 * launch instead and replays it directly: a one-node graph would run the same
 * kernel with the same arguments, after ~5 us more of graph-launch overhead
 * per replay on MI355X.
 * ipc_plan_bind discards the graph (it holds the previous buffers' addresses);
 * ipc_plan_graph_steps reports the captured step count (0: none).
 */
int ipc_plan_graph_capture(ipc_plan* plan, int steps);
int ipc_plan_graph_launch(ipc_plan* plan, int repeats, void* stream);
int ipc_plan_graph_steps(const ipc_plan* plan);

/*
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Runs `steps` iPC steps of a narrow net
 * on the whole-step kernels exactly as a plan created with IPC_PATH_AUTO,
 * fp32 storage and recompute mode would (ipc_plan_create + ipc_plan_bind +
 * ipc_plan_step: same kernels, same results), without a plan or a caller
 * workspace: the kernels' barrier words, f(x) buffers and exchange records
 * live in the library's static device scratch, 8 MiB per GPU, held until the
 * process ends.  A net that needs more is refused with IPC_ERR_SHAPE; one the
 * whole-step kernels do not take (a width above 128, L above 16, split 2)
 * with IPC_ERR_CONFIG.  x (L+1 pointers), e (L pointers, e[L] unused) and w
 * (L pointers) are laid out as for ipc_plan_bind; the caller does the forward
 * initialisation.  Each call clears the scratch words that must start at
 * zero; calls that overlap on one GPU (other streams or threads) race on the
 * scratch and must be serialised.  A wait that gives up (see ipc_plan_check)
 * sets the scratch's timeout word, which later calls leave set until
 * ipc_noalloc_check reads it.  Calls no hipMalloc, hipFree or other
 * allocating routine.
 */
int ipc_steps_noalloc(int L, const int* dims, int B, void* const* x, void* const* e, void* const* w,
                      int operand, int split, int act, float alpha, float gamma, int weight_mode, int steps,
                      void* stream);

/* Test hook: the host-side check that every LDS-DMA GEMM launch (wide path
 * and standalone 16-bit calls) makes of each of its problems before any HIP
 * call, for one problem of `phase` (IPC_PHASE_PRED, _INFER, _WEIGHT or
 * IPC_PHASE_FORWARD), prediction split `split`, fp32_w != 0 when the kernel
 * splits the fp32 W into its hi and lo operands itself, has_lo != 0 when a
 * 16-bit lo operand is passed, contraction K and k-slices `ksplit`.
 * IPC_ERR_CONFIG when a launch would refuse it: a split-2 kernel without
 * its lo operand (it would read through a null pointer), or a k-split that
 * does not cut K into whole 64-k steps.  No counterpart in the reference. */
#define IPC_PHASE_FORWARD 3
int ipc_wide_problem_check(int phase, int split, int fp32_w, int has_lo, int K, int ksplit);

/* No counterpart in the reference; the health check of ipc_steps_noalloc
 * for callers that cannot allocate.  Synchronises `stream`, then returns
 * IPC_ERR_TIMEOUT (and clears the word) if a wait of any ipc_steps_noalloc
 * call on the current device gave up since the last check: those calls'
 * outputs are invalid.  IPC_OK otherwise.  Allocates nothing. */
int ipc_noalloc_check(void* stream);

/* Test hook: >= 0 sets the polls per wait of ipc_steps_noalloc's kernels
 * (0 gives up at the first unsatisfied poll, so a host test can force the
 * timeout path while every kernel still exits normally); < 0 restores the
 * default.  Not thread-safe. */
int ipc_noalloc_set_spin_limit(int limit);

/* Test hook: > 0 replaces the device's co-resident workgroup capacity in the
 * checks of ipc_plan_create (a compute-partitioned device can be modelled
 * without one); 0 restores the device query.  Not thread-safe. */
int ipc_set_coresident_limit(int blocks);

/*
 * Caller workspace of the standalone 16-bit-storage calls on the LDS-DMA
 * kernel (ipc_pred_err, ipc_forward, ipc_weight_update with recompute,
 * ipc_infer_update).
 * Their B operand f(X_upper) is activated in the loader of every row tile,
 * which for the exponential activations costs more VALU work than the tile's
 * MFMAs once there are many row tiles.  The _ws variants take a device
 * workspace (16-byte aligned, owned by the caller, `workspace_bytes` long):
 * when it holds ipc_s16_workspace_bytes(...) bytes (> 0) the call activates
 * f(X_upper) once into it, in its own launch on `stream`, and the GEMM then
 * reads it like its other operands; otherwise (NULL or too small) the
 * loader path runs.  Same bits either way.  Calls that share a workspace must
 * be ordered on one stream.  The variants without _ws are the _ws calls with
 * no workspace.  No counterpart in the reference (TileLang fuses the
 * activation into its loader and has no workspace); the library allocates
 * nothing on either path.
 *
 * ipc_s16_workspace_bytes gives the bytes a call of `kind` (IPC_PHASE_PRED
 * for ipc_pred_err_ws / ipc_forward_ws, IPC_PHASE_WEIGHT for a recomputing
 * ipc_weight_update_ws, IPC_PHASE_INFER for ipc_infer_update_ws) with M rows,
 * contraction K, batch B and `groups` groups uses: groups * K * B * 2 when it
 * pre-activates under the current mode (groups * (M * K + K * B) * 2 for the
 * inference update, which copies W_lower and E_lower transposed into the
 * workspace so that its GEMM reads both operands k-contiguous), else 0.  The
 * automatic rule: exp-based activations from M >= 1024 and K * B >= 2^20,
 * relu from M >= 4096 and K * B >= 2^22, never identity; the inference
 * update from M * K >= 2^26 and K * B >= 2^26.  ipc_s16_preactivates(kind,
 * act, M, K, B) reports the same decision (1 / 0).  ipc_set_s16_preactivate,
 * a tuning hook, sets the mode: -1 (default) the rule, 0 never, 1 whenever a
 * workspace is given.  Not thread-safe.
 */
int ipc_pred_err_ws(const void* x_upper, const void* w, const void* x_lower, void* e,
                    int M, int K, int B, int groups,
                    int storage, int operand, int split, int act, int tile,
                    void* workspace, long long workspace_bytes, void* stream);
int ipc_forward_ws(const void* x_upper, const void* w, void* out,
                   int M, int K, int B, int groups,
                   int storage, int operand, int split, int act, int tile,
                   void* workspace, long long workspace_bytes, void* stream);
int ipc_weight_update_ws(void* w, const void* e, const void* x_upper, int M, int K, int B, int groups,
                         float alpha, int recompute, int storage, int operand, int act, int tile,
                         void* workspace, long long workspace_bytes, void* stream);
int ipc_infer_update_ws(void* x, const void* e, const void* w_lower, const void* e_lower, void* a_out,
                        int M, int K, int B, int groups, float gamma,
                        int storage, int operand, int act, int tile,
                        void* workspace, long long workspace_bytes, void* stream);
long long ipc_s16_workspace_bytes(int kind, int act, int M, int K, int B, int groups);
int ipc_set_s16_preactivate(int mode);
int ipc_s16_preactivates(int kind, int act, int M, int K, int B);

void ipc_plan_destroy(ipc_plan* plan);

#ifdef __cplusplus
}
#endif

#endif /* IPC_HIP_H */
