"""iPC trainer on MI355X: the drop-in for ``src/ipc_tilelang/trainer.py``.

``IPCConfig`` keeps the reference's fields (``trainer.py:28-53``) and adds
``master_dtype`` and ``init``.  ``HipIPC`` (also exported as ``TileLangIPC``)
keeps the reference's public methods (``trainer.py:56-833``): buffers are
allocated once per batch shape, the hidden states are initialised by a
forward prediction, and one step runs the three phases

    P: eps[l] = x[l] - W[l] f(x[l+1])                      l = 0..L-1
    I: x[l] += gamma(-eps[l] + f'(x[l]) W[l-1]^T eps[l-1])   l = 1..L-1
    W: W[l] += alpha eps[l] f(x_new[l+1])^T                  l = 0..L-1

The per-layer Python launch loop of ``step_initialized`` (``:601-679``) is
replaced by one call into the library's whole-step plan, which enqueues one
ragged multi-layer kernel per phase on torch's current stream (so it can be
captured by ``torch.cuda.graph``, i.e. a hipGraph).

Precision: ``dtype`` is the GEMM operand type (the reference's fp16 default
is kept); x, eps and W are stored in ``master_dtype`` (fp32 by default).  With
16-bit storage of everything the reference's design cannot meet a 5e-3 bound
on weight deltas at alpha=1e-4 (one fp16 ulp of W is about the size of a
per-step delta), so 16-bit storage is available only by setting
``master_dtype`` explicitly.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

import torch

from . import _native as nat
from .gridz_tuning import lookup_grid_z_cap
from .hierarchical_policy import kernel_signature, load_hierarchical_policy
from .kernels import KernelConfig, build_forward
from .layer_batching import find_internal_square_groups
from .tuning import config_to_dict


@dataclass(frozen=True)
class IPCConfig:
    dims: tuple[int, ...]
    alpha: float = 1e-4
    gamma: float = 0.5
    activation: str = "relu"
    dtype: torch.dtype = torch.float16
    kernel: KernelConfig = field(default_factory=KernelConfig)
    recompute_activation: bool = True
    # A lich_amd.tuning.TuningTable, consulted after the hierarchical policy
    # (precedence of trainer.py:183-216); its configs pick the phased path's tiles.
    tuning_table: object | None = None
    # The reference's grid.z layer batching knobs (trainer.py:38-41): the cap
    # comes from the hierarchical policy, else from the grid.z policy file
    # (gridz_tuning.py:50-73), else grid_z_max_layers, and is recorded in
    # ``grid_z_cap`` / ``layer_groups``; it changes no launch here, since every
    # phase is already one multi-layer launch.  The hierarchical policy file,
    # when present, also selects recompute and graph use per net.
    use_grid_z: bool = True
    grid_z_max_layers: int = 2
    grid_z_auto: bool = True
    grid_z_policy_path: str = "results/gridz_policy.json"
    hierarchical_policy_auto: bool = True
    hierarchical_policy_path: str = "results/hierarchical_policy.json"
    steady_state_graph_auto: bool = True
    steady_state_graph_default: bool = False
    weight_update_mode: str = "gemm"
    weight_update_policy_path: str = "results/weight_update_policy.json"
    weight_update_outer_max_batch: int = 16
    # additions
    master_dtype: torch.dtype = torch.float32
    init: str = "kaiming_a_sqrt5"
    # Prediction-phase operand split for 16-bit operands over fp32 master
    # data: 1 plain, 2 = W as hi + lo terms, 3 = W and f(x) both split.  None
    # picks, for narrow nets (every output width <= 128, L <= 16: the
    # whole-step kernels), 1 with fp16 operands and tanh or sigmoid (their
    # rounding alone stays 6x or more inside the bars, and the split costs ~6 %
    # of the step), 3 with bf16 (split 1 misses the 5e-3 weight-delta bar on
    # some seeds) or relu, silu, gelu (f' steps or crosses zero: unsplit
    # operands reach 0.5x the bar or beyond); 2 otherwise (the MFMA-bound
    # wide path).
    pred_split: int | None = None
    # Wide path tile configuration (pred, infer, weight, ksplit), -1 = default
    # (ipc_plan_set_wide_config); a policy file's tuned choice takes precedence.
    wide_config: tuple[int, int, int, int] | None = None
    # Layer-resident plans: rows of the top layer per workgroup (16, 32 or
    # 64; None = the library's default, 32) (ipc_plan_set_resident_rows); a
    # policy file's tuned choice takes precedence.
    resident_rows: int | None = None
    # Kernel path: "auto" (the layer-resident whole-step kernel when eligible,
    # else the column-block whole-step kernel for narrow nets, else the wide
    # GEMM path when eligible, else phased), "resident", "narrow" / "on",
    # "wide", "phased" / "off".
    fused: str = "auto"


def init_weights_cpu(dims: Sequence[int], *, seed: int, init: str) -> list[torch.Tensor]:
    """Seeded fp32 weights drawn on the CPU in layer order.

    ``kaiming_a_sqrt5`` is the reference's ``kaiming_uniform_(a=sqrt(5))``
    (``trainer.py:97-108``), ``xavier_uniform`` the paper-profile init.  The
    reference drew from a device generator; a CPU generator makes the initial
    weights identical on every machine, which parity checks rely on.
    """
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    out = []
    for n_l, n_u in zip(dims[:-1], dims[1:]):
        w = torch.empty((int(n_l), int(n_u)), dtype=torch.float32)
        if init == "kaiming_a_sqrt5":
            torch.nn.init.kaiming_uniform_(w, a=5 ** 0.5, generator=g)
        elif init == "xavier_uniform":
            torch.nn.init.xavier_uniform_(w, generator=g)
        else:
            raise ValueError(f"Unknown init {init!r}")
        out.append(w)
    return out


def _ptr_array(tensors) -> ctypes.Array:
    arr = (ctypes.c_void_p * len(tensors))()
    for i, t in enumerate(tensors):
        arr[i] = None if t is None else t.data_ptr()
    return arr


class HipIPC:
    """iPC model whose step runs entirely in ``libipc_hip.so`` (gfx950)."""

    def __init__(self, cfg: IPCConfig, *, device, seed: int = 0, weights: Sequence[torch.Tensor] | None = None):
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("HipIPC requires a GPU device")
        index = device.index if device.index is not None else torch.cuda.current_device()
        self.device = torch.device("cuda", index)
        try:
            self.arch = nat.device_arch(index)
        except nat.IPCNativeError as exc:
            raise ValueError(str(exc)) from exc
        if len(cfg.dims) < 2:
            raise ValueError("dims needs at least two entries")
        self.cfg = cfg
        self.act_name = str(cfg.activation).lower()
        self._act = nat.act_code(self.act_name)
        self.storage_dtype = cfg.master_dtype
        self.operand_dtype = cfg.dtype
        self._storage = nat.dtype_code(self.storage_dtype)
        self._operand = nat.dtype_code(self.operand_dtype)
        if self._storage != nat.DT_F32 and self._operand != self._storage:
            raise ValueError("16-bit master_dtype requires dtype == master_dtype")
        if cfg.pred_split is not None:
            self.pred_split = int(cfg.pred_split)
        elif self._storage == nat.DT_F32 and self._operand != nat.DT_F32:
            narrow = len(cfg.dims) - 1 <= 16 and max(int(d) for d in cfg.dims[:-1]) <= 128
            if narrow:
                # fp16 operands need no split with a monotone smooth activation; relu's
                # step and the zero crossings of silu's and gelu's f' make operand
                # rounding flip or swing derivatives, so those keep split 3
                monotone = self.act_name in ("tanh", "sigmoid")
                self.pred_split = 1 if self._operand == nat.DT_F16 and monotone else 3
            else:
                self.pred_split = 2
        else:
            self.pred_split = 1
        mode = str(cfg.weight_update_mode).lower()
        if mode not in nat.WMODE:
            raise ValueError(f"Unknown weight_update_mode {cfg.weight_update_mode!r}")
        self._wmode = nat.WMODE[mode]
        if str(cfg.fused).lower() not in nat.FUSED:
            raise ValueError(f"Unknown fused option {cfg.fused!r}")
        self._fused = nat.FUSED[str(cfg.fused).lower()]
        self._workspace: torch.Tensor | None = None
        if weights is None:
            weights = init_weights_cpu(cfg.dims, seed=seed, init=cfg.init)
        if len(weights) != len(cfg.dims) - 1:
            raise ValueError("one weight matrix per edge is required")
        self.w: list[torch.Tensor] = []
        for l, wl in enumerate(weights):
            if tuple(wl.shape) != (int(cfg.dims[l]), int(cfg.dims[l + 1])):
                raise ValueError(f"W[{l}] has shape {tuple(wl.shape)}")
            self.w.append(wl.detach().to(device=self.device, dtype=self.storage_dtype).contiguous())
        self.x: list[torch.Tensor] | None = None
        self.e: list[torch.Tensor] | None = None
        self.a: list[torch.Tensor | None] | None = None
        self._plan = None
        self._plan_key = None
        self._caches_operands = False  # the bound plan keeps operand copies or caches between launches
        self._synced_versions = None   # torch version counters of x[1..L] and W when last in sync
        self._steady_state_runner = None
        self._steady_state_graph_steps: int | None = None
        self._steady_state_graph_key = None
        self._hierarchical_policy = None
        if cfg.hierarchical_policy_auto:
            try:
                self._hierarchical_policy = load_hierarchical_policy(cfg.hierarchical_policy_path)
            except (OSError, ValueError):
                self._hierarchical_policy = None
        self._runtime_recompute: bool = bool(cfg.recompute_activation)
        self.wide_config = cfg.wide_config
        self.resident_rows = cfg.resident_rows
        self.grid_z_cap: int = max(0, int(cfg.grid_z_max_layers))
        self.layer_groups = self._groups_for(self.grid_z_cap)
        self._signature_cache: dict[int, str] = {}

    # ------------------------------------------------------------------ tuning artefacts
    def _tuned_or_default(self, kind: str, M: int, K: int, B: int) -> KernelConfig:
        """Kernel configuration for one (kind, shape): the policy's per-net
        profile, then its global entries, then the tuning table, then
        ``cfg.kernel`` (reference ``trainer.py:183-216``)."""
        dt = str(self.cfg.dtype).split(".")[-1]
        pol = self._hierarchical_policy
        if pol is not None:
            tuned = pol.lookup_profile_kernel(dims=tuple(int(d) for d in self.cfg.dims), batch=int(B), kind=kind,
                                              M=M, K=K, activation=self.cfg.activation, dtype=dt)
            if tuned is None:
                tuned = pol.lookup_kernel(kind=kind, M=M, K=K, B=B, activation=self.cfg.activation, dtype=dt)
            if tuned is not None:
                return tuned
        table = self.cfg.tuning_table
        if table is not None:
            tuned = table.lookup(kind=kind, M=M, K=K, B=B, activation=self.cfg.activation, dtype=dt)
            if tuned is not None:
                return tuned
        return self.cfg.kernel

    def _kernel_rows(self, B: int) -> list[dict]:
        rows, seen = [], set()
        dt = str(self.cfg.dtype).split(".")[-1]
        for l in range(self.L):
            shapes = [("prediction", self.cfg.dims[l], self.cfg.dims[l + 1]),
                      ("weight", self.cfg.dims[l], self.cfg.dims[l + 1])]
            if l > 0:
                shapes.append(("inference", self.cfg.dims[l], self.cfg.dims[l - 1]))
            for kind, M, K in shapes:
                if (kind, M, K) in seen:
                    continue
                seen.add((kind, M, K))
                rows.append({"kind": kind, "shape": {"M": int(M), "K": int(K), "B": int(B)},
                             "activation": self.cfg.activation, "dtype": dt,
                             "config": config_to_dict(self._tuned_or_default(kind, int(M), int(K), int(B)))})
        return rows

    def _active_kernel_signature(self, B: int) -> str:
        """Fingerprint of the kernel table in use (reference ``trainer.py:218-246``)."""
        B = int(B)
        if B not in self._signature_cache:
            self._signature_cache[B] = kernel_signature(self._kernel_rows(B))
        return self._signature_cache[B]

    def _policy_kw(self, B: int) -> dict:
        return dict(dims=tuple(int(d) for d in self.cfg.dims), batch=int(B), activation=self.cfg.activation,
                    dtype=str(self.cfg.dtype).split(".")[-1], kernel_sig=self._active_kernel_signature(B))

    def _groups_for(self, cap: int):
        if not self.cfg.use_grid_z or cap < 2:
            return ()
        return find_internal_square_groups(tuple(int(d) for d in self.cfg.dims), max_group_count=cap)

    def _apply_execution_policy(self, B: int) -> None:
        """Recompute and grid.z choices for this net and batch (reference
        ``trainer.py:158-177`` and ``:273-300``): the hierarchical policy
        first, then for grid.z the grid.z policy file keyed by this device."""
        self._runtime_recompute = bool(self.cfg.recompute_activation)
        self.wide_config = self.cfg.wide_config
        self.resident_rows = self.cfg.resident_rows
        cap = None
        pol = self._hierarchical_policy
        if pol is not None:
            kw = self._policy_kw(B)
            self._runtime_recompute = pol.selected_recompute_activation(default=self._runtime_recompute, **kw)
            self.wide_config = pol.selected_wide_config(default=self.wide_config, **kw)
            self.resident_rows = pol.selected_resident_rows(default=self.resident_rows, **kw)
            if self.cfg.use_grid_z and self.cfg.grid_z_auto:
                cap = pol.selected_grid_z(default=None, **kw)
        if cap is None and self.cfg.use_grid_z and self.cfg.grid_z_auto:
            cap = lookup_grid_z_cap(self.cfg.grid_z_policy_path, device_name=torch.cuda.get_device_name(self.device),
                                    capability=torch.cuda.get_device_capability(self.device), dims=self.cfg.dims,
                                    batch=B, activation=self.cfg.activation, dtype=self.cfg.dtype,
                                    default=int(self.cfg.grid_z_max_layers))
        self.grid_z_cap = max(0, int(self.cfg.grid_z_max_layers if cap is None else cap))
        self.layer_groups = self._groups_for(self.grid_z_cap)

    def phase_tiles(self, B: int) -> tuple[int, int, int]:
        """Tile ids of the phased path's launches: the tuned configuration of
        each phase's largest layer (-1: automatic)."""
        dims = [int(d) for d in self.cfg.dims]
        out = []
        for kind, layers in (("prediction", range(self.L)), ("inference", range(1, self.L)),
                             ("weight", range(self.L))):
            best = None
            for l in layers:
                M, K = (dims[l], dims[l - 1]) if kind == "inference" else (dims[l], dims[l + 1])
                if best is None or M * K > best[0] * best[1]:
                    best = (M, K)
            t = nat.TILE_AUTO if best is None else self._tuned_or_default(kind, best[0], best[1], B).tile_id()
            out.append(t if t in (0, 1, 2) else nat.TILE_AUTO)
        return tuple(out)

    # ------------------------------------------------------------------ plan
    @property
    def L(self) -> int:
        return len(self.w)

    @property
    def recompute_activation(self) -> bool:
        return bool(self._runtime_recompute)

    def __del__(self):
        self._destroy_plan()

    def _destroy_plan(self) -> None:
        plan = getattr(self, "_plan", None)
        if plan is not None:
            try:
                nat.lib().ipc_plan_destroy(plan)
            except Exception:
                pass
            self._plan = None
            self._plan_key = None

    def _build_plan(self, B: int) -> None:
        self._destroy_plan()
        dims = (ctypes.c_int * len(self.cfg.dims))(*[int(d) for d in self.cfg.dims])
        handle = ctypes.c_void_p()
        nat.check(nat.lib().ipc_plan_create(
            ctypes.byref(handle), self.L, dims, int(B), self._storage, self._operand, self.pred_split, self._act,
            float(self.cfg.alpha), float(self.cfg.gamma), int(self.recompute_activation), self._wmode,
            self._fused))
        self._plan = handle
        nat.check(nat.lib().ipc_plan_set_tiles(handle, *self.phase_tiles(B)))
        if self.wide_config is not None and int(nat.lib().ipc_plan_path(handle)) == nat.PATH_WIDE:
            nat.check(nat.lib().ipc_plan_set_wide_config(handle, *[int(v) for v in self.wide_config]))
        if self.resident_rows is not None and int(nat.lib().ipc_plan_path(handle)) == nat.PATH_RESIDENT:
            nat.check(nat.lib().ipc_plan_set_resident_rows(handle, int(self.resident_rows)))
        nbytes = int(nat.lib().ipc_plan_workspace_bytes(handle))
        # zero-initialised (the wide path relies on zero padding); torch's
        # allocations are 256-byte aligned as the plan requires
        self._workspace = (torch.zeros(((nbytes + 3) // 4,), dtype=torch.int32, device=self.device)
                           if nbytes else None)
        a = None if self.a is None else _ptr_array(self.a)
        ws = None if self._workspace is None else self._workspace.data_ptr()
        nat.check(nat.lib().ipc_plan_bind(handle, _ptr_array(self.x), _ptr_array(self.e), _ptr_array(self.w), a, ws))
        self._plan_key = (int(B), tuple(t.data_ptr() for t in self.w))
        self._caches_operands = self.path in ("resident", "wide")
        self._synced_versions = None

    def runtime_plan_ready(self) -> bool:
        return self._plan is not None

    def launches_per_step(self) -> int:
        return int(nat.lib().ipc_plan_launch_count(self._plan)) if self._plan is not None else 0

    @property
    def fused(self) -> bool:
        """True when the step runs as the whole-step kernel."""
        return self._plan is not None and bool(nat.lib().ipc_plan_fused(self._plan))

    @property
    def path(self) -> str | None:
        """Kernel path of the bound plan: "resident" (layer-resident whole-step
        kernel), "narrow" (column-block whole-step kernel), "wide" (LDS-DMA
        MFMA phases over 16-bit operand copies) or "phased"."""
        if self._plan is None:
            return None
        return nat.PATH_NAMES[int(nat.lib().ipc_plan_path(self._plan))]

    def sync_operand_copies(self) -> None:
        """Declare writes of ``x`` or ``w`` made outside a step: re-derives the
        wide path's 16-bit operand copies, marks the operands the
        layer-resident path caches between launches stale (f(x[L]) copies,
        f(x) of the hidden states, the top layer's next first-step partial
        products); a no-op for the other paths.

        Writes through torch (``copy_``, in-place ops, views of ``x[l]`` or
        ``w[l]``) are detected by their version counters before the next
        launch and need no call; writes torch does not count (through
        ``.data``, ``data_ptr()`` or another library) do."""
        if self._plan is not None:
            nat.check(nat.lib().ipc_plan_sync(self._plan, nat.current_stream_handle(self.device)))
            self._mark_synced()

    def _tracked_versions(self) -> tuple:
        # x[0] (the target) is read directly by every launch and never cached
        return tuple(t._version for t in self.x[1:]) + tuple(t._version for t in self.w)

    def _mark_synced(self) -> None:
        if self._caches_operands and self.x is not None:
            self._synced_versions = self._tracked_versions()

    def _sync_if_written(self) -> None:
        """The reference re-reads x and W at every launch (trainer.py:601-679),
        so a caller may write them in place between steps (trainer.py:798-817).
        The resident and wide paths keep copies and caches of them between
        launches: if torch has counted a write to x[1..L] or W since the
        library last made them consistent, re-sync before launching."""
        if self._caches_operands and self._tracked_versions() != self._synced_versions:
            self.sync_operand_copies()

    def barrier_timeouts(self) -> int:
        """Non-zero if a wait of a whole-step kernel hit its spin limit since
        the last ``check_steps`` (synchronises the device, clears nothing)."""
        if self._workspace is None:
            return 0
        return int(self._workspace[2].item())

    def check_steps(self) -> None:
        """Synchronise and raise ``RuntimeError`` if a wait of a whole-step
        kernel gave up since the last check: those steps' states and weights
        are invalid (their workgroups were not all running at once).  Every
        synchronising call of this class runs it."""
        if self._plan is not None:
            nat.check(nat.lib().ipc_plan_check(self._plan, nat.current_stream_handle(self.device)))

    def set_spin_limit(self, limit: int | None) -> None:
        """Polls per wait of the whole-step kernels (None: the default)."""
        if self._plan is None:
            raise RuntimeError("Call initialize_batch first")
        nat.check(nat.lib().ipc_plan_set_spin_limit(self._plan, -1 if limit is None else int(limit)))

    # ------------------------------------------------------------------ batch
    def initialize_batch(self, x_input: torch.Tensor, y_target: torch.Tensor) -> None:
        """Reset the endpoints and initialise hidden states by a forward
        prediction (reference ``trainer.py:453-516``)."""
        if x_input.ndim != 2 or y_target.ndim != 2:
            raise ValueError("Inputs must be [features, batch]")
        B = int(x_input.shape[1])
        if x_input.shape[0] != self.cfg.dims[-1] or y_target.shape[0] != self.cfg.dims[0]:
            raise ValueError("Batch dimensions do not match network dims")
        if y_target.shape[1] != B:
            raise ValueError("input and target batch sizes differ")
        if self.x is None or self.x[0].shape[1] != B:
            self._invalidate_steady_state_graph()
            self._destroy_plan()
            self._apply_execution_policy(B)
            kw = dict(device=self.device, dtype=self.storage_dtype)
            self.x = [torch.empty((int(d), B), **kw) for d in self.cfg.dims]
            self.e = [torch.empty((int(d), B), **kw) for d in self.cfg.dims]
            self.a = None if self.recompute_activation else [torch.empty((int(d), B), **kw) for d in self.cfg.dims]
        if self._plan is None:
            self._build_plan(B)
        self.x[-1].copy_(x_input)
        # the forward initialisation re-derives every cached operand (wide
        # copies of W and f(x); a column-kernel launch makes the resident caches stale)
        nat.check(nat.lib().ipc_plan_forward_init(self._plan, nat.current_stream_handle(self.device)))
        self.x[0].copy_(y_target)
        self._mark_synced()

    # ------------------------------------------------------------------ step
    @torch.no_grad()
    def step_initialized(self, *, collect_metrics: bool = False) -> dict[str, float]:
        if self.x is None or self._plan is None:
            raise RuntimeError("Call initialize_batch before step_initialized")
        self._sync_if_written()
        nat.check(nat.lib().ipc_plan_step(self._plan, 1, nat.current_stream_handle(self.device)))
        if collect_metrics:
            return self.metrics()
        return {}

    def metrics(self) -> dict[str, float]:
        """``max_abs_error`` over eps[0..L-1] of the last step (device reduction, one sync)."""
        assert self.e is not None
        self.check_steps()
        return {"max_abs_error": float(torch.stack([v.abs().max().float() for v in self.e[:-1]]).max().item())}

    @torch.no_grad()
    def step(self, x_input: torch.Tensor, y_target: torch.Tensor) -> dict[str, float]:
        self.initialize_batch(x_input, y_target)
        return self.step_initialized(collect_metrics=True)

    def run_steps(self, steps: int) -> None:
        """Enqueue ``steps`` steps with one library call (no Python loop)."""
        if self._plan is None:
            raise RuntimeError("Call initialize_batch first")
        self._sync_if_written()
        nat.check(nat.lib().ipc_plan_step(self._plan, int(steps), nat.current_stream_handle(self.device)))

    # ------------------------------------------------------------------ steady state / graph
    def recommended_use_cuda_graph(self, batch: int | None = None, *, default: bool = True) -> bool:
        """The policy's graph choice for this net and batch, else ``default``
        (reference ``trainer.py:248-262``)."""
        pol = self._hierarchical_policy
        if pol is None:
            return bool(default)
        if batch is None:
            if self.x is None:
                return bool(default)
            batch = int(self.x[0].shape[1])
        return pol.selected_use_graph(default=bool(default), **self._policy_kw(int(batch)))

    def _invalidate_steady_state_graph(self) -> None:
        self._steady_state_runner = None
        self._steady_state_graph_key = None
        self._steady_state_graph_steps = None

    def steady_state_graph_ready(self, steps: int) -> bool:
        return (self._steady_state_runner is not None and self._steady_state_graph_steps == int(steps)
                and self._steady_state_graph_key == self._plan_key)

    def prepare_steady_state(self, x_input, y_target, *, steps: int = 1, use_graph: bool | None = None) -> bool:
        """Prepare one fixed-shape batch for repeated execution; True when the
        graph path is active (reference ``trainer.py:693-724``)."""
        steps = max(1, int(steps))
        self.initialize_batch(x_input, y_target)
        if use_graph is None:
            use_graph = (self.recommended_use_cuda_graph(default=bool(self.cfg.steady_state_graph_default))
                         if self.cfg.steady_state_graph_auto else bool(self.cfg.steady_state_graph_default))
        if not use_graph:
            return False
        if not self.steady_state_graph_ready(steps):
            self._steady_state_runner = self.capture_graph(steps)
            self._steady_state_graph_steps = steps
            self._steady_state_graph_key = self._plan_key
        return True

    @torch.no_grad()
    def run_prepared_steady_state(self, *, steps: int | None = None, repeats: int = 1,
                                  use_graph: bool | None = None, collect_metrics: bool = False) -> dict[str, float]:
        if self.x is None or self._plan is None:
            raise RuntimeError("Call prepare_steady_state/initialize_batch first")
        steps = max(1, int(self._steady_state_graph_steps if steps is None and self._steady_state_graph_steps
                           else (steps or 1)))
        repeats = max(1, int(repeats))
        if use_graph is None:
            use_graph = self.steady_state_graph_ready(steps)
        if use_graph:
            if not self.steady_state_graph_ready(steps):
                raise RuntimeError("Requested graph replay without a matching captured graph")
            self._steady_state_runner.replay(repeats)
        else:
            self.run_steps(steps * repeats)
        torch.cuda.synchronize(self.device)
        if collect_metrics:
            return self.metrics()
        self.check_steps()
        return {}

    def reset_steady_state(self) -> None:
        self._invalidate_steady_state_graph()

    @property
    def steady_state_uses_graph(self) -> bool:
        return self._steady_state_runner is not None

    def run_steady_state_batch(self, x_input, y_target, *, steps: int = 1, repeats: int = 1,
                               use_graph: bool | None = None, collect_metrics: bool = False) -> dict[str, float]:
        self.prepare_steady_state(x_input, y_target, steps=steps, use_graph=use_graph)
        return self.run_prepared_steady_state(steps=steps, repeats=repeats, use_graph=use_graph,
                                              collect_metrics=collect_metrics)

    def precompile(self) -> None:
        """Run one step and restore every buffer, so that each kernel's code
        object is resident before graph capture (reference ``trainer.py:783-818``)."""
        if self.x is None or self._plan is None:
            raise RuntimeError("Call initialize_batch before precompile")
        backup = [[t.clone() for t in ts] for ts in (self.w, self.x, self.e)]
        a_backup = None if self.a is None else [t.clone() for t in self.a]
        # the workspace holds the wide path's 16-bit operand copies
        ws_backup = None if self._workspace is None else self._workspace.clone()
        self.step_initialized(collect_metrics=False)
        self.check_steps()
        for dst_list, src_list in zip((self.w, self.x, self.e), backup):
            for dst, src in zip(dst_list, src_list):
                dst.copy_(src)
        if a_backup is not None:
            for dst, src in zip(self.a, a_backup):
                dst.copy_(src)
        if ws_backup is not None:
            self._workspace.copy_(ws_backup)
        self._mark_synced()  # the workspace's copies and caches are restored with the buffers
        torch.cuda.synchronize(self.device)

    def capture_graph(self, steps: int):
        if self.x is None:
            raise RuntimeError("Call initialize_batch before capture_graph")
        from .hip_graph import IPCGraphRunner
        runner = IPCGraphRunner(self, steps)
        runner.capture()
        return runner

    # ------------------------------------------------------------------ inference
    @torch.no_grad()
    def predict(self, x_input: torch.Tensor) -> torch.Tensor:
        """Forward pass ``h = W[l] f(h)`` from the input down (reference ``trainer.py:828-833``)."""
        h = x_input.to(device=self.device, dtype=self.storage_dtype).contiguous()
        B = int(h.shape[1])
        for l in reversed(range(self.L)):
            M, K = int(self.cfg.dims[l]), int(self.cfg.dims[l + 1])
            out = torch.empty((M, B), device=self.device, dtype=self.storage_dtype)
            build_forward(M, K, B, self.act_name, self.storage_dtype, None,
                          operand_dtype=self.operand_dtype, split=self.pred_split)(h, self.w[l], out)
            h = out
        return h


TileLangIPC = HipIPC


def prepare_batch(images: torch.Tensor, labels: torch.Tensor, *, device, dtype=torch.float32,
                  num_classes: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``[features, B]`` input and ``[classes, B]`` one-hot target on the device
    (reference ``trainer.py:836-846``)."""
    x = images.flatten(1).T.contiguous().to(device=device, dtype=dtype, non_blocking=True)
    y = torch.nn.functional.one_hot(labels.to(device, non_blocking=True).long(), num_classes=num_classes)
    return x, y.to(dtype=dtype).T.contiguous()
