"""Operator API of the three iPC kernel families (HIP, gfx950).

Mirrors the reference's builders in ``src/ipc_tilelang/tilelang_kernels.py``:
``build_prediction_error`` (``:114-177``), ``build_inference_update``
(``:180-265``) and ``build_weight_update`` (``:268-349``).  Each builder
returns a callable with the reference's call signature and in-place
semantics; the callable validates its tensors (as TileLang's adapter did) and
enqueues one launch of ``libipc_hip.so`` on torch's current stream.

Differences from the reference, all deliberate:

* ``dtype`` is the storage type of the tensors the callable accepts
  (float32, float16 or bfloat16).  ``operand_dtype`` (new, default = storage)
  selects the type the GEMM operands are rounded to; fp32 storage with
  fp16/bf16 operands is the precision design of the trainer.
* ``gamma`` and ``alpha`` are runtime scalars, not compile-time constants, so
  one code object serves every value.
* ``KernelConfig`` names a CDNA4 tile configuration (``tile``); the reference
  fields are accepted for call compatibility and only steer the tile choice.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import torch

from . import _native as nat

_STORAGE = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


@dataclass(frozen=True)
class KernelConfig:
    """Tile configuration (reference ``tilelang_kernels.py:8-17``).

    ``tile`` selects one of the CDNA4 MFMA tile shapes of the library
    (generic kernel 0: 32x32, 1: 64x64, 2: 128x128; LDS-DMA kernel for 16-bit
    storage 3: 256x128, 4: 128x256, 5: 128x128, 6: 256x256; -1: chosen from
    the problem shape).  When
    ``tile`` is None the reference's ``block_m``/``block_n`` pick the closest
    shape; with neither given the choice is automatic.
    """

    block_m: int | None = None
    block_n: int | None = None
    block_k: int | None = None
    threads: int | None = None
    num_stages: int | None = None
    swizzle: bool = True
    swizzle_panel: int = 8
    shared_swizzle: bool = False
    tile: int | None = None

    def tile_id(self) -> int:
        if self.tile is not None:
            t = int(self.tile)
            if t < -1 or t >= nat.TILE_COUNT:
                raise ValueError(f"unknown tile id {t}")
            return t
        if self.block_m is None and self.block_n is None:
            return nat.TILE_AUTO
        side = min(int(self.block_m or 128), int(self.block_n or 128))
        return 2 if side >= 128 else (1 if side >= 64 else 0)


def _storage_dtype(dtype) -> torch.dtype:
    if isinstance(dtype, torch.dtype):
        return dtype
    try:
        return _STORAGE[str(dtype).split(".")[-1]]
    except KeyError as exc:
        raise ValueError(f"Unsupported dtype {dtype!r}") from exc


def _check(t: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, kernel expects {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, kernel expects {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class _Kernel:
    """Common state of a built kernel callable."""

    def __init__(self, kind: str, M: int, K: int, B: int, activation: str, dtype, cfg, operand_dtype,
                 groups: int = 1, split: int = 1):
        self.kind = kind
        self.M, self.K, self.B = int(M), int(K), int(B)
        self.groups = int(groups)
        if min(self.M, self.K, self.B, self.groups) < 1:
            raise ValueError(f"invalid shape M={M} K={K} B={B} groups={groups}")
        self.activation = str(activation).lower()
        self.act = nat.act_code(self.activation)
        self.dtype = _storage_dtype(dtype)
        self.storage = nat.dtype_code(self.dtype)
        self.operand = nat.dtype_code(_storage_dtype(operand_dtype) if operand_dtype is not None else self.dtype)
        if self.storage != nat.DT_F32 and self.operand != self.storage:
            raise ValueError("16-bit storage requires operand_dtype == dtype")
        self.cfg = cfg if cfg is not None else KernelConfig()
        self.tile = self.cfg.tile_id()
        if int(split) not in (1, 2, 3):
            raise ValueError(f"split must be 1, 2 or 3 (got {split})")
        self.split = int(split)

    def _shape(self, *dims):
        return (self.groups, *dims) if self.groups > 1 else tuple(dims)

    # kind code of ipc_s16_workspace_bytes (IPC_PHASE_*): -1 = never uses a workspace
    _ws_kind = -1

    @property
    def workspace_bytes(self) -> int:
        """Bytes of caller workspace that let a call evaluate f(X_upper) once
        instead of in every row tile's loader, or, for the inference update,
        copy its operands transposed (0: the call never uses one).
        Only 16-bit storage on the LDS-DMA kernel uses it; the library itself
        allocates nothing."""
        if self._ws_kind < 0 or self.storage == nat.DT_F32:
            return 0
        return int(nat.lib().ipc_s16_workspace_bytes(self._ws_kind, self.act, self.M, self.K, self.B, self.groups))

    def new_workspace(self, device=None) -> torch.Tensor | None:
        """A caller-owned workspace of ``workspace_bytes`` (None when the call
        uses none), to be passed as ``workspace=`` to calls on one stream."""
        n = self.workspace_bytes
        if n <= 0:
            return None
        return torch.empty(((n + 15) // 16 * 16,), dtype=torch.uint8, device=device or torch.device("cuda"))

    @staticmethod
    def _ws(workspace):
        if workspace is None:
            return None, 0
        if not isinstance(workspace, torch.Tensor) or workspace.device.type != "cuda" or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous device tensor")
        return workspace.data_ptr(), workspace.numel() * workspace.element_size()


class PredictionErrorKernel(_Kernel):
    """``k(X_upper[K,B], W[M,K], X_lower[M,B], E[M,B], *, workspace=None)``:
    ``E = X_lower - W f(X_upper)``.  ``workspace`` (optional, caller-owned,
    ``new_workspace()``) lets a large 16-bit call activate f(X_upper) once."""

    _ws_kind = 0

    def __call__(self, x_upper, w, x_lower, e, *, workspace=None):
        M, K, B, dt = self.M, self.K, self.B, self.dtype
        _check(x_upper, "X_upper", self._shape(K, B), dt)
        _check(w, "W", self._shape(M, K), dt)
        _check(x_lower, "X_lower", self._shape(M, B), dt)
        _check(e, "E", self._shape(M, B), dt)
        ws, nbytes = self._ws(workspace)
        nat.check(nat.lib().ipc_pred_err_ws(
            x_upper.data_ptr(), w.data_ptr(), x_lower.data_ptr(), e.data_ptr(), M, K, B, self.groups,
            self.storage, self.operand, self.split, self.act, self.tile, ws, nbytes,
            nat.current_stream_handle(e.device)))


class ForwardKernel(_Kernel):
    """``k(X_upper[K,B], W[M,K], OUT[M,B], *, workspace=None)``: ``OUT = W f(X_upper)``."""

    _ws_kind = 0

    def __call__(self, x_upper, w, out, *, workspace=None):
        M, K, B, dt = self.M, self.K, self.B, self.dtype
        _check(x_upper, "X_upper", self._shape(K, B), dt)
        _check(w, "W", self._shape(M, K), dt)
        _check(out, "OUT", self._shape(M, B), dt)
        ws, nbytes = self._ws(workspace)
        nat.check(nat.lib().ipc_forward_ws(
            x_upper.data_ptr(), w.data_ptr(), out.data_ptr(), M, K, B, self.groups,
            self.storage, self.operand, self.split, self.act, self.tile, ws, nbytes,
            nat.current_stream_handle(out.device)))


class InferenceUpdateKernel(_Kernel):
    """``k(X[M,B], E[M,B], W_lower[K,M], E_lower[K,B][, A_out[M,B]], *, workspace=None)``:
    ``X += gamma(-E + f'(X) W_lower^T E_lower)`` (and ``A_out = f(X_new)``).
    ``workspace`` (optional, caller-owned, ``new_workspace()``) lets a large
    16-bit call copy W_lower and E_lower transposed, so that its GEMM reads
    both operands k-contiguous (same bits)."""

    _ws_kind = 1

    def __init__(self, *a, gamma: float, save_activation: bool, **kw):
        super().__init__(*a, **kw)
        self.gamma = float(gamma)
        self.save_activation = bool(save_activation)

    def __call__(self, x, e, w_lower, e_lower, a_out=None, *, workspace=None):
        M, K, B, dt = self.M, self.K, self.B, self.dtype
        _check(x, "X", self._shape(M, B), dt)
        _check(e, "E", self._shape(M, B), dt)
        _check(w_lower, "W_lower", self._shape(K, M), dt)
        _check(e_lower, "E_lower", self._shape(K, B), dt)
        if self.save_activation:
            if a_out is None:
                raise ValueError("save_activation kernel needs A_out")
            _check(a_out, "A_out", self._shape(M, B), dt)
        elif a_out is not None:
            raise ValueError("A_out given to a kernel built with save_activation=False")
        ws, nbytes = self._ws(workspace)
        nat.check(nat.lib().ipc_infer_update_ws(
            x.data_ptr(), e.data_ptr(), w_lower.data_ptr(), e_lower.data_ptr(),
            a_out.data_ptr() if a_out is not None else None, M, K, B, self.groups, self.gamma,
            self.storage, self.operand, self.act, self.tile, ws, nbytes, nat.current_stream_handle(x.device)))


class WeightUpdateKernel(_Kernel):
    """``k(W[M,K], E[M,B], X_upper_or_A[K,B], *, workspace=None)``:
    ``W += alpha E f(X_upper)^T`` (recompute) or ``W += alpha E A^T`` (saved
    activation; no workspace is used then)."""

    def __init__(self, *a, alpha: float, recompute_activation: bool, **kw):
        super().__init__(*a, **kw)
        self.alpha = float(alpha)
        self.recompute_activation = bool(recompute_activation)
        self._ws_kind = 2 if self.recompute_activation else -1

    def __call__(self, w, e, x_upper, *, workspace=None):
        M, K, B, dt = self.M, self.K, self.B, self.dtype
        _check(w, "W", self._shape(M, K), dt)
        _check(e, "E", self._shape(M, B), dt)
        _check(x_upper, "X_upper", self._shape(K, B), dt)
        ws, nbytes = self._ws(workspace)
        nat.check(nat.lib().ipc_weight_update_ws(
            w.data_ptr(), e.data_ptr(), x_upper.data_ptr(), M, K, B, self.groups, self.alpha,
            int(self.recompute_activation), self.storage, self.operand, self.act, self.tile, ws, nbytes,
            nat.current_stream_handle(w.device)))


class OuterWeightUpdateKernel(_Kernel):
    """``k(W[M,K], E[M,B], X_upper_or_A[K,B])`` by rank-B outer products (B <= 32)."""

    def __init__(self, *a, alpha: float, recompute_activation: bool, **kw):
        super().__init__(*a, **kw)
        if self.B > 32:
            raise ValueError("outer-product weight update supports B <= 32")
        self.alpha = float(alpha)
        self.recompute_activation = bool(recompute_activation)

    def __call__(self, w, e, x_upper):
        M, K, B, dt = self.M, self.K, self.B, self.dtype
        _check(w, "W", self._shape(M, K), dt)
        _check(e, "E", self._shape(M, B), dt)
        _check(x_upper, "X_upper", self._shape(K, B), dt)
        nat.check(nat.lib().ipc_weight_update_outer(
            w.data_ptr(), e.data_ptr(), x_upper.data_ptr(), M, K, B, self.groups, self.alpha,
            int(self.recompute_activation), self.storage, self.act, nat.current_stream_handle(w.device)))


@lru_cache(maxsize=256)
def build_prediction_error(M: int, K: int, B: int, activation: str, dtype, cfg: KernelConfig | None = None,
                           *, operand_dtype=None, split: int = 1):
    """``W[M,K] @ f(X_upper[K,B]) -> E[M,B]`` (reference ``tilelang_kernels.py:114-177``).

    ``split`` (fp32 storage with 16-bit operands): 1 = plain 16-bit operands,
    2 = W as hi + lo 16-bit terms, 3 = W and f(X_upper) both split."""
    return PredictionErrorKernel("prediction", M, K, B, activation, dtype, cfg, operand_dtype, split=split)


@lru_cache(maxsize=256)
def build_forward(M: int, K: int, B: int, activation: str, dtype, cfg: KernelConfig | None = None,
                  *, operand_dtype=None, split: int = 1):
    """``OUT = W f(X_upper)`` (forward initialisation ``trainer.py:512-515``)."""
    return ForwardKernel("forward", M, K, B, activation, dtype, cfg, operand_dtype, split=split)


@lru_cache(maxsize=256)
def build_inference_update(M: int, K: int, B: int, activation: str, dtype, cfg: KernelConfig | None = None,
                           gamma: float = 0.5, save_activation: bool = False, *, operand_dtype=None):
    """``X += gamma*(-E + f'(X)*W.T@E_lower)`` (reference ``tilelang_kernels.py:180-265``)."""
    return InferenceUpdateKernel("inference", M, K, B, activation, dtype, cfg, operand_dtype,
                                 gamma=gamma, save_activation=save_activation)


@lru_cache(maxsize=256)
def build_weight_update(M: int, K: int, B: int, activation: str, dtype, cfg: KernelConfig | None = None,
                        alpha: float = 1e-4, recompute_activation: bool = True, *, operand_dtype=None):
    """``W += alpha * E @ A.T`` (reference ``tilelang_kernels.py:268-349``)."""
    return WeightUpdateKernel("weight", M, K, B, activation, dtype, cfg, operand_dtype,
                              alpha=alpha, recompute_activation=recompute_activation)


@lru_cache(maxsize=256)
def build_weight_update_outer(M: int, K: int, B: int, activation: str, dtype, alpha: float = 1e-4,
                              recompute_activation: bool = True, groups: int = 1):
    """Rank-B outer-product form of ``build_weight_update`` for B <= 32."""
    return OuterWeightUpdateKernel("weight_outer", M, K, B, activation, dtype, None, None, groups=groups,
                                   alpha=alpha, recompute_activation=recompute_activation)


def kernel_call(kernel, *tensors: torch.Tensor) -> None:
    """Reference ``tilelang_kernels.py:352-353``."""
    kernel(*tensors)
