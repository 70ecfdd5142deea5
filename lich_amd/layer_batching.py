"""Layer-batched ("grid.z") kernels for repeated square internal layers.

Mirrors ``src/ipc_tilelang/layer_batching.py``: ``LayerBatchGroup``
(``:16-43``), ``find_internal_square_groups`` (``:46-86``) and the batched
builders (``:89-346``) that run the same math over a leading group dimension
in one launch.  Here the group dimension is one more index of the library's
ragged launch, so groups need not be square or equal-shaped inside the
library; the square restriction is kept only for these drop-in builders.

The trainer does not need groups: its whole-step plan already launches each
phase (all layers) as one kernel.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

from .kernels import (ForwardKernel, InferenceUpdateKernel, KernelConfig, PredictionErrorKernel,
                      WeightUpdateKernel)


@dataclass(frozen=True)
class LayerBatchGroup:
    """A contiguous run of identical internal square weight layers (edges
    ``start..end``, hidden states ``start..end+1``); endpoints are never part
    of a group, so inference never updates ``x[0]`` or ``x[L]``."""

    start: int
    end: int
    width: int

    @property
    def count(self) -> int:
        return self.end - self.start + 1

    @property
    def state_count(self) -> int:
        return self.count + 1

    @property
    def edge_indices(self) -> tuple[int, ...]:
        return tuple(range(self.start, self.end + 1))

    @property
    def state_indices(self) -> tuple[int, ...]:
        return tuple(range(self.start, self.end + 2))


def find_internal_square_groups(dims: tuple[int, ...], *, max_group_count: int = 2) -> tuple[LayerBatchGroup, ...]:
    """Non-overlapping groups of at most ``max_group_count`` square internal
    edges; consecutive groups leave one edge between them so that their
    hidden-state runs never share a boundary state (reference ``:46-86``)."""
    if len(dims) < 4 or max_group_count < 2:
        return ()
    L = len(dims) - 1
    groups: list[LayerBatchGroup] = []
    l = 1
    while l <= L - 2:
        width = int(dims[l])
        if int(dims[l + 1]) != width:
            l += 1
            continue
        first = l
        while l <= L - 2 and int(dims[l]) == width and int(dims[l + 1]) == width:
            l += 1
        last = l - 1
        p = first
        while p <= last:
            q = min(p + max_group_count - 1, last)
            if q - p + 1 >= 2:
                groups.append(LayerBatchGroup(start=p, end=q, width=width))
                p = q + 2
            else:
                p += 1
    return tuple(groups)


def _square(M: int, K: int, groups: int) -> None:
    if groups < 2:
        raise ValueError("batched kernels require groups >= 2")
    if M != K:
        raise ValueError("batched kernels batch only square internal layers")


@lru_cache(maxsize=128)
def build_prediction_error_batched(M: int, K: int, B: int, groups: int, activation: str, dtype,
                                   cfg: KernelConfig | None = None, *, operand_dtype=None, split: int = 1):
    """``E[g] = X_lower[g] - W[g] f(X_upper[g])`` over ``[G, ...]`` tensors (reference ``:89-150``)."""
    _square(M, K, groups)
    return PredictionErrorKernel("prediction", M, K, B, activation, dtype, cfg, operand_dtype, groups=groups,
                                 split=split)


@lru_cache(maxsize=128)
def build_forward_batched(M: int, K: int, B: int, groups: int, activation: str, dtype,
                          cfg: KernelConfig | None = None, *, operand_dtype=None, split: int = 1):
    _square(M, K, groups)
    return ForwardKernel("forward", M, K, B, activation, dtype, cfg, operand_dtype, groups=groups, split=split)


@lru_cache(maxsize=128)
def build_inference_update_batched(M: int, K: int, B: int, groups: int, activation: str, dtype,
                                   cfg: KernelConfig | None = None, gamma: float = 0.5,
                                   save_activation: bool = False, *, operand_dtype=None):
    """Batched inference update (reference ``:153-248``)."""
    _square(M, K, groups)
    return InferenceUpdateKernel("inference", M, K, B, activation, dtype, cfg, operand_dtype, groups=groups,
                                 gamma=gamma, save_activation=save_activation)


@lru_cache(maxsize=128)
def build_weight_update_batched(M: int, K: int, B: int, groups: int, activation: str, dtype,
                                cfg: KernelConfig | None = None, alpha: float = 1e-4,
                                recompute_activation: bool = True, *, operand_dtype=None):
    """Batched ``W[g] += alpha E[g] A[g]^T`` (reference ``:251-346``)."""
    _square(M, K, groups)
    return WeightUpdateKernel("weight", M, K, B, activation, dtype, cfg, operand_dtype, groups=groups,
                              alpha=alpha, recompute_activation=recompute_activation)
