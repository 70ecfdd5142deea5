"""Small-batch weight update by rank-B outer products.

Mirrors ``src/ipc_tilelang/weight_update_specialization.py``:
``SmallBWeightPolicy`` (``:24-60``, exact-shape JSON policy selecting "gemm"
or "outer") and ``SmallBWeightUpdater`` (``:63-128``).  The reference's
updater ran ``torch.bmm`` over a ``[B,M,K]`` temporary, used ``-alpha`` (a sign
error against ``reference.py:57`` and its own GEMM path) and only supported
relu/identity.  Here the update is one HIP kernel that streams W once,
``W += +alpha * sum_b E[:,b] f(X[:,b])^T``, for every activation and B <= 32.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from .kernels import build_weight_update_outer

OUTER_MAX_BATCH = 32


def _dtype_name(dtype: Any) -> str:
    return str(dtype).split(".")[-1]


@dataclass(frozen=True)
class WeightPolicyKey:
    M: int
    K: int
    B: int
    activation: str = "relu"
    dtype: str = "float16"


_BACKENDS = ("gemm", "outer")


def _policy_row(row: object):
    """``(key, backend)`` of one policy row, or None for a row a reader must
    skip: not an object, a shape field missing or not an integer, or a
    backend other than gemm / outer."""
    if not isinstance(row, dict):
        return None
    backend = str(row.get("backend", "gemm")).lower()
    if backend not in _BACKENDS:
        return None
    try:
        shape = tuple(int(row[k]) for k in ("M", "K", "B")) + (int(row.get("count", 1)),)
    except (KeyError, TypeError, ValueError):
        return None
    return shape + (str(row.get("activation", "relu")), str(row.get("dtype", "float16"))), backend


class SmallBWeightPolicy:
    """Read-only exact-shape policy: JSON rows ``M, K, B, count, activation,
    dtype, backend`` (the reference's policy format), each choosing "gemm" or
    "outer" for one layer shape; any shape without a row uses "gemm"."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        data = json.loads(self.path.read_text(encoding="utf-8"))
        if not isinstance(data, dict):
            raise ValueError(f"{self.path}: a small-batch weight-update policy is a JSON object with an "
                             f"'entries' list, not a {type(data).__name__}")
        self.data = data
        self.entries: dict[tuple[int, int, int, int, str, str], str] = dict(
            parsed for parsed in map(_policy_row, data.get("entries", [])) if parsed is not None)

    def backend(self, *, M: int, K: int, B: int, activation: str, dtype: Any, count: int = 1) -> str:
        key = (int(M), int(K), int(B), int(count), str(activation), _dtype_name(dtype))
        return self.entries.get(key, "gemm")


class SmallBWeightUpdater:
    """Factory of rank-B outer-product update callables ``fn(w, e, src)``."""

    def __init__(self, *, alpha: float, recompute_activation: bool = True):
        self.alpha = float(alpha)
        self.recompute_activation = bool(recompute_activation)
        self._cache: dict[tuple, object] = {}

    @staticmethod
    def _supported_activation(name: str) -> bool:
        return str(name).lower() in {"relu", "identity", "linear", "tanh", "sigmoid", "silu", "gelu"}

    def make_singleton(self, *, M: int, K: int, B: int, activation: str, dtype: Any):
        if int(B) > OUTER_MAX_BATCH or not self._supported_activation(activation):
            return None
        key = (int(M), int(K), int(B), str(activation), _dtype_name(dtype), 1)
        if key not in self._cache:
            self._cache[key] = build_weight_update_outer(
                int(M), int(K), int(B), str(activation), _dtype_name(dtype), self.alpha,
                self.recompute_activation, 1)
        return self._cache[key]

    def make_grouped(self, *, count: int, M: int, K: int, B: int, activation: str, dtype: Any):
        if int(B) > OUTER_MAX_BATCH or not self._supported_activation(activation) or int(count) < 2:
            return None
        key = (int(M), int(K), int(B), str(activation), _dtype_name(dtype), int(count))
        if key not in self._cache:
            self._cache[key] = build_weight_update_outer(
                int(M), int(K), int(B), str(activation), _dtype_name(dtype), self.alpha,
                self.recompute_activation, int(count))
        return self._cache[key]
