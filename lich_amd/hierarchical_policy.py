"""Reader of the kernel + execution policy artefact (reference
``src/ipc_tilelang/hierarchical_policy.py:55-241``, files such as
``results/hierarchical_policy.json``, schema version 3).

Read-only at training time, with the reference's lookup rules: kernel
choices by exact (kind, M, K, B, activation, dtype) key, first from the
per-net ``kernel_profiles`` then from the global ``kernel_entries``; an
execution choice (``best``: grid.z cap, recompute, graph) additionally
requires the fingerprint of the kernel table actually in use
(``kernel_signature``: SHA-256 of the normalised, sorted rows, first 20 hex
digits, computed as the reference does so its files keep resolving).
Malformed rows are skipped, not fatal.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Any, Mapping

from .kernels import KernelConfig
from .tuning import config_from_dict

SCHEMA_VERSION = 3


def dtype_name(dtype: Any) -> str:
    return str(dtype).split(".")[-1]


def dims_key(dims) -> str:
    return "x".join(str(int(d)) for d in dims)


def _key(**kv) -> str:
    return json.dumps(kv, sort_keys=True, separators=(",", ":"))


def make_kernel_key(kind: str, M: int, K: int, B: int, activation: str, dtype: Any) -> str:
    return _key(kind=str(kind), M=int(M), K=int(K), B=int(B), activation=str(activation), dtype=dtype_name(dtype))


def kernel_signature(rows: list[Mapping[str, Any]]) -> str:
    """Fingerprint of a P/I/W kernel table (rows in the tuning-table form)."""
    norm = []
    for row in rows:
        shape = row.get("shape") or {}
        norm.append({"kind": str(row["kind"]), "M": int(shape["M"]), "K": int(shape["K"]), "B": int(shape["B"]),
                     "activation": str(row.get("activation", "relu")), "dtype": str(row.get("dtype", "float16")),
                     "config": dict(row["config"])})
    norm.sort(key=lambda r: (r["kind"], r["M"], r["K"], r["B"], r["activation"], r["dtype"]))
    raw = json.dumps(norm, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(raw.encode("utf-8")).hexdigest()[:20]


def make_kernel_profile_key(*, dims, batch: int, activation: str, dtype: Any) -> str:
    return _key(dims=dims_key(dims), batch=int(batch), activation=str(activation), dtype=dtype_name(dtype))


def make_execution_key(*, dims, batch: int, activation: str, dtype: Any, kernel_sig: str) -> str:
    return _key(dims=dims_key(dims), batch=int(batch), activation=str(activation), dtype=dtype_name(dtype),
                kernel_signature=str(kernel_sig))


class HierarchicalPolicy:
    def __init__(self, path: str | Path | None = None, *, data: dict | None = None):
        self.path = Path(path) if path is not None else None
        if data is None:
            if self.path is not None and self.path.exists():
                data = json.loads(self.path.read_text(encoding="utf-8"))
            else:
                data = {"schema_version": SCHEMA_VERSION, "kernel_entries": [], "execution_entries": []}
        if not isinstance(data, dict):
            raise ValueError(f"Invalid hierarchical policy: {self.path}")
        self.data = data
        self._kernels: dict[str, KernelConfig] = {}
        for row in data.get("kernel_entries", []):
            try:
                shape = row.get("shape") or {}
                self._kernels[make_kernel_key(row["kind"], shape["M"], shape["K"], shape["B"],
                                              row.get("activation", "relu"), row.get("dtype", "float16"))] = \
                    config_from_dict(row["config"])
            except (KeyError, TypeError, ValueError, AttributeError):
                continue
        self._profiles: dict[str, dict[str, KernelConfig]] = {}
        self._profile_meta: dict[str, dict] = {}
        for prof in data.get("kernel_profiles", []):
            try:
                act, dt = str(prof.get("activation", "relu")), str(prof.get("dtype", "float16"))
                pkey = make_kernel_profile_key(dims=prof["dims"], batch=prof["batch"], activation=act, dtype=dt)
                mapping = {}
                for row in prof.get("kernel_entries", []):
                    try:
                        shape = row.get("shape") or {}
                        mapping[make_kernel_key(row["kind"], shape["M"], shape["K"], shape["B"],
                                                row.get("activation", act), row.get("dtype", dt))] = \
                            config_from_dict(row["config"])
                    except (KeyError, TypeError, ValueError, AttributeError):
                        continue
                if mapping:
                    self._profiles[pkey] = mapping
                    self._profile_meta[pkey] = prof
            except (KeyError, TypeError, ValueError, AttributeError):
                continue
        self._execution: dict[str, dict] = {}
        for row in data.get("execution_entries", []):
            try:
                self._execution[make_execution_key(dims=row["dims"], batch=row["batch"],
                                                   activation=row.get("activation", "relu"),
                                                   dtype=row.get("dtype", "float16"),
                                                   kernel_sig=row["kernel_signature"])] = row
            except (KeyError, TypeError, ValueError, AttributeError):
                continue

    @property
    def exists(self) -> bool:
        return self.path is not None and self.path.exists()

    def lookup_kernel(self, *, kind, M, K, B, activation, dtype) -> KernelConfig | None:
        return self._kernels.get(make_kernel_key(kind, M, K, B, activation, dtype))

    def lookup_profile_kernel(self, *, dims, batch, kind, M, K, activation, dtype) -> KernelConfig | None:
        mapping = self._profiles.get(make_kernel_profile_key(dims=dims, batch=batch, activation=activation,
                                                             dtype=dtype))
        return None if mapping is None else mapping.get(make_kernel_key(kind, M, K, batch, activation, dtype))

    def profile_kernel_signature(self, *, dims, batch, activation, dtype) -> str | None:
        meta = self._profile_meta.get(make_kernel_profile_key(dims=dims, batch=batch, activation=activation,
                                                              dtype=dtype))
        value = None if meta is None else meta.get("kernel_signature")
        return None if value is None else str(value)

    def lookup_execution(self, *, dims, batch, activation, dtype, kernel_sig) -> dict | None:
        return self._execution.get(make_execution_key(dims=dims, batch=batch, activation=activation, dtype=dtype,
                                                      kernel_sig=kernel_sig))

    def _best(self, **kw) -> dict:
        row = self.lookup_execution(**kw)
        best = row.get("best") if isinstance(row, dict) else None
        return best if isinstance(best, dict) else {}

    def selected_grid_z(self, *, default, **kw):
        """The entry's grid.z cap, else ``default`` (which may be None)."""
        value = self._best(**kw).get("grid_z_max_layers")
        try:
            return default if value is None else int(value)
        except (TypeError, ValueError):
            return default

    def selected_recompute_activation(self, *, default: bool, **kw) -> bool:
        return bool(self._best(**kw).get("recompute_activation", default))

    def selected_wide_config(self, *, default, **kw):
        """The entry's wide-path tile configuration ``(pred, infer, weight,
        ksplit)`` (written by ``lich_amd.autotune``), else ``default``."""
        wc = self._best(**kw).get("wide_config")
        if not isinstance(wc, dict):
            return default
        try:
            return tuple(int(wc.get(k, -1)) for k in ("pred", "infer", "weight", "ksplit"))
        except (TypeError, ValueError):
            return default

    def selected_resident_rows(self, *, default, **kw):
        """The entry's layer-resident row-block size (written by
        ``lich_amd.autotune``), else ``default``."""
        rows = self._best(**kw).get("resident_rows")
        try:
            return default if rows is None else int(rows)
        except (TypeError, ValueError):
            return default

    def selected_use_graph(self, *, default: bool, **kw) -> bool:
        return bool(self._best(**kw).get("use_cuda_graph", default))

    def selected_path(self, *, default: str, **kw) -> str:
        """This build's own execution field: the kernel path ("auto",
        "resident", "narrow", "wide", "phased")."""
        return str(self._best(**kw).get("path", default))


def load_hierarchical_policy(path: str | Path) -> HierarchicalPolicy | None:
    p = Path(path)
    return HierarchicalPolicy(p) if p.exists() else None
