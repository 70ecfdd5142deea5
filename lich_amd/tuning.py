"""Per-shape kernel tuning tables in the reference's schema version 1.

The format (reference ``src/ipc_tilelang/tuning.py:10-108``) is kept so that a
table written on either side reads on the other::

    {"schema_version": 1, "device": ..., "capability": [major, minor] | null,
     "entries": [{"kind", "shape": {"M", "K", "B"}, "activation", "dtype",
                  "median_ms", "spill_suspected", "config": {...}}]}

``config`` holds ``KernelConfig`` fields.  A config written here carries this
library's ``tile`` id next to the block sizes; a config without one (a
reference table) maps to the nearest tile through ``KernelConfig.tile_id``.
The reader is stricter than the format needs: a row without its kind, shape or
config is reported with its index instead of being half-read.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field, fields
from pathlib import Path
from typing import Iterable

from .kernels import KernelConfig

SCHEMA_VERSION = 1
_ROW_DEFAULTS = {"activation": "relu", "dtype": "float16"}


def config_from_dict(data: dict) -> KernelConfig:
    """A KernelConfig from a JSON config, ignoring fields this build does not
    know (a table from another backend may carry more)."""
    known = {f.name for f in fields(KernelConfig)}
    return KernelConfig(**{k: v for k, v in dict(data).items() if k in known})


def config_to_dict(cfg: KernelConfig) -> dict:
    """The JSON form of a config: every field set, ``tile`` only when given,
    so a config without one serialises exactly like the reference's."""
    return {f.name: getattr(cfg, f.name) for f in fields(KernelConfig)
            if not (f.name == "tile" and getattr(cfg, f.name) is None)}


@dataclass(frozen=True)
class TuningKey:
    """What a tuned config is for: the kernel kind, its GEMM shape, the fused
    activation and the storage dtype name."""
    kind: str
    M: int
    K: int
    B: int
    activation: str
    dtype: str


@dataclass(frozen=True)
class TuningEntry:
    key: TuningKey
    config: KernelConfig
    median_ms: float | None = None
    spill_suspected: bool | None = None


def _row_to_entry(index: int, row: object, source: str) -> TuningEntry:
    if not isinstance(row, dict):
        raise ValueError(f"{source}: entry {index} is a {type(row).__name__}, not an object")
    missing = [k for k in ("kind", "shape", "config") if k not in row]
    if missing:
        raise ValueError(f"{source}: entry {index} lacks {', '.join(missing)}")
    shape = row["shape"]
    try:
        M, K, B = (int(shape[d]) for d in ("M", "K", "B"))
    except (KeyError, TypeError, ValueError) as exc:
        raise ValueError(f"{source}: entry {index} has no integer M, K and B in its shape") from exc
    key = TuningKey(str(row["kind"]), M, K, B, str(row.get("activation", _ROW_DEFAULTS["activation"])),
                    str(row.get("dtype", _ROW_DEFAULTS["dtype"])))
    ms = row.get("median_ms")
    return TuningEntry(key, config_from_dict(row["config"]), None if ms is None else float(ms),
                       row.get("spill_suspected"))


def _entry_to_row(e: TuningEntry) -> dict:
    k = e.key
    return {"kind": k.kind, "shape": {"M": k.M, "K": k.K, "B": k.B}, "activation": k.activation,
            "dtype": k.dtype, "median_ms": e.median_ms, "spill_suspected": e.spill_suspected,
            "config": config_to_dict(e.config)}


@dataclass(frozen=True)
class TuningTable:
    """An ordered list of entries; a lookup returns the first entry's config
    whose key matches exactly (later duplicates never win)."""
    entries: tuple[TuningEntry, ...]
    _index: dict = field(default=None, init=False, repr=False, compare=False, hash=False)

    def __post_init__(self):
        index: dict[TuningKey, KernelConfig] = {}
        for e in self.entries:
            index.setdefault(e.key, e.config)
        object.__setattr__(self, "_index", index)

    @classmethod
    def from_entries(cls, entries: Iterable[TuningEntry]) -> "TuningTable":
        return cls(tuple(entries))

    @classmethod
    def from_json(cls, path: str | Path) -> "TuningTable":
        source = str(path)
        payload = json.loads(Path(path).read_text(encoding="utf-8"))
        if not isinstance(payload, dict):
            raise ValueError(f"{source}: a tuning table is a JSON object")
        version = payload.get("schema_version")
        if version != SCHEMA_VERSION:
            raise ValueError(f"Unsupported tuning schema: {source} has schema_version {version!r}, "
                             f"and this reader handles version {SCHEMA_VERSION} only")
        rows = payload.get("entries", [])
        if not isinstance(rows, list):
            raise ValueError(f"{source}: 'entries' is not a list")
        return cls(tuple(_row_to_entry(i, r, source) for i, r in enumerate(rows)))

    def lookup(self, *, kind: str, M: int, K: int, B: int, activation: str, dtype: str) -> KernelConfig | None:
        return self._index.get(TuningKey(kind, int(M), int(K), int(B), activation, dtype))

    def to_json(self, path: str | Path, *, device: str | None = None,
                capability: tuple[int, int] | None = None) -> None:
        payload = {"schema_version": SCHEMA_VERSION, "device": device,
                   "capability": None if capability is None else list(capability),
                   "entries": [_entry_to_row(e) for e in self.entries]}
        out = Path(path)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(payload, indent=2), encoding="utf-8")
