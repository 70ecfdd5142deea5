"""Per-shape kernel tuning tables, schema version 1 (reference ``src/ipc_tilelang/tuning.py:10-108``).

The file format is the reference's, so a table written by either side reads
on the other: ``{"schema_version": 1, "device", "capability", "entries":
[{"kind", "shape": {"M", "K", "B"}, "activation", "dtype", "median_ms",
"spill_suspected", "config": {...KernelConfig fields...}}]}``.  A config
written here carries this library's ``tile`` id next to the reference's
block sizes; a reference config (block sizes only) maps to the nearest tile
(``KernelConfig.tile_id``).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Iterable

from .kernels import KernelConfig

SCHEMA_VERSION = 1


def config_from_dict(data: dict) -> KernelConfig:
    """A KernelConfig from a JSON config, ignoring fields this build does not
    know (a table from another backend may carry more)."""
    known = {f.name for f in fields(KernelConfig)}
    return KernelConfig(**{k: v for k, v in dict(data).items() if k in known})


def config_to_dict(cfg: KernelConfig) -> dict:
    """The JSON form of a config: every field set, ``tile`` only when given,
    so a config without one serialises exactly like the reference's."""
    out = {}
    for f in fields(KernelConfig):
        v = getattr(cfg, f.name)
        if f.name == "tile" and v is None:
            continue
        out[f.name] = v
    return out


@dataclass(frozen=True)
class TuningKey:
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


@dataclass(frozen=True)
class TuningTable:
    entries: tuple[TuningEntry, ...]

    @classmethod
    def from_entries(cls, entries: Iterable[TuningEntry]) -> "TuningTable":
        return cls(tuple(entries))

    @classmethod
    def from_json(cls, path: str | Path) -> "TuningTable":
        payload = json.loads(Path(path).read_text(encoding="utf-8"))
        if payload.get("schema_version") != SCHEMA_VERSION:
            raise ValueError(f"Unsupported tuning schema: {payload.get('schema_version')!r}; "
                             f"expected {SCHEMA_VERSION}")
        entries = []
        for row in payload.get("entries", []):
            shape = row["shape"]
            key = TuningKey(kind=row["kind"], M=int(shape["M"]), K=int(shape["K"]), B=int(shape["B"]),
                            activation=str(row.get("activation", "relu")), dtype=str(row.get("dtype", "float16")))
            ms = row.get("median_ms")
            entries.append(TuningEntry(key, config_from_dict(row["config"]), None if ms is None else float(ms),
                                       row.get("spill_suspected")))
        return cls(tuple(entries))

    def lookup(self, *, kind: str, M: int, K: int, B: int, activation: str, dtype: str) -> KernelConfig | None:
        key = TuningKey(kind, int(M), int(K), int(B), activation, dtype)
        for entry in self.entries:
            if entry.key == key:
                return entry.config
        return None

    def to_json(self, path: str | Path, *, device: str | None = None,
                capability: tuple[int, int] | None = None) -> None:
        rows = [{"kind": e.key.kind, "shape": {"M": e.key.M, "K": e.key.K, "B": e.key.B},
                 "activation": e.key.activation, "dtype": e.key.dtype, "median_ms": e.median_ms,
                 "spill_suspected": e.spill_suspected, "config": config_to_dict(e.config)} for e in self.entries]
        payload = {"schema_version": SCHEMA_VERSION, "device": device,
                   "capability": list(capability) if capability is not None else None, "entries": rows}
        out = Path(path)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(payload, indent=2), encoding="utf-8")
