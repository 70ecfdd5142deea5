"""Reader of the grid.z layer-batching policy file (``results/gridz_policy.json``).

The file format is the reference's (``src/ipc_tilelang/gridz_tuning.py:16-73``):
``{"version": 1, "entries": {<key>: {"grid_z_max_layers": cap, ...}}}``, where
each key is the compact, key-sorted JSON object of the device name, its
compute capability, the dims joined by ``x``, the batch, the activation and
the dtype name.  A missing file reads as an empty policy, a malformed one
raises ``ValueError``, and a shape without an entry gets the caller's
default, so a trainer given the reference's policy path behaves the same
whether or not the file exists.

On this build the cap selects nothing in the execution: every phase of a
step is already one launch over all layers (or the whole step is one
launch).  The trainer records the cap it read (``HipIPC.grid_z_cap``) and the
groups it implies (``HipIPC.layer_groups``) for callers that inspect them.
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Any


def dtype_name(dtype: Any) -> str:
    """``torch.float16`` -> ``"float16"``; strings pass through."""
    return str(dtype).split(".")[-1]


def dims_key(dims) -> str:
    return "x".join(str(int(d)) for d in dims)


def make_policy_key(*, device_name: str, capability, dims, batch: int, activation: str, dtype: Any) -> str:
    fields = {"device": str(device_name), "capability": [int(c) for c in capability], "dims": dims_key(dims),
              "batch": int(batch), "activation": str(activation), "dtype": dtype_name(dtype)}
    return json.dumps(fields, sort_keys=True, separators=(",", ":"))


def load_policy(path) -> dict:
    p = Path(path)
    if not p.exists():
        return {"version": 1, "entries": {}}
    with p.open("r", encoding="utf-8") as fh:
        data = json.load(fh)
    entries = data.get("entries", {}) if isinstance(data, dict) else None
    if not isinstance(entries, dict):
        raise ValueError(f"{p}: a grid.z policy is an object with an 'entries' object")
    return data


def lookup_grid_z_cap(path, *, device_name: str, capability, dims, batch: int, activation: str, dtype: Any,
                      default: int = 2) -> int:
    """The policy's ``grid_z_max_layers`` for this device and net, else ``default``."""
    row = load_policy(path)["entries"].get(make_policy_key(device_name=device_name, capability=capability,
                                                           dims=dims, batch=batch, activation=activation,
                                                           dtype=dtype))
    if not isinstance(row, dict):
        return int(default)
    return int(row.get("grid_z_max_layers", default))
