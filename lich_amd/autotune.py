"""CDNA4 tuning artefacts for a net (reference ``scripts/autotune.py`` kernel
search and ``scripts/hierarchical_autotune.py`` execution search, reduced to
this library's choices).

* Kernel level: for every prediction / inference / weight shape of the net,
  each tile configuration of the standalone kernels is timed (HIP events
  around graph replays of back-to-back launches on the launch stream, the
  method of ``autotune.py:200-215``); the fastest goes into a TuningTable
  (schema 1).
* Execution level: one iPC step is timed on every eligible path ("resident",
  "narrow", "wide", "phased") with activation recompute on and off and with
  and without graph replay; the fastest becomes the ``best`` of an execution
  entry of a policy file (schema 3) next to the kernel table as a
  ``kernel_profiles`` entry, so ``HipIPC`` reads its choices through the
  reference's precedence.

    python -m lich_amd.autotune --dims 10,64,64,64,784 --batch 128 --activation tanh \\
        --dtype float16 --table results/tuning_cdna4.json --policy results/hierarchical_policy.json
"""
from __future__ import annotations

import argparse
import json
import time
from pathlib import Path

import torch

from . import _native as nat
from .hierarchical_policy import SCHEMA_VERSION, kernel_signature
from .kernels import KernelConfig, build_inference_update, build_prediction_error, build_weight_update
from .trainer import HipIPC, IPCConfig, init_weights_cpu
from .tuning import TuningEntry, TuningKey, TuningTable, config_to_dict

TILES = (0, 1, 2, 3)


def _time_us(fn, reps: int, replays: int) -> float:
    """Average microseconds of one ``fn()`` from HIP events around graph replays."""
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * replays)


def net_shapes(dims) -> list[tuple[str, int, int]]:
    """(kind, M, K) of every kernel of a step, the rows of the reference's table."""
    L = len(dims) - 1
    out = []
    for l in range(L):
        out += [("prediction", dims[l], dims[l + 1]), ("weight", dims[l], dims[l + 1])]
        if l > 0:
            out.append(("inference", dims[l], dims[l - 1]))
    return list(dict.fromkeys(out))


def tune_kernels(dims, B: int, activation: str, dtype: torch.dtype, *, reps: int = 20, replays: int = 3,
                 storage: torch.dtype = torch.float32, seed: int = 0) -> TuningTable:
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(seed)
    dt = str(dtype).split(".")[-1]
    entries = []
    for kind, M, K in net_shapes([int(d) for d in dims]):
        def rnd(*shape):
            return torch.randn(shape, generator=g).to(device=dev, dtype=storage)
        best = None
        for tile in TILES:
            cfg = KernelConfig(tile=tile)
            try:
                if kind == "prediction":
                    k = build_prediction_error(M, K, B, activation, storage, cfg, operand_dtype=dtype)
                    xu, w, xl, e = rnd(K, B), rnd(M, K) * 0.05, rnd(M, B), rnd(M, B)
                    fn = lambda: k(xu, w, xl, e)  # noqa: E731
                elif kind == "inference":
                    k = build_inference_update(M, K, B, activation, storage, cfg, operand_dtype=dtype)
                    x, e, wl, el = rnd(M, B), rnd(M, B), rnd(K, M) * 0.05, rnd(K, B)
                    fn = lambda: k(x, e, wl, el)  # noqa: E731
                else:
                    k = build_weight_update(M, K, B, activation, storage, cfg, operand_dtype=dtype)
                    w, e, xu = rnd(M, K), rnd(M, B), rnd(K, B)
                    fn = lambda: k(w, e, xu)  # noqa: E731
                us = _time_us(fn, reps, replays)
            except (ValueError, nat.IPCNativeError):
                continue  # tile not eligible for this shape / storage
            if best is None or us < best[0]:
                best = (us, cfg)
        if best is not None:
            entries.append(TuningEntry(TuningKey(kind, M, K, B, activation, dt), best[1], best[0] / 1e3, False))
    return TuningTable.from_entries(entries)


def tune_execution(dims, B: int, activation: str, dtype: torch.dtype, *, steps: int = 4, replays: int = 50,
                   seed: int = 0) -> tuple[dict, list[dict]]:
    """Best (path, recompute, graph) for one step, and every trial."""
    dev = torch.device("cuda", torch.cuda.current_device())
    w0 = init_weights_cpu(dims, seed=seed, init="xavier_uniform")
    g = torch.Generator().manual_seed(seed + 7919)
    x_in = torch.rand((dims[-1], B), generator=g).to(dev)
    y = torch.nn.functional.one_hot(torch.randint(0, dims[0], (B,), generator=g), dims[0]).float().T.contiguous().to(dev)
    trials = []
    for path in ("resident", "narrow", "wide", "phased"):
        for recompute in (True, False):
            for graph in (True, False):
                cfg = IPCConfig(dims=tuple(dims), activation=activation, dtype=dtype, fused=path,
                                recompute_activation=recompute, hierarchical_policy_auto=False)
                try:
                    m = HipIPC(cfg, device=dev, weights=w0)
                    m.prepare_steady_state(x_in, y, steps=steps, use_graph=graph)
                except (ValueError, nat.IPCNativeError):
                    continue  # path not eligible for this net
                m.run_prepared_steady_state(steps=steps, repeats=3, use_graph=graph)
                t0 = time.perf_counter()
                m.run_prepared_steady_state(steps=steps, repeats=replays, use_graph=graph)
                dt = time.perf_counter() - t0
                step_ms = dt * 1e3 / (steps * replays)
                trials.append({"path": path, "recompute_activation": recompute, "use_cuda_graph": graph,
                               "grid_z_max_layers": 1, "step_ms": step_ms, "samples_per_s": B / step_ms * 1e3,
                               "status": "ok", "source": "gpu"})
                del m
    best = min(trials, key=lambda t: t["step_ms"])
    return best, trials


def write_policy(path: str | Path, dims, B: int, activation: str, dtype: torch.dtype, table: TuningTable,
                 best: dict, trials: list[dict]) -> dict:
    """Adds (or replaces) this net's kernel profile and execution entry in a
    schema-3 policy file."""
    p = Path(path)
    data = json.loads(p.read_text(encoding="utf-8")) if p.exists() else {}
    data.setdefault("schema_version", SCHEMA_VERSION)
    data.setdefault("kernel_entries", [])
    data.setdefault("kernel_profiles", [])
    data.setdefault("execution_entries", [])
    data["device"] = torch.cuda.get_device_name(0)
    data["arch"] = nat.device_arch(0)
    dt = str(dtype).split(".")[-1]
    rows = [{"kind": e.key.kind, "shape": {"M": e.key.M, "K": e.key.K, "B": e.key.B},
             "activation": e.key.activation, "dtype": e.key.dtype, "config": config_to_dict(e.config)}
            for e in table.entries]
    sig = kernel_signature(rows)
    same = lambda r: list(r.get("dims", [])) == list(dims) and r.get("batch") == B and \
        r.get("activation") == activation and r.get("dtype") == dt  # noqa: E731
    data["kernel_profiles"] = [r for r in data["kernel_profiles"] if not same(r)] + [
        {"dims": list(dims), "batch": B, "activation": activation, "dtype": dt, "kernel_signature": sig,
         "selection_source": "lich_amd.autotune", "kernel_entries": rows}]
    data["execution_entries"] = [r for r in data["execution_entries"] if not same(r)] + [
        {"dims": list(dims), "batch": B, "activation": activation, "dtype": dt, "kernel_signature": sig,
         "best": dict(best, depth=len(dims) - 2), "candidates": trials, "fidelity": "full"}]
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(json.dumps(data, indent=2), encoding="utf-8")
    return data


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="CDNA4 kernel and execution tuning for one net")
    ap.add_argument("--dims", required=True, help="comma-separated, d_0 (classes) first")
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--activation", default="tanh")
    ap.add_argument("--dtype", choices=["float16", "bfloat16"], default="float16")
    ap.add_argument("--table", default="results/tuning_cdna4.json")
    ap.add_argument("--policy", default="results/hierarchical_policy.json")
    ap.add_argument("--steps", type=int, default=4)
    a = ap.parse_args(argv)
    dims = [int(v) for v in a.dims.split(",")]
    dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16}[a.dtype]
    table = tune_kernels(dims, a.batch, a.activation, dtype)
    table.to_json(a.table, device=torch.cuda.get_device_name(0))
    best, trials = tune_execution(dims, a.batch, a.activation, dtype, steps=a.steps)
    write_policy(a.policy, dims, a.batch, a.activation, dtype, table, best, trials)
    print(json.dumps({"table": a.table, "policy": a.policy, "kernels": len(table.entries), "best": best}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
