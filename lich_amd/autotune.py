"""CDNA4 tuning artefacts for a net (reference ``scripts/autotune.py`` kernel
search and ``scripts/hierarchical_autotune.py`` execution search, reduced to
this library's choices), every candidate gated on correctness.

* Kernel level: for every prediction / inference / weight shape of the net,
  each tile configuration of the standalone kernels (generic 32x32, 64x64,
  128x128 and the LDS-DMA tile) is run on seeded data, checked against torch
  on the device with the reference's probe (``autotune.py:250-260``: at most
  1 % of the elements outside ``atol + rtol |ref|``, rtol = atol = 2e-2) and,
  if it passes, timed (HIP events around graph replays of back-to-back
  launches, the method of ``autotune.py:200-215``); the fastest passing one
  goes into a TuningTable (schema 1).
* Wide path (nets the wide GEMM path serves): each phase's tile
  configurations and the k-split of the output layer's prediction
  (``ipc_plan_set_wide_config``).  A candidate runs one step from a fixed
  state, is checked against a float32 torch step on the device with the same
  probe (states, errors, weight deltas), and its phase launch is then timed;
  the fastest passing configuration of each phase is kept.
* Execution level: one iPC step is timed on every eligible path ("resident",
  "narrow", "wide", "phased") with activation recompute on and off and with
  and without graph replay; the fastest becomes the ``best`` of an execution
  entry of a policy file (schema 3), with the wide configuration, next to the
  kernel table as a ``kernel_profiles`` entry, so ``HipIPC`` reads its
  choices through the reference's precedence.

* Standalone kernels with 16-bit storage (the per-kernel sweep's operator
  calls, ``tune_standalone``): the generic tiles and the four LDS-DMA tile
  configurations (256x128, 128x256, 128x128, 256x256) per (kind, M, K, B), under the
  same probe.
* Layer-resident plans: the top layer's row-block size (16, 32 or 64 rows,
  ``ipc_plan_set_resident_rows``) is part of the execution search; every
  execution candidate runs one step from the forward-initialised state and
  must pass the probe on states, errors and weight deltas against a float32
  torch step before it is timed.

Candidates that fail the probe are never selected; they are recorded with
the reason (``rejected``).

    python -m lich_amd.autotune --dims 10,64,64,64,784 --batch 128 --activation tanh \\
        --dtype float16 --table results/tuning_cdna4.json --policy results/hierarchical_policy.json
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import time
from pathlib import Path

import torch

from . import _native as nat
from .hierarchical_policy import SCHEMA_VERSION, kernel_signature
from .kernels import KernelConfig, build_inference_update, build_prediction_error, build_weight_update
from .reference import get_activation
from .trainer import HipIPC, IPCConfig, init_weights_cpu
from .tuning import TuningEntry, TuningKey, TuningTable, config_to_dict

TILES = (0, 1, 2, 3, 4, 5, 6)  # generic 32x32, 64x64, 128x128; LDS-DMA 256x128, 128x256, 128x128, 256x256
RESIDENT_ROWS = (16, 32, 64)
RTOL = ATOL = 2e-2
MAX_BAD = 0.01


def probe(out: torch.Tensor, ref: torch.Tensor, *, rtol: float = RTOL, atol: float = ATOL,
          max_bad: float = MAX_BAD) -> tuple[bool, str | None]:
    """The reference's correctness probe (``scripts/autotune.py:250-260``):
    fails when more than ``max_bad`` of the elements lie outside
    ``atol + rtol |ref|`` (a NaN counts as outside)."""
    got, ref = out.float(), ref.float()
    diff = (got - ref).abs()
    bad = ~(diff <= atol + rtol * ref.abs())
    ratio = float(bad.float().mean().item()) if bad.numel() else 0.0
    if ratio > max_bad:
        max_abs = float(diff.max().item()) if diff.numel() else 0.0
        return False, f"mismatch ratio={ratio:.6f} max_abs={max_abs:.6g}"
    return True, None


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


def _kernel_case(kind, M, K, B, activation, dtype, storage, cfg, g, dev):
    """(callable that runs the kernel once, callable returning (output, torch reference))."""
    act = get_activation(activation) if activation != "identity" else None
    f = (lambda t: t) if act is None else act.forward
    df = (lambda t: torch.ones_like(t)) if act is None else act.derivative
    rnd = lambda *shape: torch.randn(shape, generator=g).to(device=dev, dtype=storage)  # noqa: E731
    op = lambda t: t.to(dtype).float()  # noqa: E731  (operands as the kernel rounds them)
    if kind == "prediction":
        k = build_prediction_error(M, K, B, activation, storage, cfg, operand_dtype=dtype)
        xu, w, xl, e = rnd(K, B), rnd(M, K) * 0.05, rnd(M, B), rnd(M, B)
        return (lambda: k(xu, w, xl, e)), (lambda: (e, xl.float() - op(w) @ op(f(xu.float()))))
    if kind == "inference":
        k = build_inference_update(M, K, B, activation, storage, cfg, operand_dtype=dtype)
        x0, e, wl, el = rnd(M, B), rnd(M, B), rnd(K, M) * 0.05, rnd(K, B)
        x = x0.clone()
        ref = x0.float() + 0.5 * (-e.float() + df(x0.float()) * (op(wl).T @ op(el)))

        def run():
            x.copy_(x0)
            k(x, e, wl, el)
        return run, (lambda: (x, ref))
    k = build_weight_update(M, K, B, activation, storage, cfg, operand_dtype=dtype, alpha=1e-2)
    w0, e, xu = rnd(M, K), rnd(M, B), rnd(K, B)
    w = w0.clone()
    ref = 1e-2 * (op(e) @ op(f(xu.float())).T)

    def run():
        w.copy_(w0)
        k(w, e, xu)
    return run, (lambda: (w.float() - w0.float(), ref))


def tune_kernels(dims, B: int, activation: str, dtype: torch.dtype, *, reps: int = 20, replays: int = 3,
                 storage: torch.dtype = torch.float32, seed: int = 0, rejected: list | None = None,
                 perturb=None, timer=None, shapes=None) -> TuningTable:
    """Fastest passing tile per (kind, M, K) of the net (or of ``shapes``).
    ``perturb(kind, M, K, tile, out)`` (tests) may alter a candidate's output
    before the probe; ``timer(kind, M, K, tile, us)`` may replace a measured
    time."""
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator().manual_seed(seed)
    dt = str(dtype).split(".")[-1]
    entries = []
    for kind, M, K in (shapes if shapes is not None else net_shapes([int(d) for d in dims])):
        best = None
        for tile in TILES:
            cfg = KernelConfig(tile=tile)
            try:
                run, result = _kernel_case(kind, M, K, B, activation, dtype, storage, cfg, g, dev)
                run()
                torch.cuda.synchronize()
            except (ValueError, nat.IPCNativeError):
                continue  # tile not eligible for this shape / storage
            out, ref = result()
            if perturb is not None:
                perturb(kind, M, K, tile, out)
            ok, why = probe(out, ref)
            if not ok:
                if rejected is not None:
                    rejected.append({"kind": kind, "M": M, "K": K, "B": B, "tile": tile, "reason": why})
                continue
            us = _time_us(run, reps, replays)
            if timer is not None:
                us = timer(kind, M, K, tile, us)
            if best is None or us < best[0]:
                best = (us, cfg)
        if best is not None:
            entries.append(TuningEntry(TuningKey(kind, M, K, B, activation, dt), best[1], best[0] / 1e3, False))
    return TuningTable.from_entries(entries)


def tune_standalone(points, activation: str, dtype: torch.dtype, *, reps: int = 5, replays: int = 3, seed: int = 0,
                    rejected: list | None = None, perturb=None, timer=None) -> TuningTable:
    """The operator calls with 16-bit storage (``dtype`` both storage and
    operand type), as the per-kernel sweep makes them: for every (M, K, B) of
    ``points`` the prediction, inference and weight kernels over every tile
    (the four LDS-DMA configurations where the shape allows them), gated and
    timed like ``tune_kernels``."""
    entries = []
    for M, K, B in points:
        t = tune_kernels(None, int(B), activation, dtype, reps=reps, replays=replays, storage=dtype, seed=seed,
                         rejected=rejected, perturb=perturb, timer=timer,
                         shapes=[("prediction", int(M), int(K)), ("inference", int(M), int(K)),
                                 ("weight", int(M), int(K))])
        entries += list(t.entries)
    return TuningTable.from_entries(entries)


def _batch(dims, B, seed, dev):
    g = torch.Generator().manual_seed(seed + 7919)
    x_in = torch.randn((dims[-1], B), generator=g).to(dev)
    y = torch.nn.functional.one_hot(torch.randint(0, dims[0], (B,), generator=g), dims[0]).float().T.contiguous()
    return x_in, y.to(dev)


def _torch_step(x, w, act, alpha=1e-4, gamma=0.5):
    """One float32 iPC step with torch on the device (the probe's reference)."""
    L = len(w)
    e = [x[l] - w[l] @ act.forward(x[l + 1]) for l in range(L)]
    xn = [x[0]] + [x[l] + gamma * (-e[l] + act.derivative(x[l]) * (w[l - 1].T @ e[l - 1])) for l in range(1, L)] \
        + [x[L]]
    wn = [w[l] + alpha * (e[l] @ act.forward(xn[l + 1]).T) for l in range(L)]
    return xn, e, wn


def tune_wide(dims, B: int, activation: str, dtype: torch.dtype, *, seed: int = 0, reps: int = 5, replays: int = 3,
              rejected: list | None = None, perturb=None, timer=None) -> dict | None:
    """Fastest passing tile configuration of each wide-path phase and k-split
    ({"pred", "infer", "weight", "ksplit"}, -1 = default), or None when the
    net does not take the wide path.  ``perturb(phase, cfg, model)`` (tests)
    may alter a candidate's state after its step; ``timer(phase, cfg, us)``
    may replace a measured time."""
    dev = torch.device("cuda", torch.cuda.current_device())
    dims = [int(d) for d in dims]
    w0 = init_weights_cpu(dims, seed=seed, init="xavier_uniform")
    x_in, y = _batch(dims, B, seed, dev)
    act = get_activation(activation)
    base = IPCConfig(dims=tuple(dims), activation=activation, dtype=dtype, fused="wide", hierarchical_policy_auto=False)
    try:
        probe_model = HipIPC(base, device=dev, weights=w0)
        probe_model.initialize_batch(x_in, y)
    except (ValueError, nat.IPCNativeError):
        return None
    split = probe_model.pred_split
    x0 = [t.clone() for t in probe_model.x]
    ref_x, ref_e, ref_w = _torch_step(x0, [w.to(dev) for w in w0], act)
    ref_dw = [rw - w.to(dev) for rw, w in zip(ref_w, w0)]
    del probe_model

    def candidates(phase):
        n = int(nat.lib().ipc_plan_wide_config_count(phase, split))
        if phase == nat_phase("pred"):
            return [(c, k) for c in range(n) for k in (-1, 1, 2, 4, 8, 16)]
        return [(c, -1) for c in range(n)]

    chosen = {"pred": -1, "infer": -1, "weight": -1, "ksplit": -1}
    for name in ("pred", "infer", "weight"):
        phase = nat_phase(name)
        best = None
        for cfg, ks in candidates(phase):
            wc = [-1, -1, -1, ks]
            wc[phase] = cfg
            try:
                m = HipIPC(dataclasses.replace(base, wide_config=tuple(wc)), device=dev, weights=w0)
                m.initialize_batch(x_in, y)
            except (ValueError, nat.IPCNativeError):
                continue  # k-split not available for this net
            m.run_steps(1)
            torch.cuda.synchronize()
            if perturb is not None:
                perturb(name, (cfg, ks), m)
            L = len(dims) - 1
            fails = _probe_group("x", m.x[1:L], ref_x[1:L]) + _probe_group("eps", m.e[:L], ref_e) + \
                _probe_group("dW", [m.w[l] - w0[l].to(dev) for l in range(L)], ref_dw)
            if fails:
                if rejected is not None:
                    rejected.append({"phase": name, "config": cfg, "ksplit": ks, "reason": "; ".join(fails)})
                del m
                continue
            us = _time_us(lambda: nat.check(nat.lib().ipc_plan_phase(m._plan, phase, 1, nat.current_stream_handle())),
                          reps, replays)
            if timer is not None:
                us = timer(name, (cfg, ks), us)
            if best is None or us < best[0]:
                best = (us, cfg, ks)
            del m
        if best is not None:
            chosen[name] = best[1]
            if name == "pred":
                chosen["ksplit"] = best[2]
    return chosen


def _probe_group(what, outs, refs) -> list[str]:
    """The probe on every tensor of a group (states, errors or weight deltas
    of all layers), each scaled by the group's largest reference magnitude so
    that the tolerances are relative to the quantity's size; the layers above
    the forward initialisation's wavefront have errors and deltas of rounding
    size only, which the group scale keeps from failing on noise."""
    scale = max((float(r.abs().max()) for r in refs if r.numel()), default=0.0) or 1.0
    out = []
    for l, (o, r) in enumerate(zip(outs, refs)):
        ok, why = probe(o / scale, r / scale)
        if not ok:
            out.append(f"{what}[{l}]: {why}")
    return out


def nat_phase(name: str) -> int:
    return {"pred": 0, "infer": 1, "weight": 2}[name]


def tune_execution(dims, B: int, activation: str, dtype: torch.dtype, *, steps: int = 4, replays: int = 50,
                   seed: int = 0, wide_config=None, rejected: list | None = None, perturb=None,
                   timer=None) -> tuple[dict, list[dict]]:
    """Best (path, recompute, graph, resident row blocks) for one step, and
    every trial.  Each candidate first runs one step from the forward
    initialisation and must pass the probe (states, errors, weight deltas)
    against a float32 torch step; ``perturb(trial, model)`` (tests) may alter
    its state before the probe, ``timer(trial, step_ms)`` replace a time."""
    dev = torch.device("cuda", torch.cuda.current_device())
    w0 = init_weights_cpu(dims, seed=seed, init="xavier_uniform")
    g = torch.Generator().manual_seed(seed + 7919)
    x_in = torch.rand((dims[-1], B), generator=g).to(dev)
    y = torch.nn.functional.one_hot(torch.randint(0, dims[0], (B,), generator=g), dims[0]).float().T.contiguous().to(dev)
    act = get_activation(activation)
    L = len(dims) - 1
    trials = []
    for path in ("resident", "narrow", "wide", "phased"):
        for rows in (RESIDENT_ROWS if path == "resident" else (None,)):
            for recompute in (True, False):
                for graph in (True, False):
                    trial = {"path": path, "recompute_activation": recompute, "use_cuda_graph": graph,
                             "grid_z_max_layers": 1}
                    if rows is not None:
                        trial["resident_rows"] = rows
                    cfg = IPCConfig(dims=tuple(dims), activation=activation, dtype=dtype, fused=path,
                                    recompute_activation=recompute, hierarchical_policy_auto=False,
                                    wide_config=wide_config if path == "wide" else None, resident_rows=rows)
                    try:
                        m = HipIPC(cfg, device=dev, weights=w0)
                        m.initialize_batch(x_in, y)
                    except (ValueError, nat.IPCNativeError):
                        continue  # path (or row-block size) not eligible for this net
                    x0 = [t.clone() for t in m.x]
                    m.run_steps(1)
                    m.check_steps()
                    if perturb is not None:
                        perturb(trial, m)
                    ref_x, ref_e, ref_w = _torch_step(x0, [w.to(dev) for w in w0], act)
                    fails = _probe_group("x", m.x[1:L], ref_x[1:L]) + _probe_group("eps", m.e[:L], ref_e) + \
                        _probe_group("dW", [m.w[l] - w0[l].to(dev) for l in range(L)],
                                     [rw - w.to(dev) for rw, w in zip(ref_w, w0)])
                    if fails:
                        if rejected is not None:
                            rejected.append(dict(trial, reason="; ".join(fails)))
                        del m
                        continue
                    for l, w in enumerate(w0):
                        m.w[l].copy_(w.to(dev))
                    m.prepare_steady_state(x_in, y, steps=steps, use_graph=graph)
                    m.run_prepared_steady_state(steps=steps, repeats=3, use_graph=graph)
                    t0 = time.perf_counter()
                    m.run_prepared_steady_state(steps=steps, repeats=replays, use_graph=graph)
                    dt = time.perf_counter() - t0
                    step_ms = dt * 1e3 / (steps * replays)
                    if timer is not None:
                        step_ms = timer(trial, step_ms)
                    trials.append(dict(trial, step_ms=step_ms, samples_per_s=B / step_ms * 1e3, status="ok",
                                       source="gpu"))
                    del m
    best = min(trials, key=lambda t: t["step_ms"])
    return best, trials


def write_policy(path: str | Path, dims, B: int, activation: str, dtype: torch.dtype, table: TuningTable,
                 best: dict, trials: list[dict], *, wide_config: dict | None = None,
                 rejected: list | None = None) -> dict:
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
    best = dict(best, depth=len(dims) - 2)
    if wide_config is not None:
        best["wide_config"] = dict(wide_config)
    data["execution_entries"] = [r for r in data["execution_entries"] if not same(r)] + [
        {"dims": list(dims), "batch": B, "activation": activation, "dtype": dt, "kernel_signature": sig,
         "best": best, "candidates": trials, "rejected": list(rejected or []), "fidelity": "full"}]
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
    ap.add_argument("--no-kernels", action="store_true", help="skip the standalone kernel table")
    ap.add_argument("--standalone", default="",
                    help="semicolon-separated M,K,B points: tune the 16-bit-storage operator calls at those "
                         "shapes (the per-kernel sweep) into --table, and nothing else")
    a = ap.parse_args(argv)
    dims = [int(v) for v in a.dims.split(",")]
    dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16}[a.dtype]
    rejected: list = []
    if a.standalone:
        points = [tuple(int(v) for v in pt.split(",")) for pt in a.standalone.split(";") if pt]
        table = tune_standalone(points, a.activation, dtype, rejected=rejected)
        table.to_json(a.table, device=torch.cuda.get_device_name(0))
        print(json.dumps({"table": a.table, "kernels": len(table.entries), "rejected": len(rejected),
                          "tiles": {f"{e.key.kind} {e.key.M}x{e.key.K}x{e.key.B}": e.config.tile
                                    for e in table.entries}}), flush=True)
        return 0
    table = TuningTable.from_entries([]) if a.no_kernels else \
        tune_kernels(dims, a.batch, a.activation, dtype, rejected=rejected)
    table.to_json(a.table, device=torch.cuda.get_device_name(0))
    wide = tune_wide(dims, a.batch, a.activation, dtype, rejected=rejected)
    wide_tuple = None if wide is None else tuple(wide[k] for k in ("pred", "infer", "weight", "ksplit"))
    best, trials = tune_execution(dims, a.batch, a.activation, dtype, steps=a.steps, wide_config=wide_tuple,
                                  rejected=rejected)
    write_policy(a.policy, dims, a.batch, a.activation, dtype, table, best, trials,
                 wide_config=wide, rejected=rejected)
    print(json.dumps({"table": a.table, "policy": a.policy, "kernels": len(table.entries), "wide": wide,
                      "rejected": len(rejected), "best": best}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
