"""Command-line drop-in for the reference's ``scripts/run_cli.py:20-41``.

    python -m lich_amd.cli smoke [--M 64 --K 64 --B 128 --activation relu]
    python -m lich_amd.cli reference [--depth 3 --hidden 64 --batch 8 --steps 5]
    python -m lich_amd.cli autotune --dims 10,64,64,64,784 [...]
    python -m lich_amd.cli train-mnist [--data ./data | --synthetic 60000] [...]
    python -m lich_amd.cli efficiency --depths 3 4 6 [--graph] [...]
    python -m lich_amd.cli thermal-bench [--seconds 120 --graph] [...]
    python -m lich_amd.cli steady-state [--dims 784 64 64 10] [...]
    python -m lich_amd.cli toolchain

Each subcommand takes the arguments of the reference script it replaces
(``smoke.py``, ``validate_reference.py``, ``autotune.py``, ``train_mnist.py``,
``train_paper_efficiency.py``, ``thermal_bench.py``,
``benchmark_stage2_4_steady_state.py``, ``toolchain_probe.py``).  Differences:
datasets come from local IDX files (``--data``) or ``--synthetic N`` (there is
no download); the thermal guard reads ``amd-smi`` and a ``--temperature-max``
of 0 turns it off; the device gate is gfx950 instead of SM86.
"""
from __future__ import annotations

import argparse
import json
import shutil
import statistics
import subprocess
import sys
import time
from pathlib import Path

import torch


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("a GPU is required")
    return torch.device("cuda", 0)


def _dataset(a, subset: int = 0):
    from .data import load_dataset, synthetic_dataset

    if a.synthetic:
        ds = synthetic_dataset(a.synthetic, seed=getattr(a, "seed", 0))
        return ds.subset(subset) if subset else ds
    return load_dataset(a.data, a.dataset, train=True, subset=subset)


# ------------------------------------------------------------------ smoke
def smoke_main(argv=None) -> int:
    """Kernel smoke of ``scripts/smoke.py:10-67``: prediction + error, the
    inference update and the weight update (recomputed and saved activation)
    with 16-bit storage against torch on the device, plus the 10-row tail of
    the paper profile's output layer."""
    from .kernels import build_inference_update, build_prediction_error, build_weight_update
    from .reference import get_activation

    p = argparse.ArgumentParser(prog="lich_amd.cli smoke")
    p.add_argument("--M", type=int, default=64)
    p.add_argument("--K", type=int, default=64)
    p.add_argument("--B", type=int, default=128)
    p.add_argument("--activation", default="relu")
    a = p.parse_args(argv)
    dev, h = _device(), torch.float16
    act = get_activation(a.activation)
    f = lambda t: act.forward(t.float())  # noqa: E731
    g = torch.Generator(device=dev).manual_seed(0)
    rn = lambda *s: torch.randn(s, generator=g, device=dev, dtype=h)  # noqa: E731
    x_up, w, x_lo = rn(a.K, a.B), rn(a.M, a.K) * 0.05, rn(a.M, a.B)
    e = torch.empty_like(x_lo)
    build_prediction_error(a.M, a.K, a.B, a.activation, h)(x_up, w, x_lo, e)
    torch.cuda.synchronize()
    ref_e = x_lo.float() - w.float() @ f(x_up)
    torch.testing.assert_close(e.float(), ref_e, rtol=2e-2, atol=2e-2)

    x = x_lo.clone()
    e_low = rn(a.K, a.B)
    w_low = rn(a.K, a.M) * 0.05  # W_{l-1}: [K, M], read transposed
    build_inference_update(a.M, a.K, a.B, a.activation, h, None, 0.5)(x, e, w_low, e_low)
    torch.cuda.synchronize()
    ref_x = x_lo.float() + 0.5 * (-e.float() + act.derivative(x_lo.float()) * (w_low.float().T @ e_low.float()))
    torch.testing.assert_close(x.float(), ref_x, rtol=3e-2, atol=3e-2)

    alpha = 1e-4
    w2 = w.clone()
    build_weight_update(a.M, a.K, a.B, a.activation, h, None, alpha, True)(w2, e, x_up)
    torch.cuda.synchronize()
    ref_w = w.float() + alpha * (e.float() @ f(x_up).T)
    torch.testing.assert_close(w2.float(), ref_w, rtol=2e-2, atol=2e-2)

    m2, k2 = 10, 64  # the paper profile's 10-class output layer
    xu2, ws, xs = rn(k2, a.B), rn(m2, k2) * 0.05, rn(m2, a.B)
    es = torch.empty_like(xs)
    build_prediction_error(m2, k2, a.B, a.activation, h)(xu2, ws, xs, es)
    ws2 = ws.clone()
    build_weight_update(m2, k2, a.B, a.activation, h, None, alpha, True)(ws2, es, xu2)
    torch.cuda.synchronize()
    torch.testing.assert_close(es.float(), xs.float() - ws.float() @ f(xu2), rtol=3e-2, atol=3e-2)
    torch.testing.assert_close(ws2.float(), ws.float() + alpha * (es.float() @ f(xu2).T), rtol=2e-2, atol=2e-2)

    w3 = w.clone()
    build_weight_update(a.M, a.K, a.B, a.activation, h, None, alpha, False)(w3, e, f(x_up).to(h).contiguous())
    torch.cuda.synchronize()
    torch.testing.assert_close(w3.float(), ref_w, rtol=2e-2, atol=2e-2)
    print("MI355X HIP kernel smoke test: PASS (regular + tail-safe + save-A paths)", flush=True)
    return 0


# ------------------------------------------------------------------ reference
def reference_main(argv=None) -> int:
    """CPU trajectory of ``scripts/validate_reference.py:13-35``: the pure
    PyTorch fp32 step from a forward-initialised state."""
    from . import reference as R

    p = argparse.ArgumentParser(prog="lich_amd.cli reference")
    p.add_argument("--depth", type=int, default=3)
    p.add_argument("--hidden", type=int, default=64)
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--steps", type=int, default=5)
    p.add_argument("--activation", default="relu")
    a = p.parse_args(argv)
    # the script's random stream: one global seed, then the input, then the
    # weights layer by layer from the same global generator
    torch.manual_seed(0)
    dims = (10,) + (a.hidden,) * a.depth + (28 * 28,)
    f32 = torch.float32
    x_in = torch.randn((dims[-1], a.batch), dtype=f32)
    y = R.one_hot(torch.arange(a.batch) % 10, 10, dtype=f32)
    w = []
    for rows, cols in zip(dims[:-1], dims[1:]):
        t = torch.empty((rows, cols), dtype=f32)
        torch.nn.init.kaiming_uniform_(t, a=5 ** 0.5)
        w.append(t)
    act = R.get_activation(a.activation)
    x = [torch.zeros((d, a.batch), dtype=f32) for d in dims]
    x[-1].copy_(x_in)
    for l in reversed(range(1, len(w))):  # forward initialisation of the hidden states
        x[l].copy_(w[l] @ act.forward(x[l + 1]))
    x[0].copy_(y)
    st = R.ReferenceState(x=x, w=w)
    for i in range(a.steps):
        st, m = R.ipc_step(st, act=act, alpha=1e-4, gamma=0.5, fixed_low=y, fixed_high=x_in)
        print(i, float(m["energy"]), float(m["max_abs_error"]), flush=True)
    print("Reference iPC trajectory computed successfully.", flush=True)
    return 0


# ------------------------------------------------------------------ efficiency
def efficiency_main(argv=None) -> int:
    """Paper efficiency profile of ``scripts/train_paper_efficiency.py:19-96``:
    for each depth, epochs over a subset, one JSONL row per epoch.  Rows carry
    both throughput definitions: examples per second (each example once per
    batch, the script's own) and iPC-step samples per second (batch x steps
    per batch, the published per-step figure)."""
    from .telemetry import ThermalGuard
    from .trainer import IPCConfig, TileLangIPC, prepare_batch

    p = argparse.ArgumentParser(prog="lich_amd.cli efficiency")
    p.add_argument("--dataset", choices=["MNIST", "FashionMNIST"], default="MNIST")
    p.add_argument("--data", default="./data")
    p.add_argument("--synthetic", type=int, default=0, help="N seeded synthetic samples instead of IDX files")
    p.add_argument("--hidden", type=int, default=64)
    p.add_argument("--depth", type=int, choices=[3, 4, 6], default=None)
    p.add_argument("--depths", type=int, nargs="+", choices=[3, 4, 6], default=None)
    p.add_argument("--batch", type=int, default=128)
    p.add_argument("--epochs", type=int, default=1)
    p.add_argument("--steps", type=int, default=1)
    p.add_argument("--subset", type=int, default=250)
    p.add_argument("--out", default="results/paper_efficiency.jsonl")
    p.add_argument("--temperature-max", type=float, default=76.0, help="0 turns the guard off")
    p.add_argument("--thermal-poll", type=float, default=0.5)
    p.add_argument("--graph", action="store_true")
    p.add_argument("--save-activation", action="store_true")
    p.add_argument("--activation", default="relu")
    p.add_argument("--seed", type=int, default=0)
    a = p.parse_args(argv)
    dev = _device()
    depths = a.depths if a.depths is not None else ([a.depth] if a.depth is not None else [4])
    ds = _dataset(a, subset=a.subset)
    guard = ThermalGuard(max_temp_c=a.temperature_max, poll_s=a.thermal_poll) if a.temperature_max > 0 else None
    out = Path(a.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    with out.open("a", encoding="utf-8") as fh:
        for depth in depths:
            dims = (ds.num_classes,) + (a.hidden,) * depth + (ds.features,)
            model = TileLangIPC(IPCConfig(dims=dims, alpha=1e-4, gamma=0.5, activation=a.activation,
                                          dtype=torch.float16, recompute_activation=not a.save_activation),
                                device=dev, seed=a.seed)
            runner = None
            for epoch in range(a.epochs):
                t0 = time.perf_counter()
                examples = 0
                for images, labels in ds.batches(a.batch, shuffle=False, drop_last=True):
                    if guard is not None:
                        guard.wait_until_safe(verbose=True)
                    x, y = prepare_batch(images, labels, device=dev, dtype=torch.float32, num_classes=ds.num_classes)
                    model.initialize_batch(x, y)
                    if a.graph:
                        if runner is None:
                            runner = model.capture_graph(a.steps)
                        runner.replay()
                    else:
                        model.run_steps(a.steps)
                    examples += int(labels.numel())
                model.check_steps()  # synchronises; raises if a whole-step launch timed out
                dt = time.perf_counter() - t0
                t = guard.check(force=True) if guard is not None else None
                row = {"dataset": ds.name, "depth": depth, "hidden": a.hidden, "batch": a.batch, "epoch": epoch + 1,
                       "steps": a.steps, "seconds": dt, "samples_per_s": examples / max(dt, 1e-12),
                       "ipc_step_samples_per_s": examples * a.steps / max(dt, 1e-12), "path": model.path,
                       "temperature_c": None if t is None else t.temperature_c,
                       "power_w": None if t is None else t.power_w,
                       "gfx_clock_mhz": None if t is None else t.clock_gfx_mhz,
                       "throttle_reasons": None if t is None else t.throttle_status}
                fh.write(json.dumps(row) + "\n")
                fh.flush()
                print(json.dumps(row), flush=True)
            del model
    return 0


# ------------------------------------------------------------------ thermal bench
def thermal_main(argv=None) -> int:
    """Sustained throughput under the thermal guard (``scripts/thermal_bench.py:16-91``):
    one fixed batch, ``--steps`` steps per replay for ``--seconds``, a status
    line per second and a final line with samples/s (batch x steps per
    elapsed second)."""
    from .telemetry import ThermalGuard
    from .trainer import IPCConfig, TileLangIPC, prepare_batch
    from .tuning import TuningTable

    p = argparse.ArgumentParser(prog="lich_amd.cli thermal-bench")
    p.add_argument("--hidden", type=int, default=64)
    p.add_argument("--depth", type=int, default=2)
    p.add_argument("--batch", type=int, default=128)
    p.add_argument("--steps", type=int, default=4)
    p.add_argument("--seconds", type=float, default=120.0)
    p.add_argument("--temperature-max", type=float, default=76.0, help="0 turns the guard off")
    p.add_argument("--poll", type=float, default=0.5)
    p.add_argument("--graph", action="store_true")
    p.add_argument("--save-activation", action="store_true")
    p.add_argument("--tuning", default=None, help="optional tuning table (schema 1)")
    p.add_argument("--activation", default="relu")
    a = p.parse_args(argv)
    dev = _device()
    tuning = TuningTable.from_json(a.tuning) if a.tuning else None
    dims = (10,) + (a.hidden,) * a.depth + (784,)
    model = TileLangIPC(IPCConfig(dims=dims, alpha=1e-4, gamma=0.5, activation=a.activation, dtype=torch.float16,
                                  recompute_activation=not a.save_activation, tuning_table=tuning), device=dev)
    labels = torch.arange(a.batch, dtype=torch.long).remainder(10)
    images = torch.rand((a.batch, 1, 28, 28))
    x, y = prepare_batch(images, labels, device=dev, dtype=torch.float32, num_classes=10)
    model.initialize_batch(x, y)
    runner = model.capture_graph(a.steps) if a.graph else None
    guard = ThermalGuard(max_temp_c=a.temperature_max if a.temperature_max > 0 else float("inf"), poll_s=a.poll,
                         telemetry_interval_s=1.0)
    guard.wait_until_safe(verbose=True)
    start = last = time.perf_counter()
    replays = steps = samples = 0
    while time.perf_counter() - start < a.seconds:
        guard.wait_until_safe(verbose=True)
        if runner is not None:
            runner.replay()
        else:
            model.run_steps(a.steps)
        replays += 1
        steps += a.steps
        samples += a.batch * a.steps
        now = time.perf_counter()
        if now - last >= 1.0:
            torch.cuda.synchronize()
            el = now - start
            print(f"t={el:7.1f}s replays={replays:7d} ipc_steps={steps:8d} samples/s={samples / max(el, 1e-9):10.1f} "
                  f"{guard.format_status(guard.check(force=True))}", flush=True)
            last = now
    model.check_steps()
    el = time.perf_counter() - start
    print(f"FINAL elapsed={el:.3f}s replays={replays} ipc_steps={steps} samples/s={samples / max(el, 1e-9):.1f} "
          f"{guard.format_status(guard.check(force=True))}", flush=True)
    return 0


# ------------------------------------------------------------------ steady state A/B
def steady_main(argv=None) -> int:
    """Direct vs captured steady state (``scripts/benchmark_stage2_4_steady_state.py:33-126``):
    the same prepared batch run ``repeats`` times each way, the median
    wall-clock of a block of ``steps`` steps, written as JSON."""
    from .trainer import IPCConfig, TileLangIPC

    p = argparse.ArgumentParser(prog="lich_amd.cli steady-state")
    p.add_argument("--dims", nargs="+", type=int, default=[784, 64, 64, 10])
    p.add_argument("--batch", type=int, default=128)
    p.add_argument("--steps", type=int, default=4)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--repeats", type=int, default=30)
    p.add_argument("--out", default="results/steady_state.json")
    p.add_argument("--no-policy", action="store_true")
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--activation", default="relu")
    a = p.parse_args(argv)
    dev = _device()
    g = torch.Generator().manual_seed(a.seed)
    x = torch.randn((a.dims[-1], a.batch), generator=g).to(dev)
    labels = torch.randint(0, a.dims[0], (a.batch,), generator=g)
    y = torch.nn.functional.one_hot(labels, a.dims[0]).float().T.contiguous().to(dev)
    cfg = IPCConfig(dims=tuple(a.dims), activation=a.activation, dtype=torch.float16,
                    hierarchical_policy_auto=not a.no_policy, steady_state_graph_auto=True,
                    steady_state_graph_default=False, weight_update_mode="gemm")
    model = TileLangIPC(cfg, device=dev, seed=a.seed)

    def timed(fn):
        for _ in range(a.warmup):
            fn()
        torch.cuda.synchronize()
        vals = []
        for _ in range(a.repeats):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            vals.append((time.perf_counter() - t0) * 1e3)
        return vals

    graph_active = model.prepare_steady_state(x, y, steps=a.steps, use_graph=None)
    direct = timed(lambda: model.run_prepared_steady_state(steps=a.steps, repeats=1, use_graph=False))
    graph_active = model.prepare_steady_state(x, y, steps=a.steps, use_graph=True)
    graph = timed(lambda: model.run_prepared_steady_state(steps=a.steps, repeats=1, use_graph=True))
    d_step, g_step = statistics.median(direct) / a.steps, statistics.median(graph) / a.steps
    result = {"device": torch.cuda.get_device_name(dev), "arch": model.arch, "dims": list(a.dims), "batch": a.batch,
              "steps": a.steps, "warmup": a.warmup, "repeats": a.repeats, "graph_active": bool(graph_active),
              "path": model.path, "direct_ms_block_median": statistics.median(direct),
              "graph_ms_block_median": statistics.median(graph), "direct_ms_step": d_step, "graph_ms_step": g_step,
              "graph_speedup": d_step / g_step if g_step > 0 else float("inf"),
              "direct_samples": direct, "graph_samples": graph}
    print(f"direct={d_step:.4f} ms/step graph={g_step:.4f} ms/step speedup={result['graph_speedup']:.3f}x "
          f"path={model.path}", flush=True)
    out = Path(a.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(result, indent=2), encoding="utf-8")
    print(f"Wrote {out}", flush=True)
    return 0


# ------------------------------------------------------------------ toolchain
def toolchain_main(argv=None) -> int:
    """Toolchain and device report (``scripts/toolchain_probe.py``): hipcc,
    the built library's ABI version and the device architecture."""
    from . import _native as nat

    argparse.ArgumentParser(prog="lich_amd.cli toolchain").parse_args(argv)
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    try:
        ver = subprocess.run([hipcc, "--version"], capture_output=True, text=True, timeout=60).stdout.strip()
    except (OSError, subprocess.TimeoutExpired) as exc:
        ver = f"unavailable ({exc})"
    report = {"python": sys.version.split()[0], "torch": torch.__version__, "hip": torch.version.hip,
              "hipcc": ver.splitlines()[0] if ver else None, "library": str(nat.LIB_PATH),
              "library_built": nat.LIB_PATH.exists()}
    if nat.LIB_PATH.exists():
        report["abi_version"] = int(nat.lib().ipc_abi_version())
    if torch.cuda.is_available():
        try:
            report["device_arch"] = nat.device_arch(0)
        except (nat.IPCNativeError, ValueError) as exc:
            report["device_arch"] = f"refused: {exc}"
    print(json.dumps(report, indent=2), flush=True)
    return 0


def _autotune(argv):
    from .autotune import main
    return main(argv)


def _train(argv):
    from .train import main
    return main(argv)


COMMANDS = {"smoke": smoke_main, "reference": reference_main, "autotune": _autotune, "train-mnist": _train,
            "efficiency": efficiency_main, "thermal-bench": thermal_main, "steady-state": steady_main,
            "toolchain": toolchain_main}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m lich_amd.cli", description="iPC training step on MI355X")
    p.add_argument("command", choices=sorted(COMMANDS))
    ns, extra = p.parse_known_args(argv)
    return int(COMMANDS[ns.command](extra) or 0)


if __name__ == "__main__":
    raise SystemExit(main())
