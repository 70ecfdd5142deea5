"""Benchmark of the iPC training step on one MI355X.

Workload (the headline metric's configuration): the paper efficiency profile
at depth 6, dims (10, 64 x 6, 784), batch 128, tanh, alpha=1e-4, gamma=0.5,
fp32 master states/weights with fp16 GEMM operands and fp32 accumulation,
T=4 steps captured for replay (``prepare_steady_state(use_graph=True)``: for
this plan the T steps are one launch of the layer-resident whole-step kernel,
which the capture records and each replay relaunches).  A "step" is one iPC step (prediction
errors, inference updates, weight updates) over the batch; ``value`` is
batch * steps / elapsed with inputs resident in HBM.

The same run also reports
* each phase kernel's average duration (HIP events around a graph of
  back-to-back launches of that kernel on its stream) and the roofline of the
  dominant one;
* the wide MFMA-bound configuration (1000, 4096 x 4, 4096), batch 1024, bf16
  operands: ms/step and achieved TFLOP/s against the bf16 dense MFMA peak;
* the CPU baseline: the oracle's fp32 step on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-wide] [--no-cpu]
       python bench.py --wide-only | --sweep | --small-batch | --copy-calibration
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "iPC train samples/sec (L=6,h=64,B=128); fused-GEMM TFLOP/s vs MFMA peak"
# HBM bytes that one launch of the dominant kernel moved in a profiling pass
# (not measured by this run): rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes
# (one counter per pass) over `bench.py --no-cpu --no-wide`, each scaled by
# the same counter's reading for a plain device copy of known size
# (`bench.py --copy-calibration`: FETCH_SIZE x 2.0, WRITE_SIZE x 1.0).  Keyed
# by kernel: (bytes, the profile summary that records the pass, the commit of
# the source it measured; the resident figure is the fp16 unsplit-operand
# build that the trainer runs by default).
MEASURED_TRAFFIC = {
    "layer-resident whole-step kernel, 4 steps per launch":
        (4_299_264 + 3_373_504, "profiles/resident_whole_step_d6_h64_B128.md", "3d2f799"),
    "whole-step kernel, 4 steps per launch":
        (13_065_152 + 3_926_848, "profiles/narrow_whole_step_d6_h64_B128.md", "8dc03d3"),
}
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense, no sparsity
FP16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def step_bytes(dims, B, s=4):
    """Algorithmic HBM bytes of one iPC step at storage size s: W read and
    written, hidden states read and written, target and input read
    (s * [2S + 2 sum_hidden d B + (d_0 + d_L) B]); eps stays on chip."""
    L = len(dims) - 1
    S = sum(dims[l] * dims[l + 1] for l in range(L))
    hidden = sum(dims[l] for l in range(1, L))
    return s * (2 * S + 2 * hidden * B + (dims[0] + dims[L]) * B)


def host_cpu():
    """CPU model and core counts of this host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return {"cpu_model": model, "host_logical_cpus": os.cpu_count(), "cpus_available_to_process": avail}


def phase_bytes_flops(dims, B, s=4):
    """Algorithmic HBM bytes and GEMM flops of each phase launch (P, I, W)."""
    L = len(dims) - 1
    pb = sum(s * (dims[l] * dims[l + 1] + dims[l + 1] * B + 2 * dims[l] * B) for l in range(L))
    ib = sum(s * (dims[l - 1] * dims[l] + dims[l - 1] * B + 3 * dims[l] * B) for l in range(1, L))
    wb = sum(s * (2 * dims[l] * dims[l + 1] + dims[l] * B + dims[l + 1] * B) for l in range(L))
    S = sum(dims[l] * dims[l + 1] for l in range(L))
    S_I = S - dims[L - 1] * dims[L]
    return {"pred": (pb, 2 * B * S), "infer": (ib, 2 * B * S_I), "weight": (wb, 2 * B * S)}


def make_model(dims, B, act, dtype, seed, input_dist="uniform"):
    import torch

    from lich_amd.trainer import HipIPC, IPCConfig, init_weights_cpu

    w0 = init_weights_cpu(dims, seed=seed, init="xavier_uniform")
    g = torch.Generator().manual_seed(seed + 7919)
    x_in = torch.rand((dims[-1], B), generator=g) if input_dist == "uniform" else torch.randn((dims[-1], B), generator=g)
    labels = torch.randint(0, dims[0], (B,), generator=g)
    y = torch.nn.functional.one_hot(labels, dims[0]).float().T.contiguous()
    dev = torch.device("cuda", 0)
    model = HipIPC(IPCConfig(dims=tuple(dims), activation=act, dtype=dtype, alpha=1e-4, gamma=0.5),
                   device=dev, weights=w0)
    return model, x_in.to(dev), y.to(dev)


def time_phases(model, reps=50, replays=5):
    """Average duration of one launch of each phase kernel, from HIP events
    recorded on the stream the kernels run on, around graph replays of `reps`
    back-to-back launches."""
    import torch

    from lich_amd import _native as nat

    out = {}
    # a whole-step plan's single-phase launches run on the column-block kernel
    phases = ((0, "column_kernel_phaseA_pred+infer"), (2, "column_kernel_phaseB_weight")) if model.fused else \
        ((0, "pred"), (1, "infer"), (2, "weight"))
    for phase, name in phases:
        graph = torch.cuda.CUDAGraph()
        nat.check(nat.lib().ipc_plan_phase(model._plan, phase, 2, nat.current_stream_handle()))  # warm
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            nat.check(nat.lib().ipc_plan_phase(model._plan, phase, reps, nat.current_stream_handle()))
        graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
        end.synchronize()
        out[name] = start.elapsed_time(end) * 1e3 / (reps * replays)  # microseconds per launch
        del graph
    return out


def time_step_launch(model, T, reps=50, replays=5):
    """Average duration of one T-step launch of a whole-step plan, from HIP
    events on the launch stream around graph replays of `reps` back-to-back
    launches (the graph launch itself amortised, as rocprof's kernel trace
    measures it)."""
    import torch

    from lich_amd import _native as nat

    graph = torch.cuda.CUDAGraph()
    nat.check(nat.lib().ipc_plan_step(model._plan, T, nat.current_stream_handle()))  # warm
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            nat.check(nat.lib().ipc_plan_step(model._plan, T, nat.current_stream_handle()))
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    end.synchronize()
    del graph
    return start.elapsed_time(end) * 1e3 / (reps * replays)


def run_steady(model, x, y, T, warmup_steps, steps):
    """Replays the captured T steps (prepare_steady_state with use_graph=True); returns (wall seconds, steps done, GPU
    microseconds per replay from HIP events on the replay stream)."""
    import torch

    assert model.prepare_steady_state(x, y, steps=T, use_graph=True)
    runner = model._steady_state_runner
    # at least `warmup_steps` steps, in whole replays of the T captured steps
    runner.replay(max(1, -(-warmup_steps // T)))
    replays = steps // T
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    runner.replay(replays)  # the replays, enqueued by one library call
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    model.check_steps()  # raises if a whole-step launch gave up a wait (outside the timed region)
    # GPU time per replay from HIP events, in a pass of its own after the
    # timed one (the event records would otherwise sit in the timed region)
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    runner.replay(replays)
    end.record(stream)
    end.synchronize()
    model.check_steps()
    return wall, replays * T, start.elapsed_time(end) * 1e3 / replays


def cpu_baseline(dims, B, act, threads, warmup=20, steps=200, repeats=5):
    """The oracle's fp32 step (reference.py:42-59 semantics) on the host cores."""
    import torch

    from oracle import ipc_oracle as O

    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        w = O.init_weights(dims, seed=0, init="xavier_uniform")
        x_in, _l, y = O.make_batch(dims, B, seed=0)
        x = O.forward_init(x_in, y, w, act)
        with torch.no_grad():
            for _ in range(warmup):
                x, w, _e, _m = O.ipc_step(x, w, act=act, alpha=1e-4, gamma=0.5)
            per_step = []
            for _ in range(repeats):
                t0 = time.perf_counter()
                for _ in range(steps):
                    x, w, _e, _m = O.ipc_step(x, w, act=act, alpha=1e-4, gamma=0.5)
                per_step.append((time.perf_counter() - t0) / steps)
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(per_step)
    return B / med, med


def sweep_point_bytes_flops(kind, M, K, B, save=False, s=2):
    """Algorithmic HBM bytes and GEMM flops of one standalone kernel launch at
    storage size s: P s(MK+KB+2MB), I s(MK+KB+3MB) (+MB with A_out),
    W s(2MK+MB+KB)."""
    flops = 2 * M * K * B
    if kind == "pred":
        return s * (M * K + K * B + 2 * M * B), flops
    if kind == "infer":
        return s * (M * K + K * B + 3 * M * B + (M * B if save else 0)), flops
    return s * (2 * M * K + M * B + K * B), flops


def time_launch(fn, reps, replays=3, graph=True):
    """Microseconds per call of `fn` (its launches on the current stream), from
    HIP events around graph replays of `reps` back-to-back calls, or around
    `reps * replays` direct calls (graph=False)."""
    import torch

    fn()
    torch.cuda.synchronize()
    if not graph:
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps * replays):
            fn()
        end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) * 1e3 / (reps * replays)
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
    us = start.elapsed_time(end) * 1e3 / (reps * replays)
    del graph
    return us


def kernel_sweep(sizes=(1024, 4096, 8192), batches=(256, 2048, 8192), acts=("tanh", "relu")):
    """Per-kernel roofline sweep: prediction+error, transposed inference update
    and weight update, each standalone at M=K in `sizes`, B in `batches`, bf16
    storage and operands (fp32 accumulation), W ~ N(0, 1/K), states and errors
    ~ N(0, 1), tanh/relu fused; the inference update with and without the saved
    activation output, the weight update recomputing f(X) and reading a saved
    A.  Each point's bound is min(MFMA peak, AI x HBM peak).  Each call is timed
    as the allocation-free default and, where a caller workspace lets it
    evaluate f(X) once, with one (``*_workspace`` fields)."""
    import torch

    from lich_amd import kernels as K_

    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(0)
    bf = torch.bfloat16
    rows = []
    for n in sizes:
        for B in batches:
            M = K = n
            w = (torch.randn((M, K), generator=g) / K ** 0.5).to(dev, bf)
            xu = torch.randn((K, B), generator=g).to(dev, bf)
            xl = torch.randn((M, B), generator=g).to(dev, bf)
            e = torch.randn((M, B), generator=g).to(dev, bf)
            el = torch.randn((K, B), generator=g).to(dev, bf)
            aout = torch.empty((M, B), device=dev, dtype=bf)
            big = 2 * M * K * B > 2e11
            reps = 3 if big else (10 if 2 * M * K * B > 1e10 else 50)
            ws_buf = None  # the caller workspace of the pre-activating calls, allocated once per shape
            for act in acts:
                kp = K_.build_prediction_error(M, K, B, act, bf)
                cases = [("pred", False, kp)]
                for save in (False, True):
                    cases.append(("infer", save, K_.build_inference_update(M, K, B, act, bf, None, 0.5, save)))
                for rec in (True, False):
                    cases.append(("weight", not rec, K_.build_weight_update(M, K, B, act, bf, None, 1e-4, rec)))
                wl = w  # W_lower is [K, M]; M == K here

                def call(kind, save, kern, ws=None):
                    if kind == "pred":
                        return lambda: kern(xu, w, xl, e, workspace=ws)
                    if kind == "infer":
                        return lambda: kern(xl, e, wl, el, aout if save else None, workspace=ws)
                    return lambda: kern(w, e, xu, workspace=ws)

                for kind, save, kern in cases:
                    # the default call (no workspace: f(X) in every row tile's
                    # loader, the inference update's operands read transposed;
                    # the library allocates nothing) and, where the call would
                    # use one (f(X) evaluated once, or the inference update's
                    # operands copied transposed), the caller-workspace call
                    us = time_launch(call(kind, save, kern), reps)
                    need = kern.workspace_bytes
                    us_ws = None
                    if need > 0:
                        if ws_buf is None or ws_buf.numel() < need:
                            ws_buf = torch.empty((need,), dtype=torch.uint8, device=dev)
                        us_ws = time_launch(call(kind, save, kern, ws_buf), reps)
                    nbytes, flops = sweep_point_bytes_flops(kind, M, K, B, save=save and kind == "infer")
                    ai = flops / nbytes
                    attain = min(BF16_PEAK_TFLOPS, ai * HBM_PEAK_GBS / 1e3)
                    tf = flops / (us * 1e-6) / 1e12
                    row = {"kernel": kind, "M": M, "K": K, "B": B, "act": act,
                           "variant": ("save A_out" if save else "no A_out") if kind == "infer" else
                           (("saved A" if save else "recompute f(X)") if kind == "weight" else "-"),
                           "us": round(us, 2), "TFLOP/s": round(tf, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                           "AI": round(ai, 1), "bound": "mfma" if attain >= BF16_PEAK_TFLOPS else "hbm",
                           "attainable_TFLOP/s": round(attain, 1), "frac": round(tf / attain, 4),
                           "timing": "graph replays, no workspace"}
                    if us_ws is not None:
                        tfw = flops / (us_ws * 1e-6) / 1e12
                        row.update({"us_workspace": round(us_ws, 2), "TFLOP/s_workspace": round(tfw, 2),
                                    "frac_workspace": round(tfw / attain, 4)})
                    rows.append(row)
                    log(f"sweep: {row}")
            del w, xu, xl, e, el, aout, ws_buf
            torch.cuda.empty_cache()
    return rows


def wide_config(T):
    """The MFMA-bound wide configuration (1000, 4096 x 4, 4096), B=1024, bf16
    operands: ms/step, TFLOP/s, per-phase launch times and the roofline of the
    dominant phase kernel."""
    import torch

    wdims = (1000,) + (4096,) * 4 + (4096,)
    WB = 1024
    wmodel, wx, wy = make_model(wdims, WB, "tanh", torch.bfloat16, seed=0, input_dist="normal")
    w_elapsed, w_done, _w_replay_us = run_steady(wmodel, wx, wy, T, 2 * T, 5 * T)
    w_ms = w_elapsed * 1e3 / w_done
    flops_step = sum(v[1] for v in phase_bytes_flops(wdims, WB).values())
    tflops = flops_step / (w_ms * 1e-3) / 1e12
    wphase = time_phases(wmodel, reps=5, replays=3)
    wbf = phase_bytes_flops(wdims, WB)
    wphases = {k: {"us": round(v, 2), "TFLOP/s": round(wbf[k][1] / (v * 1e-6) / 1e12, 2)}
               for k, v in wphase.items()}
    wdom = max(wphase, key=wphase.get)
    wide = {"workload": "wide iPC MLP dims (1000,4096x4,4096), B=1024, tanh, bf16 operands, fp32 master, T=4",
            "path": wmodel.path, "pred_split": wmodel.pred_split,
            "ms_per_step": round(w_ms, 4), "samples_per_s": round(WB / (w_ms * 1e-3), 1),
            "gflop_per_step": round(flops_step / 1e9, 3), "tflops": round(tflops, 2),
            "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
            "phases": wphases,
            # the dominant phase kernel against the dense bf16 MFMA peak
            "roofline": {"bound": "mfma", "kernel": f"wide {wdom} phase", "achieved": wphases[wdom]["TFLOP/s"],
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(wphases[wdom]["TFLOP/s"] / BF16_PEAK_TFLOPS, 4),
                         "algorithmic_flops_per_launch": wbf[wdom][1], "avg_launch_us": wphases[wdom]["us"]}}
    log(f"wide: {wide}")
    del wmodel

    return wide


def small_batch_config():
    """The small-batch online configuration (10, 64^4, 784), fp32, tanh, T=8,
    B in {1, 4, 8}, next to the oracle's fp32 step on the host cores."""
    import torch

    dims, T = (10,) + (64,) * 4 + (784,), 8
    rows = []
    threads = torch.get_num_threads()
    for B in (1, 4, 8):
        model, x, y = make_model(dims, B, "tanh", torch.float32, seed=B)
        el, done, replay_us = run_steady(model, x, y, T, 800, 40000)
        # the oracle on all host cores and on one (these matrices are small enough for
        # thread start-up to dominate); the faster of the two is the baseline
        cpu = [cpu_baseline(dims, B, "tanh", n, warmup=20, steps=400, repeats=5) + (n,) for n in (threads, 1)]
        cpu_val, cpu_step, cpu_cores = max(cpu)
        gpu_val = done * B / el
        rows.append({"B": B, "path": model.path, "launches_per_step": model.launches_per_step(),
                     "us_per_step": round(el * 1e6 / done, 3), "us_per_replay": round(replay_us, 2),
                     "samples_per_s": round(gpu_val, 1), "cpu_samples_per_s": round(cpu_val, 1),
                     "cpu_us_per_step": round(cpu_step * 1e6, 2), "cpu_cores": cpu_cores,
                     "cpu_samples_per_s_by_cores": {str(n): round(v, 1) for v, _s, n in cpu},
                     "gpu_over_cpu": round(gpu_val / cpu_val, 2)})
        del model
    return {"workload": "small-batch online iPC MLP dims (10, 64x4, 784), fp32, tanh, T=8 steps per graph replay, "
                        "rank-B outer-product weight update",
            "data": "synthetic (seeded U[0,1] inputs, uniform labels, Xavier W)",
            "cpu_kind": "port (oracle fp32 step on the host cores)", "rows": rows}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-wide", action="store_true", help="skip the wide and small-batch configurations")
    ap.add_argument("--wide-only", action="store_true",
                    help="run only the wide configuration and print its JSON object")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep", action="store_true",
                    help="run only the per-kernel roofline sweep (M=K in {1024,4096,8192}, "
                         "B in {256,2048,8192}, bf16) and print it as one JSON line")
    ap.add_argument("--small-batch", action="store_true",
                    help="run only the small-batch online configuration (10, 64^4, 784), fp32, tanh, T=8, "
                         "B in {1,4,8}, next to the oracle's fp32 step on the host cores, as one JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of a known size (the reference point that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2
    if args.small_batch:
        print(json.dumps({"small_batch": small_batch_config()}), flush=True)
        return 0
    if args.copy_calibration:
        import torch

        nbytes = 256 << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read_per_copy": nbytes, "bytes_written_per_copy": nbytes,
                                               "copies": 10}}), flush=True)
        return 0
    if args.sweep:
        rows = kernel_sweep()
        print(json.dumps({"sweep": "per-kernel roofline, bf16 storage/operands, fp32 accumulation",
                          "peaks": {"bf16_TFLOP/s": BF16_PEAK_TFLOPS, "hbm_GB/s": HBM_PEAK_GBS},
                          "rows": rows}), flush=True)
        return 0

    import torch

    from lich_amd import _native as nat

    T = 4
    dims = (10,) + (64,) * 6 + (784,)
    B = 128
    steps = max(T, (args.steps // T) * T)
    warmup = max(T, args.warmup)
    log(f"device {torch.cuda.get_device_name(0)} arch {nat.device_arch(0)}")

    if args.wide_only:
        print(json.dumps({"wide": wide_config(T)}), flush=True)
        return 0
    # The kernel-level figures first (HIP events around back-to-back launches
    # of a separate model); the headline's timed region follows them.
    bf = phase_bytes_flops(dims, B)
    per_step_bytes = step_bytes(dims, B, s=4)
    step_flops = sum(v[1] for v in bf.values())
    # per-phase kernel durations on a fresh model (the timing loops disturb state)
    pmodel, px, py = make_model(dims, B, "tanh", torch.float16, seed=1)
    pmodel.initialize_batch(px, py)
    phase_us = time_phases(pmodel)
    phases = {k: {"us": round(v, 3)} for k, v in phase_us.items()}
    log(f"phases: {phases}")
    if pmodel.fused:
        # the dominant (only) kernel is a whole-step kernel, one launch per
        # T-step replay; its duration is timed over back-to-back launches
        launch_us = time_step_launch(pmodel, T)
        name = "layer-resident whole-step kernel" if pmodel.path == "resident" else "whole-step kernel"
        kernel = f"{name}, {T} steps per launch"
        launch_bytes, launch_flops = T * per_step_bytes, T * step_flops
    else:
        dom = max(phase_us, key=phase_us.get)
        launch_us = phase_us[dom]
        kernel = f"{dom} phase"
        launch_bytes, launch_flops = bf[dom]
    achieved = launch_bytes / (launch_us * 1e-6) / 1e9
    traffic, traffic_src, traffic_commit = MEASURED_TRAFFIC.get(kernel, (None, None, None))
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic, "kernel": kernel,
                "traffic_source": (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes, {traffic_src}, kernel source "
                                   f"at commit {traffic_commit}") if traffic_src else None,
                "algorithmic_bytes_per_launch": launch_bytes,
                "algorithmic_bytes_rule": f"{per_step_bytes} B per step (storage s=4: 2S + 2 sum_hidden d B + "
                                          f"(d_0+d_L) B) x {T if pmodel.fused else 1} steps per launch",
                "avg_launch_us": round(launch_us, 3),
                "achieved_tflops": round(launch_flops / (launch_us * 1e-6) / 1e12, 4)}
    pmodel_fused = pmodel.fused
    del pmodel

    model, x, y = make_model(dims, B, "tanh", torch.float16, seed=0)
    elapsed, done, replay_us = run_steady(model, x, y, T, warmup, steps)
    ms_per_step = elapsed * 1e3 / done
    value = B * done / elapsed
    log(f"headline: {ms_per_step * 1e3:.2f} us/step, {value:,.0f} samples/s, path={model.path}, "
        f"{model.launches_per_step()} launch(es) per step call, {replay_us:.2f} us per {T}-step replay")

    wide = None if args.no_wide else wide_config(T)
    # the small-batch configuration times the host oracle as well: skipped with --no-cpu
    small = None if args.no_wide or args.no_cpu else small_batch_config()

    cpu = None
    if not args.no_cpu:
        threads = torch.get_num_threads()
        cpu_val, cpu_step = cpu_baseline(dims, B, "tanh", threads)
        cpu1_val, _ = cpu_baseline(dims, B, "tanh", 1, warmup=10, steps=100, repeats=3)
        cpu = {"value": round(cpu_val, 1), "unit": "samples/s", "cores": threads, "kind": "port", **host_cpu(),
               "sample": f"oracle fp32 step, same dims/B/tanh, 20 warm-up + 5x200 timed steps, median "
                         f"({cpu_step * 1e3:.3f} ms/step); 1 thread: {cpu1_val:.1f} samples/s",
               "gpu_over_cpu": round(value / cpu_val, 2)}
        log(f"cpu: {cpu}")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "samples/s", "n_gpus": 1, "steps": done,
        "warmup": warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic (seeded U[0,1] inputs, uniform labels, Xavier W)",
        "config": {"workload": "paper profile depth 6: dims (10,64x6,784), B=128, tanh, alpha=1e-4, gamma=0.5, "
                               "T=4 steps per replay of the captured steps (one whole-step kernel launch), fp32 master x/eps/W, "
                               "fp16 operands, fp32 accumulate",
                   "global_batch": B, "seq_len": None, "parallelism": "single GPU",
                   "fused_whole_step_kernel": model.fused, "path": model.path, "phases": phases,
                   "replay_forms": {
                       "direct_relaunch_us_per_step": round(ms_per_step * 1e3, 4),
                       "hipgraph_replay_us_per_step": round(launch_us / T, 4) if pmodel_fused else None,
                       "note": "headline: the captured T steps replayed by relaunching their one whole-step "
                               "launch; hipgraph: the same launch recorded 50 times into a torch.cuda.graph, "
                               "HIP events around its replays"}},
        "roofline": roofline, "cpu_baseline": cpu, "wide": wide, "small_batch": small,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
