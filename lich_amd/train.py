"""Training and accuracy loop (reference ``scripts/train_mnist.py``).

    python -m lich_amd.train --data ./data --dataset MNIST --depth 2 --epochs 5 --graph
    python -m lich_amd.train --synthetic 60000 --epochs 2

Per batch: the thermal guard (``--temperature-max``), the staged batch
(``BatchStager``: pinned host slots, H2D on a side stream, one batch ahead),
``initialize_batch``, ``--steps`` iPC steps (one captured graph replay with
``--graph``, captured on the first batch), then ``predict`` and the argmax
accuracy against the labels (``train_mnist.py:79-86``).  Datasets are read
from local IDX files only (``lich_amd.data``); ``--synthetic N`` trains on the
seeded MNIST-shaped stand-in instead.
"""
from __future__ import annotations

import argparse
import json
import time

import torch

from .data import BatchStager, load_dataset, synthetic_dataset
from .telemetry import ThermalGuard
from .trainer import IPCConfig, TileLangIPC


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--data", default="./data")
    p.add_argument("--dataset", choices=["MNIST", "FashionMNIST"], default="MNIST")
    p.add_argument("--synthetic", type=int, default=0, help="train on N seeded synthetic samples instead")
    p.add_argument("--hidden", type=int, default=64)
    p.add_argument("--depth", type=int, default=2, help="number of hidden layers")
    p.add_argument("--batch", type=int, default=128)
    p.add_argument("--epochs", type=int, default=5)
    p.add_argument("--steps", type=int, default=4)
    p.add_argument("--alpha", type=float, default=1e-4)
    p.add_argument("--gamma", type=float, default=0.5)
    p.add_argument("--activation", default="relu")
    p.add_argument("--dtype", choices=["float16", "bfloat16", "float32"], default="float16",
                   help="GEMM operand type (states and weights stay fp32)")
    p.add_argument("--subset", type=int, default=0, help="0 = full train set")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--temperature-max", type=float, default=0.0, help="pause above this junction temperature (0 = off)")
    p.add_argument("--thermal-poll", type=float, default=0.5)
    p.add_argument("--graph", action="store_true", help="capture the fixed iPC step loop in a hipGraph")
    p.add_argument("--save-activation", action="store_true",
                   help="materialise f(x) for weight updates instead of recomputing it")
    p.add_argument("--json", action="store_true", help="one JSON line per epoch")
    return p.parse_args(argv)


def batch_correct(model, x: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Correct predictions of ``predict(x)`` (argmax over the class rows), as a
    device scalar: the loop adds them up on the device and synchronises once
    per epoch instead of once per batch."""
    logits = model.predict(x)                     # [classes, B]
    return (logits.float().argmax(dim=0) == labels).sum()


def batch_accuracy(model, x: torch.Tensor, labels: torch.Tensor) -> int:
    """Correct predictions of ``predict(x)`` as a host integer."""
    return int(batch_correct(model, x, labels).item())


def train(a: argparse.Namespace):
    """Runs the loop; returns (per-epoch records, the model)."""
    device = torch.device("cuda", 0)
    if a.synthetic:
        ds = synthetic_dataset(a.synthetic, seed=a.seed)
    else:
        ds = load_dataset(a.data, a.dataset, train=True, subset=a.subset)
    dims = (ds.num_classes,) + (a.hidden,) * a.depth + (ds.features,)
    op = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}[a.dtype]
    model = TileLangIPC(IPCConfig(dims=dims, alpha=a.alpha, gamma=a.gamma, activation=a.activation, dtype=op,
                                  recompute_activation=not a.save_activation),
                        device=device, seed=a.seed)
    guard = ThermalGuard(max_temp_c=a.temperature_max, poll_s=a.thermal_poll) if a.temperature_max > 0 else None
    stager = BatchStager(a.batch, ds.features, ds.num_classes, device=device, dtype=torch.float32)
    runner = None
    history = []
    for epoch in range(a.epochs):
        t0 = time.perf_counter()
        total = 0
        correct = torch.zeros((), dtype=torch.int64, device=device)
        it = ds.batches(a.batch, shuffle=True, seed=a.seed, epoch=epoch, drop_last=True)
        pending = next(it, None)
        if pending is not None:
            stager.put(*pending)
        while pending is not None:
            if guard is not None:
                guard.wait_until_safe(verbose=True)
            x, y, labels = stager.get()
            pending = next(it, None)
            if pending is not None:
                stager.put(*pending)          # the next batch's H2D overlaps this batch's steps
            model.initialize_batch(x, y)
            if a.graph:
                if runner is None:
                    runner = model.capture_graph(a.steps)
                runner.replay()
            else:
                model.run_steps(a.steps)
            correct += batch_correct(model, x, labels)
            total += int(labels.numel())
        n_correct = int(correct.item())
        model.check_steps()                   # raises if a whole-step launch of this epoch timed out
        dt = time.perf_counter() - t0
        rec = {"epoch": epoch + 1, "time_s": round(dt, 3), "train_acc": n_correct / max(total, 1),
               "samples_per_s": round(total / dt, 1), "samples": total, "path": model.path, "dataset": ds.name}
        history.append(rec)
        if a.json:
            print(json.dumps(rec), flush=True)
        else:
            print(f"epoch={epoch + 1:03d} time={dt:.3f}s train_acc={rec['train_acc']:.4f} "
                  f"samples/s={rec['samples_per_s']:.1f}", flush=True)
    return history, model


def main(argv=None) -> int:
    train(parse_args(argv))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
