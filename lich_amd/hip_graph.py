"""Graph capture of a fixed number of iPC steps.

Mirrors ``IPCGraphRunner`` (``src/ipc_tilelang/cuda_graph.py:6-36``).  On
ROCm ``torch.cuda.CUDAGraph`` records a hipGraph: the plan's launches read
torch's current stream at call time, so the ``steps`` steps land on the
capture stream and replay as one graph launch.  Buffer addresses stay fixed because the model reuses its buffers for
every batch of the same shape.
"""
from __future__ import annotations

import torch


class IPCGraphRunner:
    def __init__(self, model, steps: int):
        if steps < 1:
            raise ValueError("steps must be >= 1")
        self.model = model
        self.steps = int(steps)
        self.graph = None
        self._captured = False

    def capture(self) -> None:
        torch.cuda.synchronize()
        self.model.precompile()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            # the same `steps` steps as a loop of step_initialized calls, enqueued
            # by one library call (the whole-step kernel runs them in one launch)
            self.model.run_steps(self.steps)
        torch.cuda.synchronize()
        self._captured = True

    def replay(self) -> None:
        if not self._captured:
            raise RuntimeError("Graph has not been captured")
        self.graph.replay()
