"""Graph capture of a fixed number of iPC steps.

Mirrors ``IPCGraphRunner`` (``src/ipc_tilelang/cuda_graph.py:6-36``): warm
the kernels (``precompile``, which restores every buffer), capture ``steps``
steps into a graph, replay it.  The graph is the plan's own
(``ipc_plan_graph_capture``): a hipGraph recorded on a private stream inside
the library and replayed with one ``hipGraphLaunch`` per replay on torch's
current stream, holding the plan's launches only.  When the captured steps
are a single launch of a whole-step kernel the library records that launch
and replays it directly instead, which is what a one-node graph does, without
the ~5 us of graph-launch overhead per replay measured on MI355X (49.1 us per
replay of the depth-6 layer-resident launch against 44.3 us direct).  Buffer
addresses stay fixed because the model reuses its buffers for every batch of
the same shape; a new plan (another batch size) discards the graph, and
replaying a discarded graph raises.
"""
from __future__ import annotations

import torch

from . import _native as nat


class IPCGraphRunner:
    def __init__(self, model, steps: int):
        if steps < 1:
            raise ValueError("steps must be >= 1")
        self.model = model
        self.steps = int(steps)
        self._plan = None
        self._generation = None

    def capture(self) -> None:
        torch.cuda.synchronize()
        self.model.precompile()
        torch.cuda.synchronize()
        plan = self.model._plan
        nat.check(nat.lib().ipc_plan_graph_capture(plan, self.steps))
        self.model._graph_generation = getattr(self.model, "_graph_generation", 0) + 1
        self._plan = plan
        self._generation = self.model._graph_generation

    def replay(self, repeats: int = 1) -> None:
        """Launch the captured steps ``repeats`` times on the current stream
        (one library call however many replays)."""
        plan = self.model._plan
        if (self._plan is None or plan is None or plan.value != self._plan.value
                or self._generation != getattr(self.model, "_graph_generation", None)):
            raise RuntimeError("Graph has not been captured (or was discarded by a later capture or a new plan)")
        # writes of x / W counted by torch since the last launch: re-sync the
        # plan's operand copies and caches first (outside the graph)
        self.model._sync_if_written()
        # the library refuses a plan whose graph a rebind discarded (IPC_ERR_STATE)
        nat.check(nat.lib().ipc_plan_graph_launch(plan, int(repeats), nat.current_stream_handle(self.model.device)))
