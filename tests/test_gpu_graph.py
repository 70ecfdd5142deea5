"""Whole-step plans captured into the caller's own graph.

The reference's runner captures T calls of step_initialized with
torch.cuda.graph and replays the graph (src/ipc_tilelang/cuda_graph.py:22-31).
The library launches on torch's current stream, read at call time, so the
same capture records the layer-resident and column-block whole-step launches;
every replay must give the bits of the same steps launched directly,
replay after replay (the resident kernel's step flags count across
launches, so a replayed launch must find its base from them as a direct
one does).
"""
import pytest
import torch

from lich_amd.trainer import HipIPC, IPCConfig
from oracle import ipc_oracle as O
from tests.helpers import DEV, report

pytestmark = pytest.mark.gpu

D6 = (10,) + (64,) * 6 + (784,)
C3 = (10,) + (64,) * 4 + (784,)


def _model(dims, B, dtype, seed, wmode):
    w0 = O.init_weights(dims, seed=seed, init="xavier_uniform")
    x_in, _l, y = O.make_batch(dims, B, seed=seed)
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=dtype, weight_update_mode=wmode,
                         hierarchical_policy_auto=False), device=DEV, weights=w0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    return m


@pytest.mark.parametrize("form", ["step_loop", "run_steps"])
@pytest.mark.parametrize("path,dims,B,dtype,wmode", [
    ("resident", D6, 128, torch.float16, "auto"),
    ("resident", D6, 96, torch.bfloat16, "auto"),
    ("resident", C3, 8, torch.float32, "auto"),
    ("narrow", (10, 64, 64, 64, 784), 128, torch.float32, "auto"),
    ("narrow", D6, 16, torch.float16, "auto"),
])
def test_whole_step_plan_replays_of_a_torch_graph_equal_direct_launches(path, dims, B, dtype, wmode, form):
    T = 8 if dtype == torch.float32 and B <= 16 else 4
    report("torch-graph", path=path, L=len(dims) - 1, B=B, dtype=str(dtype), form=form)
    direct = _model(dims, B, dtype, 3, wmode)
    graphed = _model(dims, B, dtype, 3, wmode)
    assert direct.path == graphed.path == path
    snaps = []
    for _ in range(3):
        direct.run_steps(T)
        torch.cuda.synchronize()
        snaps.append([t.clone() for t in direct.x + direct.e[:-1] + direct.w])
    direct.check_steps()

    graphed.precompile()  # warm every kernel, then restore the buffers
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        if form == "step_loop":
            for _ in range(T):
                graphed.step_initialized()
        else:
            graphed.run_steps(T)
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        got = graphed.x + graphed.e[:-1] + graphed.w
        for i, (a, b) in enumerate(zip(got, snaps[r])):
            assert torch.equal(a, b), (r, i, float((a - b).abs().max()))
    graphed.check_steps()
    del g


def test_stream_handle_follows_the_current_stream_and_the_capture_stream():
    """The handle every library call launches on is torch's current stream,
    read at call time: the default stream, a side stream inside its context
    manager, and the capture stream inside torch.cuda.graph."""
    from lich_amd import _native as nat

    report("stream-handle")
    assert nat.current_stream_handle() == torch.cuda.current_stream().cuda_stream
    assert nat.current_stream_handle(DEV) == torch.cuda.current_stream(DEV).cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert nat.current_stream_handle(DEV) == side.cuda_stream
        assert nat.current_stream_handle() == side.cuda_stream
    seen = []
    g = torch.cuda.CUDAGraph()
    x = torch.zeros(4, device=DEV)
    with torch.cuda.graph(g):
        seen.append((nat.current_stream_handle(DEV), torch.cuda.current_stream(DEV).cuda_stream))
        x.add_(1.0)
    g.replay()
    torch.cuda.synchronize()
    assert seen[0][0] == seen[0][1] and seen[0][0] != torch.cuda.current_stream(DEV).cuda_stream
