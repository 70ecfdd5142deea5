"""Whole-step kernels never hand back a timed-out step silently, and the
trainer reads the grid.z policy file.

The timeout path is forced from the host: a spin limit of 0 makes every wait
of the layer-resident and column kernels give up at its first unsatisfied
poll, so the kernels still run to their end (no fault, no hang) while the
timeout word is raised; the trainer must then raise instead of returning
numbers, clear the word, and run correct steps again once the limit is
restored.
"""
import json

import pytest
import torch

from lich_amd.trainer import HipIPC, IPCConfig
from oracle import ipc_oracle as O
from tests.helpers import DEV, report

pytestmark = pytest.mark.gpu


def _model(dims, B, dtype, seed):
    w0 = O.init_weights(dims, seed=seed, init="xavier_uniform")
    x_in, _l, y = O.make_batch(dims, B, seed=seed)
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=dtype, hierarchical_policy_auto=False),
               device=DEV, weights=w0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    return m, w0, x_in, y


@pytest.mark.parametrize("path,dims,dtype", [
    ("resident", (10,) + (64,) * 6 + (784,), torch.float16),
    ("narrow", (10, 64, 64, 64, 784), torch.float32),
])
def test_timed_out_steps_raise_and_the_plan_recovers(path, dims, dtype):
    report("health-timeout", path=path)
    T, B = 4, 128
    m, w0, x_in, y = _model(dims, B, dtype, seed=3)
    assert m.path == path
    m.set_spin_limit(0)
    m.run_steps(T)
    with pytest.raises(RuntimeError, match="spin limit"):
        m.check_steps()
    assert m.barrier_timeouts() == 0  # the check cleared the word
    m.run_steps(T)
    with pytest.raises(RuntimeError, match="spin limit"):
        m.metrics()
    m.run_steps(T)
    with pytest.raises(RuntimeError, match="spin limit"):
        m.run_prepared_steady_state(steps=T, repeats=1, use_graph=False)
    # restored limit and weights: the next batch trains correctly and checks clean
    m.set_spin_limit(None)
    for l, w in enumerate(w0):
        m.w[l].copy_(w.to(DEV))
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    m.run_steps(T)
    m.check_steps()
    x = O.forward_init(x_in, y, w0, "tanh")
    x_t, w_t, _e = O.run_steps(x, w0, T, act="tanh", alpha=1e-4, gamma=0.5)
    s_err = O.global_rel_err(m.x[1:-1], x_t[1:-1])
    dw = O.global_rel_err([m.w[l].cpu().double() - w0[l].double() for l in range(len(w0))],
                          [w_t[l].double() - w0[l].double() for l in range(len(w0))])
    bars = (1e-5, 1e-5) if dtype == torch.float32 else (2e-2, 5e-3)
    print(f"after recovery: state {s_err:.3e}, dW {dw:.3e}", flush=True)
    assert s_err <= bars[0] and dw <= bars[1]


def test_trainer_reads_the_grid_z_policy_file(tmp_path):
    """A grid.z policy entry for this device and net sets the recorded cap and
    its groups (reference gridz_tuning.py:50-73, trainer.py:273-300)."""
    report("health-gridz")
    from lich_amd.gridz_tuning import make_policy_key
    from lich_amd.layer_batching import find_internal_square_groups

    dims = (10,) + (64,) * 6 + (784,)
    key = make_policy_key(device_name=torch.cuda.get_device_name(DEV), capability=torch.cuda.get_device_capability(DEV),
                          dims=dims, batch=128, activation="tanh", dtype=torch.float16)
    path = tmp_path / "gridz_policy.json"
    path.write_text(json.dumps({"version": 1, "entries": {key: {"grid_z_max_layers": 5}}}))
    x_in, _l, y = O.make_batch(dims, 128, seed=0)
    cfg = IPCConfig(dims=dims, activation="tanh", dtype=torch.float16, grid_z_policy_path=str(path),
                    hierarchical_policy_auto=False)
    m = HipIPC(cfg, device=DEV, seed=0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    assert m.grid_z_cap == 5
    assert m.layer_groups == find_internal_square_groups(dims, max_group_count=5)
    m2 = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=torch.float16, grid_z_policy_path=str(path),
                          hierarchical_policy_auto=False, grid_z_auto=False), device=DEV, seed=0)
    m2.initialize_batch(x_in.to(DEV), y.to(DEV))
    assert m2.grid_z_cap == 2  # grid_z_auto off: the configured cap
