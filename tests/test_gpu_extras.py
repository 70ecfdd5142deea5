"""Training loop, batch pipeline, telemetry and tuning artefacts on the GPU."""
import json

import pytest
import torch

from lich_amd import autotune as AT
from lich_amd import data as D
from lich_amd import telemetry as TM
from lich_amd import train as TR
from lich_amd.kernels import KernelConfig
from lich_amd.trainer import HipIPC, IPCConfig, prepare_batch
from lich_amd.tuning import TuningEntry, TuningKey, TuningTable
from oracle import ipc_oracle as O
from tests.helpers import DEV, report

pytestmark = pytest.mark.gpu


def test_batch_stager_equals_prepare_batch():
    report("stager")
    ds = D.synthetic_dataset(256, seed=2)
    st = D.BatchStager(64, ds.features, 10, device=DEV)
    batches = list(ds.batches(64, seed=1))
    st.put(*batches[0])
    for i, (img, lab) in enumerate(batches):
        x, y, labels = st.get()
        if i + 1 < len(batches):
            st.put(*batches[i + 1])      # the next copy is in flight while this batch is checked
        xr, yr = prepare_batch(img, lab, device=DEV, dtype=torch.float32, num_classes=10)
        assert torch.equal(x, xr) and torch.equal(y, yr) and torch.equal(labels.cpu(), lab)
    with pytest.raises(RuntimeError, match="no staged batch"):
        st.get()


@pytest.mark.parametrize("graph", [False, True])
def test_training_loop_on_synthetic_data(graph):
    report("train-loop", graph=graph)
    args = TR.parse_args(["--synthetic", "1024", "--epochs", "2", "--batch", "128", "--depth", "2",
                          "--activation", "tanh", "--json"] + (["--graph"] if graph else []))
    hist, model = TR.train(args)
    assert [h["epoch"] for h in hist] == [1, 2] and all(h["samples"] == 1024 for h in hist)
    assert all(0.0 <= h["train_acc"] <= 1.0 for h in hist) and model.path == "resident"
    assert model.barrier_timeouts() == 0
    # the accuracy of one batch is argmax(predict) against the labels
    ds = D.synthetic_dataset(1024, seed=0)
    img, lab = next(ds.batches(128, shuffle=False))
    x, _ = prepare_batch(img, lab, device=DEV, dtype=torch.float32, num_classes=10)
    ref = O.predict([w.cpu() for w in model.w], x.cpu(), "tanh").argmax(dim=0)
    got = TR.batch_accuracy(model, x, lab.to(DEV))
    assert abs(got - int((ref == lab).sum())) <= 2   # fp16-operand forward vs fp32 oracle: ties may flip


def test_graph_and_direct_training_give_the_same_weights():
    report("train-graph-vs-direct")
    runs = []
    for graph in (False, True):
        args = TR.parse_args(["--synthetic", "512", "--epochs", "1", "--batch", "128", "--depth", "3",
                              "--activation", "relu", "--json"] + (["--graph"] if graph else []))
        runs.append(TR.train(args)[1])
    for a, b in zip(runs[0].w, runs[1].w):
        assert torch.equal(a, b)


def test_telemetry_reads_the_device():
    t = TM.read_telemetry(0)
    print("telemetry:", TM.ThermalGuard.format_status(t))
    assert t.temperature_c is not None and 0.0 < t.temperature_c < 150.0
    assert t.clock_gfx_max_mhz is not None and t.clock_gfx_max_mhz > 0.0
    g = TM.ThermalGuard(max_temp_c=200.0)
    assert g.wait_until_safe().temperature_c == t.temperature_c or g.pauses == 0


def _phased_run(dims, w0, x, y, table=None, policy=None):
    kw = {} if policy is None else dict(hierarchical_policy_path=str(policy))
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=torch.float16, fused="phased",
                         tuning_table=table, hierarchical_policy_auto=policy is not None, **kw),
               device=DEV, weights=w0)
    m.initialize_batch(x, y)
    m.run_steps(3)
    torch.cuda.synchronize()
    return m


def test_tuning_table_tiles_reach_the_phased_plan():
    report("tuning-table")
    dims, B = (10, 64, 64, 784), 128
    w0 = O.init_weights(dims, seed=8, init="xavier_uniform")
    x, _l, y = O.make_batch(dims, B, seed=8)
    x, y = x.to(DEV), y.to(DEV)
    table = TuningTable.from_entries([
        TuningEntry(TuningKey("prediction", 64, 784, B, "tanh", "float16"), KernelConfig(tile=0)),
        TuningEntry(TuningKey("inference", 64, 64, B, "tanh", "float16"), KernelConfig(tile=2)),
        TuningEntry(TuningKey("weight", 64, 784, B, "tanh", "float16"), KernelConfig(block_m=64, block_n=64)),
    ])
    base, tuned = _phased_run(dims, w0, x, y), _phased_run(dims, w0, x, y, table=table)
    assert base.phase_tiles(B) == (-1, -1, -1) and tuned.phase_tiles(B) == (0, 2, 1)
    # every generic tile computes the same bits
    for a, b in zip(base.w + base.x, tuned.w + tuned.x):
        assert torch.equal(a, b)


def test_autotune_writes_tables_the_trainer_reads(tmp_path):
    report("autotune")
    dims, B = [10, 64, 64, 784], 128
    table = AT.tune_kernels(dims, B, "tanh", torch.float16, reps=5, replays=2)
    assert len(table.entries) == len(AT.net_shapes(dims)) == 8
    assert all(e.config.tile in (0, 1, 2) and e.median_ms > 0 for e in table.entries)
    table.to_json(tmp_path / "table.json")
    assert TuningTable.from_json(tmp_path / "table.json") == table
    best = {"path": "narrow", "recompute_activation": False, "use_cuda_graph": False, "grid_z_max_layers": 3,
            "step_ms": 1.0, "status": "ok", "source": "test"}
    pol = tmp_path / "policy.json"
    AT.write_policy(pol, dims, B, "tanh", torch.float16, table, best, [best])
    assert json.loads(pol.read_text())["schema_version"] == 3
    w0 = O.init_weights(tuple(dims), seed=9, init="xavier_uniform")
    x, _l, y = O.make_batch(tuple(dims), B, seed=9)
    m = _phased_run(tuple(dims), w0, x.to(DEV), y.to(DEV), policy=pol)
    # the execution entry resolves through the kernel-table fingerprint
    assert m.recompute_activation is False and m.grid_z_cap == 3
    assert m.recommended_use_cuda_graph(default=True) is False
    exp = tuple(next(e.config.tile for e in table.entries if (e.key.kind, e.key.M, e.key.K) == s)
                for s in (("prediction", 64, 784), ("inference", 64, 64), ("weight", 64, 784)))
    assert m.phase_tiles(B) == exp


def test_execution_tuning_times_every_eligible_path():
    report("autotune-exec")
    best, trials = AT.tune_execution([10, 64, 64, 784], 128, "tanh", torch.float16, steps=4, replays=5)
    # fp16 operands default to split 1 on narrow nets, which the wide path also runs
    assert {t["path"] for t in trials} == {"resident", "narrow", "phased", "wide"}
    # recompute on / off x graph on / off per path, and per row-block size (16, 32, 64) on the resident path
    per_path = {p: sum(t["path"] == p for t in trials) for p in ("resident", "narrow", "phased", "wide")}
    assert per_path == {"resident": 12, "narrow": 4, "phased": 4, "wide": 4}
    assert {t["resident_rows"] for t in trials if t["path"] == "resident"} == {16, 32, 64}
    assert best in trials and best["step_ms"] == min(t["step_ms"] for t in trials)
    assert best["path"] == "resident"
