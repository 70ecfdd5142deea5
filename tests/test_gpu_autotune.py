"""The correctness-gated tuner: a candidate that fails the reference's probe
(scripts/autotune.py:250-260) is never selected, however fast, and is
recorded; the wide path's tile configurations are bit-identical to each other;
a tuned wide configuration reaches the trainer through the policy file."""
import json

import pytest
import torch

from lich_amd import autotune as AT
from lich_amd.trainer import HipIPC, IPCConfig, init_weights_cpu
from tests.helpers import DEV, report

pytestmark = pytest.mark.gpu


def test_kernel_tuner_never_selects_a_failing_tile():
    report("autotune-kernels")
    dims, B = (10, 64, 64, 784), 128
    rejected = []

    def corrupt(kind, M, K, tile, out):
        if tile == 2:
            out.add_(1.0)  # a broken candidate: every element off by 1

    def fastest_is_2(kind, M, K, tile, us):
        return 1.0 if tile == 2 else 10.0 + tile

    table = AT.tune_kernels(dims, B, "tanh", torch.float16, reps=3, replays=1, rejected=rejected,
                            perturb=corrupt, timer=fastest_is_2)
    assert table.entries, "every shape must have a passing tile"
    assert all(e.config.tile_id() != 2 for e in table.entries)
    assert {r["tile"] for r in rejected} == {2} and len(rejected) == len(AT.net_shapes(dims))
    assert all("mismatch ratio" in r["reason"] for r in rejected)


def test_wide_tuner_gates_candidates_and_configs_agree_bitwise(tmp_path):
    report("autotune-wide")
    dims, B = (1000, 1024, 1024, 1024), 256
    rejected = []

    def corrupt(phase, cand, m):
        if phase == "weight" and cand[0] == 1:
            m.w[0].add_(1.0)

    def fastest_weight_1(phase, cand, us):
        return 1.0 if phase == "weight" and cand[0] == 1 else us

    chosen = AT.tune_wide(dims, B, "tanh", torch.bfloat16, reps=2, replays=1, rejected=rejected,
                          perturb=corrupt, timer=fastest_weight_1)
    print("chosen", chosen, "rejected", rejected, flush=True)
    assert chosen is not None and chosen["weight"] != 1
    assert [r for r in rejected if r["phase"] == "weight"] and all(r["config"] == 1 for r in rejected)
    # every tile configuration of a phase gives the same bits (k-split left automatic)
    w0 = init_weights_cpu(dims, seed=4, init="xavier_uniform")
    g = torch.Generator().manual_seed(4)
    x_in = torch.randn((dims[-1], B), generator=g).to(DEV)
    y = torch.nn.functional.one_hot(torch.randint(0, dims[0], (B,), generator=g), dims[0]).float().T.contiguous().to(DEV)
    outs = []
    for wc in ((-1, -1, -1, -1), (1, 1, 1, -1), (0, 0, 2, -1), (0, 3, 4, -1)):
        m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=torch.bfloat16, fused="wide", wide_config=wc,
                             hierarchical_policy_auto=False), device=DEV, weights=w0)
        m.initialize_batch(x_in, y)
        m.run_steps(3)
        torch.cuda.synchronize()
        outs.append([t.clone() for t in m.x + m.e[:-1] + m.w])
        del m
    for other in outs[1:]:
        assert all(torch.equal(a, b) for a, b in zip(outs[0], other))
    # the tuned choice travels through a policy file into the trainer
    # a table of the default kernel configuration for every shape: the profile
    # the execution entry is keyed by (its kernel signature) is then the one
    # the trainer computes for itself
    table = AT.TuningTable.from_entries([AT.TuningEntry(AT.TuningKey(k, M, K, B, "tanh", "bfloat16"),
                                                        AT.KernelConfig(), None, False)
                                         for k, M, K in AT.net_shapes(dims)])
    best = {"path": "wide", "recompute_activation": True, "use_cuda_graph": True, "grid_z_max_layers": 1}
    pol = tmp_path / "policy.json"
    AT.write_policy(pol, list(dims), B, "tanh", torch.bfloat16, table, best, [best], wide_config=chosen,
                    rejected=rejected)
    assert json.loads(pol.read_text())["execution_entries"][0]["rejected"]
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=torch.bfloat16, hierarchical_policy_path=str(pol)),
               device=DEV, weights=w0)
    m.initialize_batch(x_in, y)
    assert m.path == "wide"
    assert m.wide_config == tuple(chosen[k] for k in ("pred", "infer", "weight", "ksplit"))


def test_standalone_tuner_searches_the_dma_tiles_and_the_choice_reaches_the_builders():
    """The operator calls with bf16 storage at a per-kernel sweep shape: the
    LDS-DMA tile configurations are candidates; one that fails the probe
    is never selected (however fast), and the chosen tile is what a builder
    given the table's config runs."""
    from lich_amd.kernels import build_prediction_error

    report("autotune-standalone")
    M = K = 1024
    B = 256
    rejected = []

    def corrupt(kind, M_, K_, tile, out):
        if tile == 4:
            out.add_(1.0)

    def prefer(kind, M_, K_, tile, us):
        return {4: 0.5, 5: 1.0}.get(tile, 10.0 + tile)

    table = AT.tune_standalone([(M, K, B)], "tanh", torch.bfloat16, reps=2, replays=1, rejected=rejected,
                               perturb=corrupt, timer=prefer)
    kinds = {e.key.kind for e in table.entries}
    assert kinds == {"prediction", "inference", "weight"}
    assert all(e.config.tile == 5 for e in table.entries), [e.config for e in table.entries]
    assert {r["tile"] for r in rejected} == {4} and len(rejected) == 3
    cfg = table.lookup(kind="prediction", M=M, K=K, B=B, activation="tanh", dtype="bfloat16")
    k = build_prediction_error(M, K, B, "tanh", torch.bfloat16, cfg)
    assert k.tile == 5
    g = torch.Generator().manual_seed(3)
    xu = torch.randn((K, B), generator=g).to(DEV, torch.bfloat16)
    w = (torch.randn((M, K), generator=g) / 32).to(DEV, torch.bfloat16)
    xl = torch.randn((M, B), generator=g).to(DEV, torch.bfloat16)
    e5, e3 = torch.empty_like(xl), torch.empty_like(xl)
    k(xu, w, xl, e5)
    build_prediction_error(M, K, B, "tanh", torch.bfloat16)(xu, w, xl, e3)
    torch.cuda.synchronize()
    assert (e5 != e3).float().mean() <= 1e-2


def test_execution_tuner_gates_resident_row_blocks_and_the_choice_reaches_the_trainer(tmp_path):
    """Layer-resident row-block sizes are execution candidates: a size whose
    step fails the probe is never chosen; the chosen size travels through the
    policy file into the plan the trainer builds."""
    from lich_amd import _native as nat

    report("autotune-resident-rows")
    dims, B = (10,) + (64,) * 4 + (784,), 128
    rejected = []

    def corrupt(trial, m):
        if trial.get("resident_rows") == 16:
            m.w[0].add_(1.0)

    def prefer(trial, step_ms):
        if trial["path"] != "resident":
            return 1.0
        return {16: 1e-4, 64: 2e-4}.get(trial["resident_rows"], 1e-3)

    best, trials = AT.tune_execution(dims, B, "tanh", torch.float16, steps=4, replays=2, rejected=rejected,
                                     perturb=corrupt, timer=prefer)
    print("best", best, flush=True)
    assert best["path"] == "resident" and best["resident_rows"] == 64
    assert all(t.get("resident_rows") != 16 for t in trials)
    assert rejected and all(r["resident_rows"] == 16 for r in rejected)
    table = AT.TuningTable.from_entries([AT.TuningEntry(AT.TuningKey(k, M, K, B, "tanh", "float16"),
                                                        AT.KernelConfig(), None, False)
                                         for k, M, K in AT.net_shapes(dims)])
    pol = tmp_path / "policy.json"
    AT.write_policy(pol, list(dims), B, "tanh", torch.float16, table, best, trials, rejected=rejected)
    w0 = init_weights_cpu(dims, seed=0, init="xavier_uniform")
    g = torch.Generator().manual_seed(7919)
    x_in = torch.rand((dims[-1], B), generator=g).to(DEV)
    y = torch.nn.functional.one_hot(torch.randint(0, dims[0], (B,), generator=g), dims[0]).float().T.contiguous().to(DEV)
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=torch.float16, hierarchical_policy_path=str(pol)),
               device=DEV, weights=w0)
    m.initialize_batch(x_in, y)
    assert m.path == "resident" and m.resident_rows == 64
    assert nat.lib().ipc_plan_resident_rows(m._plan) == 64
