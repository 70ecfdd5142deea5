"""The command-line drop-in on the GPU: the kernel smoke (scripts/smoke.py),
the paper efficiency sweep on synthetic data (scripts/train_paper_efficiency.py),
the sustained-throughput bench (scripts/thermal_bench.py) and the direct vs
captured steady-state A/B (scripts/benchmark_stage2_4_steady_state.py)."""
import json

import pytest

from lich_amd import cli
from tests.helpers import report

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("act", ["relu", "tanh"])
def test_cli_kernel_smoke(act, capsys):
    report("cli-smoke", act=act)
    assert cli.main(["smoke", "--activation", act]) == 0
    assert "PASS" in capsys.readouterr().out


def test_cli_efficiency_on_synthetic_data(tmp_path, capsys):
    report("cli-efficiency")
    out = tmp_path / "eff.jsonl"
    assert cli.main(["efficiency", "--synthetic", "1024", "--subset", "1024", "--depths", "3", "6", "--steps", "4",
                     "--graph", "--temperature-max", "0", "--out", str(out)]) == 0
    rows = [json.loads(ln) for ln in out.read_text().splitlines()]
    assert [r["depth"] for r in rows] == [3, 6]
    for r in rows:
        assert r["path"] == "resident" and r["samples_per_s"] > 0
        assert r["ipc_step_samples_per_s"] == pytest.approx(4 * r["samples_per_s"])


def test_cli_thermal_bench_and_steady_state(tmp_path, capsys):
    report("cli-thermal-steady")
    assert cli.main(["thermal-bench", "--depth", "6", "--seconds", "1.5", "--temperature-max", "0", "--graph"]) == 0
    assert "FINAL" in capsys.readouterr().out
    out = tmp_path / "steady.json"
    assert cli.main(["steady-state", "--dims", "10", "64", "64", "784", "--repeats", "10", "--out", str(out)]) == 0
    res = json.loads(out.read_text())
    assert res["graph_active"] and res["direct_ms_step"] > 0 and res["graph_ms_step"] > 0
