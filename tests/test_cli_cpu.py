"""The command-line drop-in (reference scripts/run_cli.py:20-41) and the
pure-PyTorch reference API it exposes, on the CPU."""
import json

import pytest
import torch

from lich_amd import cli
from lich_amd import reference as R
from oracle import ipc_oracle as O


def test_dispatch_knows_the_reference_commands():
    assert {"smoke", "reference", "autotune", "train-mnist", "efficiency", "thermal-bench"} <= set(cli.COMMANDS)
    with pytest.raises(SystemExit) as exc:
        cli.main(["no-such-command"])
    assert exc.value.code == 2
    with pytest.raises(SystemExit) as exc:
        cli.main(["efficiency", "--depths", "5"])  # the reference's choices are 3, 4, 6
    assert exc.value.code == 2


def test_reference_command_prints_a_trajectory(capsys):
    assert cli.main(["reference", "--depth", "2", "--hidden", "16", "--batch", "4", "--steps", "3"]) == 0
    lines = capsys.readouterr().out.strip().splitlines()
    assert lines[-1] == "Reference iPC trajectory computed successfully."
    rows = [ln.split() for ln in lines[:-1]]
    assert [int(r[0]) for r in rows] == [0, 1, 2]
    assert all(float(r[1]) >= 0 and float(r[2]) >= 0 for r in rows)


@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid", "silu", "gelu"])
def test_reference_api_step_equals_the_oracle(act):
    """lich_amd.reference.ipc_step against the pinned oracle (float64, tiny net)."""
    dims, B = (3, 5, 4, 6), 7
    w = O.init_weights(dims, seed=2, init="kaiming_a_sqrt5")
    x_in, _l, y = O.make_batch(dims, B, seed=2)
    x = [t.double() for t in O.forward_init(x_in, y, w, act)]
    w = [t.double() for t in w]
    st = R.ReferenceState(x=list(x), w=list(w))
    spec = R.get_activation(act)
    for _ in range(3):
        st, m = R.ipc_step(st, act=spec, alpha=1e-2, gamma=0.5, fixed_low=x[0], fixed_high=x[-1])
        x, w, e, mo = O.ipc_step(x, w, act=act, alpha=1e-2, gamma=0.5)
    assert O.global_rel_err(st.x, x) < 1e-12 and O.global_rel_err(st.w, w) < 1e-12
    # the reference reports its metrics in float32 (reference.py:58)
    assert abs(float(m["max_abs_error"]) - mo["max_abs_error"]) <= 1e-6 * mo["max_abs_error"]


def test_reference_api_helpers():
    y = R.one_hot(torch.tensor([2, 0]), 3, dtype=torch.float32)
    assert y.tolist() == [[0, 1], [0, 0], [1, 0]]
    ws = R.init_weights((10, 64, 784), dtype=torch.float32, device="cpu", seed=3)
    assert ws[0].shape == (10, 64) and float(ws[0].abs().max()) <= 1 / 64 ** 0.5
    st = R.initialize_state(torch.ones(784, 2), y[:, :2].repeat(4, 1)[:10], (10, 64, 784), dtype=torch.float32,
                            device="cpu")
    assert torch.count_nonzero(st.x[1]) == 0 and torch.equal(st.x[-1], torch.ones(784, 2))
    with pytest.raises(ValueError):
        R.get_activation("swish")
    d = R.get_activation("relu").derivative(torch.tensor([0.0, 1.0, -1.0]))
    assert d.tolist() == [0.0, 1.0, 0.0]


def test_toolchain_report_runs_without_a_gpu(capsys):
    assert cli.main(["toolchain"]) == 0
    rep = json.loads(capsys.readouterr().out)
    assert rep["library_built"] is True and rep["abi_version"] >= 5


def test_reference_command_follows_the_scripts_random_stream(capsys):
    """scripts/validate_reference.py:16-35 seeds the global generator once and
    draws the input, then each W by kaiming_uniform_(a=sqrt(5)) from that same
    generator; relu; forward initialisation; alpha 1e-4, gamma 0.5.  The
    command's printed energies are that sequence's (recomputed here with the
    oracle's step, itself pinned by tests/test_oracle.py)."""
    from oracle import ipc_oracle as O

    assert cli.main(["reference", "--depth", "3", "--hidden", "64", "--batch", "8", "--steps", "4"]) == 0
    rows = [ln.split() for ln in capsys.readouterr().out.splitlines() if ln[:1].isdigit()]
    torch.manual_seed(0)
    dims = (10, 64, 64, 64, 784)
    x_in = torch.randn((784, 8))
    y = O.one_hot(torch.arange(8) % 10, 10)
    w = [torch.nn.init.kaiming_uniform_(torch.empty((r, c)), a=5 ** 0.5) for r, c in zip(dims[:-1], dims[1:])]
    x = O.forward_init(x_in, y, w, "relu")
    for i in range(4):
        x, w, _e, m = O.ipc_step(x, w, act="relu", alpha=1e-4, gamma=0.5)
        assert int(rows[i][0]) == i
        assert abs(float(rows[i][1]) - m["energy"]) <= 1e-5 * m["energy"]
        assert abs(float(rows[i][2]) - m["max_abs_error"]) <= 1e-5 * m["max_abs_error"]
