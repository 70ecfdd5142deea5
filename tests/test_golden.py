"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture.  GPU: the HIP path (fp32
operands, whole-step kernel and per-phase launches) reproduces them within the
fp32 bar (1e-5 relative, globally normalised).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ipc_oracle as O

from tests.helpers import delta_w_check

FIXTURES = sorted((Path(__file__).parent / "golden").glob("*.npz"))


def _load(path):
    z = np.load(path, allow_pickle=False)
    dims = tuple(int(v) for v in z["dims"])
    L = len(dims) - 1
    t = lambda k: torch.from_numpy(z[k].copy())  # noqa: E731
    return {
        "dims": dims, "L": L, "B": int(z["batch"]), "T": int(z["steps"]), "alpha": float(z["alpha"]),
        "gamma": float(z["gamma"]), "act": str(z["act"]), "x_in": t("x_in"), "y": t("y"),
        "w0": [t(f"w0_{l}") for l in range(L)], "wT": [t(f"wT_{l}") for l in range(L)],
        "eT": [t(f"eT_{l}") for l in range(L)], "x0": [t(f"x0_{l}") for l in range(L + 1)],
        "xT": [t(f"xT_{l}") for l in range(L + 1)],
    }


def test_fixtures_exist():
    assert len(FIXTURES) >= 4


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_oracle_reproduces_fixture(path):
    g = _load(path)
    x0 = O.forward_init(g["x_in"], g["y"], g["w0"], g["act"])
    assert O.global_rel_err(x0[1:-1], g["x0"][1:-1]) <= 1e-6
    xt, wt, et = O.run_steps(x0, g["w0"], g["T"], act=g["act"], alpha=g["alpha"], gamma=g["gamma"])
    assert O.global_rel_err(xt, g["xT"]) <= 1e-6
    assert O.global_rel_err(wt, g["wT"]) <= 1e-6
    assert O.global_rel_err(et, g["eT"]) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("fused", ["on", "off"])
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_hip_path_reproduces_fixture(path, fused):
    from lich_amd.trainer import HipIPC, IPCConfig

    g = _load(path)
    dev = torch.device("cuda", 0)
    print(f"[case] golden {path.stem} fused={fused}", flush=True)
    m = HipIPC(IPCConfig(dims=g["dims"], activation=g["act"], dtype=torch.float32, alpha=g["alpha"],
                         gamma=g["gamma"], fused=fused), device=dev, weights=g["w0"])
    m.initialize_batch(g["x_in"].to(dev), g["y"].to(dev))
    assert O.global_rel_err(m.x[1:-1], g["x0"][1:-1]) <= 1e-5
    m.run_steps(g["T"])
    torch.cuda.synchronize()
    assert O.global_rel_err(m.x, g["xT"]) <= 1e-5
    assert O.global_rel_err(m.w, g["wT"]) <= 1e-5
    ok, msg = delta_w_check(m.w, g["w0"], g["wT"], g["x0"], g["T"], act=g["act"], alpha=g["alpha"],
                            gamma=g["gamma"])
    print(f"golden {path.stem} fused={fused}: {msg}")
    assert ok, msg
    assert O.global_rel_err(m.e[:-1], g["eT"]) <= 1e-5
