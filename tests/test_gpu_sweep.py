"""The standalone kernels at the per-kernel roofline sweep's shapes.

Prediction + error, the transposed inference update (with and without the
saved activation) and the weight update (recomputing f(X) and reading a saved
A), each with bf16 storage and operands (fp32 accumulation), tanh and relu,
M = K in {1024, 4096, 8192}, B in {256, 2048, 8192}: W ~ N(0, 1/K), states
and errors ~ N(0, 1), as ``bench.py --sweep`` times them.

* M = K = 1024: every output element against the fp32 oracle evaluated on the
  bf16-rounded inputs (the reference's correctness gate of
  ``scripts/autotune.py:250-260``: at most 1 % of the elements outside
  2e-2 + 2e-2 |ref|, plus a 2e-2 max-norm bound as in ``scripts/smoke.py:28-66``)
  and against a float64 model of the kernel's own rounding steps (16-bit
  operands, exact products, the storage-precision epilogue of
  ``tilelang_kernels.py:173,227-231,319-320``): at most 2 bf16 ulps of the
  output's max-norm apart, with under 1 % of the elements differing at all.
* every other point (M = K = 1024 with B = 8192, and M = K in {4096, 8192} with
  every B): a seeded sample of 64 rows x 64
  columns of each output against the oracle (same gate), and for relu the
  LDS-DMA kernel bit-identical to the generic MFMA kernel on a 256-row slice
  (each output row depends only on its own rows of W and X, and both kernels
  add the contraction in the same order).

The inputs are drawn on the device from a seeded generator and copied back
only where the oracle reads them.
"""
import math

import pytest
import torch

from lich_amd.kernels import KernelConfig, build_inference_update, build_prediction_error, build_weight_update
from oracle import ipc_oracle as O
from tests.helpers import DEV, rel_err, report

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
DMA = KernelConfig(tile=3)
GEN = KernelConfig(tile=2)
ALPHA, GAMMA = 0.01, 0.5
SMALL = [(1024, 256), (1024, 2048)]
LARGE = [(1024, 8192), (4096, 256), (4096, 2048), (4096, 8192), (8192, 256), (8192, 2048), (8192, 8192)]


def _inputs(n, B, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    r = lambda shape, s=1.0: (torch.randn(shape, generator=g, device=DEV) * s).to(BF)  # noqa: E731
    return {"w": r((n, n), 1 / math.sqrt(n)), "xu": r((n, B)), "xl": r((n, B)), "e": r((n, B)), "el": r((n, B))}


def _gate(got, ref, what):
    """scripts/autotune.py:250-260 (rtol = atol = 2e-2, at most 1 % outside) and a max-norm bound."""
    got, ref = got.double().cpu(), ref.double().cpu()
    bad = float((~((got - ref).abs() <= 2e-2 + 2e-2 * ref.abs())).double().mean())  # NaN counts as outside
    err = rel_err(got, ref)
    print(f"{what}: {bad:.2e} of elements outside the gate, max-norm rel err {err:.2e}", flush=True)
    assert bad <= 0.01 and err <= 2e-2, what


def _near_model(got, model, what):
    got, model = got.double().cpu(), model.double().cpu()
    differ = float((got != model).double().mean())
    err = rel_err(got, model)
    print(f"{what}: {differ:.2e} of elements differ from the rounding model, rel err {err:.2e}", flush=True)
    assert err <= 2 * 2.0 ** -8 and differ <= 0.01, what


def _run(kind, act, t, variant, cfg=DMA, rows=None):
    """Runs one kernel on (a row slice of) the inputs; returns its output."""
    n, B = t["w"].shape[0], t["xu"].shape[1]
    M = n if rows is None else rows
    if kind == "pred":
        e = torch.empty((M, B), device=DEV, dtype=BF)
        build_prediction_error(M, n, B, act, BF, cfg)(t["xu"], t["w"][:M].contiguous(), t["xl"][:M].contiguous(), e)
        return e
    if kind == "infer":
        save = variant == "save"
        x = t["xl"][:M].clone()
        a = torch.empty((M, B), device=DEV, dtype=BF) if save else None
        wl = t["w"][:, :M].contiguous()  # W_lower [K, M]
        build_inference_update(M, n, B, act, BF, cfg, GAMMA, save)(x, t["e"][:M].contiguous(), wl, t["el"], a)
        return (x, a) if save else x
    recompute = variant == "recompute"
    w = t["w"][:M].clone()
    src = t["xu"] if recompute else O.act_forward(act, t["xu"].float()).to(BF)
    build_weight_update(M, n, B, act, BF, cfg, ALPHA, recompute)(w, t["e"][:M].contiguous(), src)
    return w


CASES = [("pred", "-"), ("infer", "no-save"), ("infer", "save"), ("weight", "recompute"), ("weight", "saved-A")]


@pytest.mark.parametrize("act", ["tanh", "relu"])
@pytest.mark.parametrize("kind,variant", CASES)
@pytest.mark.parametrize("n,B", SMALL)
def test_sweep_small_shapes_against_oracle_and_model(n, B, kind, variant, act):
    report("sweep-small", n=n, B=B, kind=kind, variant=variant, act=act)
    t = _inputs(n, B, seed=n + B + len(kind))
    out = _run(kind, act, t, variant)
    torch.cuda.synchronize()
    c = {k: v.double().cpu() for k, v in t.items()}
    if kind == "pred":
        acc = c["w"] @ O.act_forward(act, c["xu"]).to(BF).double()
        _gate(out, O.pred_err(c["xu"], c["w"], c["xl"], act), "pred vs oracle")
        model = (c["xl"].float() - acc.float().to(BF).float()).to(BF)
        _near_model(out, model, "pred vs model")
    elif kind == "infer":
        x_ref, a_ref = O.infer_update(c["xl"], c["e"], c["w"], c["el"], act, GAMMA)
        x_out = out[0] if variant == "save" else out
        _gate(x_out, x_ref, "infer vs oracle")
        sig = c["w"].T @ c["el"]
        xn = c["xl"].float() + GAMMA * (-c["e"].float() + O.act_derivative(act, c["xl"].float()) * sig.float())
        _near_model(x_out, xn.to(BF), "infer vs model")
        if variant == "save":
            _gate(out[1], a_ref, "A_out vs oracle")
            _near_model(out[1], O.act_forward(act, xn).to(BF), "A_out vs model")
    else:
        a = O.act_forward(act, c["xu"]).to(BF).double()
        ref = O.weight_update(c["w"], c["e"], c["xu"], act, ALPHA)
        _gate(out.double().cpu() - c["w"], ref - c["w"], "weight delta vs oracle")
        model = (c["w"].float() + ALPHA * (c["e"] @ a.T).float()).to(BF)
        _near_model(out, model, "weight vs model")


@pytest.mark.parametrize("act", ["tanh", "relu"])
@pytest.mark.parametrize("kind,variant", CASES)
@pytest.mark.parametrize("n,B", LARGE)
def test_sweep_large_shapes_sampled(n, B, kind, variant, act):
    report("sweep-large", n=n, B=B, kind=kind, variant=variant, act=act)
    t = _inputs(n, B, seed=7 * n + B + len(variant))
    out = _run(kind, act, t, variant)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(n ^ B)
    R = torch.randperm(n, generator=g)[:64].sort().values.to(DEV)
    C = torch.randperm(B if kind != "weight" else n, generator=g)[:64].sort().values.to(DEV)
    d = lambda v: v.double().cpu()  # noqa: E731
    if kind == "pred":
        ref = O.pred_err(d(t["xu"][:, C]), d(t["w"][R]), d(t["xl"][R][:, C]), act)
        _gate(out[R][:, C], ref, "pred sample vs oracle")
    elif kind == "infer":
        x_ref, a_ref = O.infer_update(d(t["xl"][R][:, C]), d(t["e"][R][:, C]), d(t["w"][:, R]), d(t["el"][:, C]),
                                      act, GAMMA)
        x_out = out[0] if variant == "save" else out
        _gate(x_out[R][:, C], x_ref, "infer sample vs oracle")
        if variant == "save":
            _gate(out[1][R][:, C], a_ref, "A_out sample vs oracle")
    else:
        w0 = d(t["w"][R][:, C])
        ref = O.weight_update(w0, d(t["e"][R]), d(t["xu"][C]), act, ALPHA)
        _gate(d(out[R][:, C]) - w0, ref - w0, "weight delta sample vs oracle")
    if act == "relu":
        gen = _run(kind, act, t, variant, cfg=GEN, rows=256)
        torch.cuda.synchronize()
        full = out[0] if isinstance(out, tuple) else out
        part = gen[0] if isinstance(gen, tuple) else gen
        assert torch.equal(full[:256], part), "LDS-DMA and generic kernels differ on the 256-row slice"
        if isinstance(out, tuple):
            assert torch.equal(out[1][:256], gen[1])
