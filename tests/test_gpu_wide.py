"""The wide GEMM path (IPC_PATH_WIDE) against the oracle, against the rounding
model of its operand design (oracle/emulate.py) and against the phased path.

The wide path computes with the same 16-bit operand values as the phased path
(16-bit copies of W, W^T, eps and f(x) written by the epilogues instead of
conversions in the loaders); only the fp32 accumulation order differs.  Its
forward initialisation uses the prediction kernel itself, so the first
step's prediction errors above the wavefront are exactly zero, as on the
other paths.
"""
import pytest
import torch

from lich_amd.trainer import HipIPC, IPCConfig
from oracle import ipc_oracle as O
from tests.helpers import DEV, report
from tests.test_gpu_trainer import _errors, _gate_fraction, _model_run, _oracle_run, _setup

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16


def _model(dims, B, act, op, path, w0, x_in, y, T, **cfg):
    m = HipIPC(IPCConfig(dims=dims, activation=act, dtype=op, fused=path, **cfg), device=DEV, weights=w0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    m.run_steps(T)
    torch.cuda.synchronize()
    return m


# dims, B, act, operand, split, recompute, input distribution
CASES = [
    ((10, 300, 200, 784), 128, "tanh", BF16, 2, True, "uniform"),
    ((10, 300, 200, 784), 128, "tanh", F16, 1, False, "uniform"),
    ((33, 520, 129, 300, 64), 100, "silu", BF16, 2, False, "normal"),
    ((1000, 1024, 1024, 1000), 256, "gelu", BF16, 2, True, "normal"),
    ((10, 784), 64, "sigmoid", F16, 2, True, "uniform"),           # L = 1: no inference phase
    ((7, 130, 65, 257), 37, "tanh", F16, 2, True, "uniform"),       # ragged: no tile/vector alignment
    ((10,) + (300,) * 17 + (784,), 64, "tanh", BF16, 2, True, "uniform"),  # 18 layers: chunked launches
    # every contraction a multiple of 64: the split-2 prediction reads the fp32 W itself
    ((10, 256, 192, 768), 128, "tanh", BF16, 2, True, "uniform"),
]


def _id(c):
    dims, B, act, op, split, rec, dist = c
    return f"L{len(dims) - 1}-{dims[0]}x{max(dims)}-B{B}-{act}-{str(op)[6:]}-s{split}-{'rec' if rec else 'save'}"


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_wide_matches_oracle_and_rounding_model(case):
    dims, B, act, op, split, rec, dist = case
    T = 4
    report("wide-oracle", case=_id(case))
    w0, x_in, y = _setup(dims, B, seed=3, input_dist=dist)
    _x0, x_t, w_t, _e = _oracle_run(w0, x_in, y, act, T)
    m = _model(dims, B, act, op, "wide", w0, x_in, y, T, pred_split=split, recompute_activation=rec)
    assert m.path == "wide" and m.launches_per_step() == (3 if len(dims) > 2 else 2) * (1 + (len(dims) - 2) // 16)
    s_err, dw_err = _errors(m, w0, x_t, w_t)
    x_m, w_m = _model_run(dims, w0, x_in, y, act, T, op, split)
    s_m, dw_m = _errors(m, w0, x_m, w_m)
    print(f"wide {_id(case)}: oracle state={s_err:.3e} dW={dw_err:.3e} | model state={s_m:.3e} dW={dw_m:.3e}")
    assert s_err <= 2e-2 and dw_err <= 5e-3
    # The rounding model predicts the GPU up to fp32 summation-order noise,
    # which the eps << W f(x) cancellation of the hidden layers amplifies in
    # eps and dW (the phased path shows the same distance to the model).
    assert s_m <= 2.5e-3 and dw_m <= 2.5e-3


def test_wide_relu_gate():
    """relu states get the reference's own gate (see test_c2_relu_fp16_operands)."""
    dims, B, T = (10, 300, 200, 784), 128, 4
    report("wide-relu", dims=dims)
    w0, x_in, y = _setup(dims, B, seed=5)
    _x0, x_t, w_t, _e = _oracle_run(w0, x_in, y, "relu", T)
    m = _model(dims, B, "relu", F16, "wide", w0, x_in, y, T)
    s_err, dw_err = _errors(m, w0, x_t, w_t)
    frac = _gate_fraction(m.x[1:-1], x_t[1:-1])
    print(f"wide relu: state={s_err:.3e} gate_frac={frac:.2e} dW={dw_err:.3e}")
    assert dw_err <= 5e-3 and frac <= 0.01


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[5], CASES[7]], ids=_id)
def test_wide_equals_phased_path(case):
    """Same 16-bit operands, different fp32 summation order: states and weights
    agree to the fp32 bar, errors and weight deltas (small differences of
    large terms) to 1e-4."""
    dims, B, act, op, split, rec, dist = case
    T = 3
    report("wide-vs-phased", case=_id(case))
    w0, x_in, y = _setup(dims, B, seed=9, input_dist=dist)
    kw = dict(pred_split=split, recompute_activation=rec)
    wd = _model(dims, B, act, op, "wide", w0, x_in, y, T, **kw)
    ph = _model(dims, B, act, op, "phased", w0, x_in, y, T, **kw)
    assert wd.path == "wide" and ph.path == "phased"
    L = len(dims) - 1
    s = O.global_rel_err(wd.x[1:-1], ph.x[1:-1]) if L > 1 else 0.0
    w = O.global_rel_err(wd.w, ph.w)
    e = O.global_rel_err(wd.e[:-1], ph.e[:-1])
    dw = O.global_rel_err([wd.w[l].double() - w0[l].to(DEV).double() for l in range(L)],
                          [ph.w[l].double() - w0[l].to(DEV).double() for l in range(L)])
    print(f"wide vs phased {_id(case)}: x={s:.2e} w={w:.2e} e={e:.2e} dW={dw:.2e}")
    assert s <= 1e-5 and w <= 1e-5 and e <= 1e-4 and dw <= 1e-4


@pytest.mark.parametrize("op,split", [(BF16, 2), (F16, 1)], ids=["bf16-s2", "f16-s1"])
def test_wide_k_split_prediction(op, split):
    """Layer 0 (999 rows, K = 4096) after the whole tiles of layer 1 (K = 512):
    the plan cuts layer 0's prediction tiles into k-slices that fill the CUs
    left idle by the whole tiles, and a fourth launch adds the slices' partial
    products (ragged: M = 999 and B = 1000 end inside a tile), for both
    default prediction tile configurations (split 2: 128 x 256, split 1: 256 x 128).

    The first step's prediction sees the same operands on both paths, so its
    eps[0] differs from the unsplit phased path only by the fp32 summation
    order.  Later steps round those differences into the 16-bit operand
    copies (an element on a rounding boundary moves by one 16-bit ulp), so
    from there on the paths are compared through their distance to the
    oracle, which the split must not increase."""
    dims, B, act, T = (999, 4096, 512), 1000, "tanh", 4
    report("wide-k-split", dims=dims, B=B, op=op, split=split)
    w0, x_in, y = _setup(dims, B, seed=11, input_dist="normal")
    _x0, x_t, w_t, _e = _oracle_run(w0, x_in, y, act, T)
    m = _model(dims, B, act, op, "wide", w0, x_in, y, 1, pred_split=split)
    ph = _model(dims, B, act, op, "phased", w0, x_in, y, 1, pred_split=split)
    assert m.path == "wide" and m.launches_per_step() == 4
    e1 = O.global_rel_err([m.e[0]], [ph.e[0]])
    for mod in (m, ph):
        mod.run_steps(T - 1)
    torch.cuda.synchronize()
    s_err, dw_err = _errors(m, w0, x_t, w_t)
    s_ph, dw_ph = _errors(ph, w0, x_t, w_t)
    x_m, w_m = _model_run(dims, w0, x_in, y, act, T, op, split)
    s_m, dw_m = _errors(m, w0, x_m, w_m)
    print(f"wide k-split {op} split {split}: step-1 eps[0] vs phased {e1:.2e} | oracle state={s_err:.3e} "
          f"dW={dw_err:.3e} (phased {s_ph:.3e} {dw_ph:.3e}) | model state={s_m:.3e} dW={dw_m:.3e}")
    assert e1 <= 1e-5
    assert s_err <= 2e-2 and dw_err <= 5e-3
    assert s_err <= 1.1 * s_ph + 1e-4 and dw_err <= 1.1 * dw_ph + 1e-4
    assert s_m <= 2.5e-3 and dw_m <= 2.5e-3


def test_wide_forward_init_wavefront_is_exact():
    dims, B, T = (10, 300, 300, 300, 300, 784), 128, 3
    w0, x_in, y = _setup(dims, B, seed=7)
    m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=BF16, fused="wide"), device=DEV, weights=w0)
    m.initialize_batch(x_in.to(DEV), y.to(DEV))
    x0 = [t.clone() for t in m.x]
    for t in range(T):
        m.step_initialized()
        torch.cuda.synchronize()
        for l in range(t + 1, m.L):
            assert torch.count_nonzero(m.e[l]) == 0, (t, l)
        for l in range(t + 2, m.L):
            assert torch.equal(m.x[l], x0[l]), (t, l)
    for l in range(m.L):
        nz = torch.count_nonzero(m.w[l].cpu() - w0[l])
        assert (nz == 0) if l >= T else (nz > 0), l


def test_wide_graph_replay_equals_direct_bitwise():
    dims, B, T = (10, 300, 200, 784), 128, 4
    w0, x_in, y = _setup(dims, B, seed=13)
    direct = _model(dims, B, "tanh", BF16, "wide", w0, x_in, y, 0)
    for _ in range(3):
        direct.run_steps(T)
    graph = _model(dims, B, "tanh", BF16, "wide", w0, x_in, y, 0)
    runner = graph.capture_graph(T)
    for _ in range(3):
        runner.replay()
        torch.cuda.synchronize()  # eager work between replays
    torch.cuda.synchronize()
    for a, b in zip(direct.x + direct.e[:-1] + direct.w, graph.x + graph.e[:-1] + graph.w):
        assert torch.equal(a, b)


def test_wide_sync_after_external_weight_write():
    """Masters written outside a step must be followed by sync_operand_copies();
    the result then equals the phased path with the same edit."""
    dims, B, T = (10, 300, 200, 784), 128, 2
    w0, x_in, y = _setup(dims, B, seed=17)
    models = {}
    for path in ("wide", "phased"):
        m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=BF16, fused=path), device=DEV, weights=w0)
        m.initialize_batch(x_in.to(DEV), y.to(DEV))
        m.w[1].mul_(1.01)
        m.x[2].add_(0.01)
        m.sync_operand_copies()
        m.run_steps(T)
        models[path] = m
    torch.cuda.synchronize()
    wd, ph = models["wide"], models["phased"]
    assert O.global_rel_err(wd.x[1:-1], ph.x[1:-1]) <= 1e-5
    assert O.global_rel_err(wd.w, ph.w) <= 1e-5


def test_wide_torch_writes_need_no_sync_call():
    """Writes of W and x that torch counts re-derive the wide path's operand
    copies before the next launch by themselves: the same edits with and
    without sync_operand_copies() give the same bits, and the phased path
    (no copies) agrees to the fp32 bar."""
    dims, B, T = (10, 300, 200, 784), 128, 2
    report("wide-torch-writes", dims=dims, B=B)
    w0, x_in, y = _setup(dims, B, seed=19)
    x_in2 = torch.randn((dims[-1], B), generator=torch.Generator().manual_seed(20))
    models = {}
    for name, path, explicit in (("auto", "wide", False), ("explicit", "wide", True), ("phased", "phased", False)):
        m = HipIPC(IPCConfig(dims=dims, activation="tanh", dtype=BF16, fused=path), device=DEV, weights=w0)
        m.initialize_batch(x_in.to(DEV), y.to(DEV))
        m.run_steps(T)
        m.w[1].mul_(1.01)
        m.x[2].add_(0.01)
        if explicit:
            m.sync_operand_copies()
        m.run_steps(T)
        m.x[-1].copy_(x_in2.to(DEV))
        m.w[0][:16].mul_(0.5)
        if explicit:
            m.sync_operand_copies()
        m.run_steps(T)
        models[name] = m
    torch.cuda.synchronize()
    au, ex, ph = models["auto"], models["explicit"], models["phased"]
    assert au.path == ex.path == "wide"
    for u, v in zip(au.x + au.w + au.e[:-1], ex.x + ex.w + ex.e[:-1]):
        assert torch.equal(u, v)
    assert O.global_rel_err(au.x[1:-1], ph.x[1:-1]) <= 1e-5
    assert O.global_rel_err(au.w, ph.w) <= 1e-5
