"""Pins the CPU oracle (``oracle/ipc_oracle.py``) before anything is checked against it.

Each check is chosen so that a plausible mistake fails it: independent
float64 loops (``oracle/ipc_brute.py``) catch wrong indices, transposes and
phase order; ``torch.autograd`` pins every activation derivative; closed forms
and invariants pin special cases.  The reference ships no golden vectors for
this path, so these checks are the anchor.
"""
import math

import pytest
import torch

from oracle import ipc_brute as brute
from oracle import ipc_oracle as O

ACTS = ["relu", "tanh", "sigmoid", "silu", "gelu", "identity"]


def _tol(a, b):
    return float((torch.as_tensor(a, dtype=torch.float64) - torch.as_tensor(b, dtype=torch.float64)).abs().max())


def _to_list(t):
    return t.double().tolist()


@pytest.mark.parametrize("act", ACTS)
def test_activation_values_match_math_module(act):
    xs = torch.linspace(-4, 4, 101, dtype=torch.float64)
    got = O.act_forward(act, xs)
    ref = torch.tensor([brute.f(act, float(v)) for v in xs], dtype=torch.float64)
    assert _tol(got, ref) < 1e-12


@pytest.mark.parametrize("act", ACTS)
def test_activation_derivative_matches_autograd(act):
    xs = torch.linspace(-4, 4, 97, dtype=torch.float64)  # avoids exactly 0 for relu
    xs = xs[xs != 0].clone().requires_grad_(True)
    y = O.act_forward(act, xs).sum()
    (g,) = torch.autograd.grad(y, xs)
    assert _tol(O.act_derivative(act, xs.detach()), g) < 1e-12
    ref = torch.tensor([brute.df(act, float(v)) for v in xs.detach()], dtype=torch.float64)
    assert _tol(O.act_derivative(act, xs.detach()), ref) < 1e-12


def test_relu_derivative_is_strict_at_zero():
    # activations.py:17 and tilelang_kernels.py:79 use x > 0.
    assert float(O.act_derivative("relu", torch.zeros(1))) == 0.0


def test_gelu_is_the_tanh_approximation():
    v = 1.3
    k = math.sqrt(2 / math.pi)
    expect = 0.5 * v * (1 + math.tanh(k * (v + 0.044715 * v ** 3)))
    assert abs(float(O.act_forward("gelu", torch.tensor([v], dtype=torch.float64))) - expect) < 1e-15


def test_one_hot_layout_is_classes_by_batch():
    y = O.one_hot(torch.tensor([2, 0, 1]), 4)
    assert y.shape == (4, 3)
    assert y[:, 0].tolist() == [0, 0, 1, 0] and y[:, 1].tolist() == [1, 0, 0, 0]


@pytest.mark.parametrize("init", ["kaiming_a_sqrt5", "xavier_uniform"])
def test_init_bounds_and_layer_order(init):
    dims = (10, 64, 64, 784)
    ws = O.init_weights(dims, seed=3, init=init)
    for w, (n_l, n_u) in zip(ws, zip(dims[:-1], dims[1:])):
        assert w.shape == (n_l, n_u)
        bound = 1 / math.sqrt(n_u) if init == "kaiming_a_sqrt5" else math.sqrt(6 / (n_l + n_u))
        assert float(w.abs().max()) <= bound * (1 + 1e-6)
        assert float(w.abs().max()) > 0.9 * bound  # uses the full range
    # one generator consumed strictly in layer order: the first layer does not
    # depend on later shapes, and the draw is reproducible from the seed.
    ws2 = O.init_weights((10, 64, 32, 784), seed=3, init=init)
    assert torch.equal(ws[0], ws2[0])
    assert torch.equal(O.init_weights(dims, seed=3, init=init)[2], ws[2])
    assert not torch.equal(O.init_weights(dims, seed=4, init=init)[0], ws[0])


def _tiny(act, seed=0, dims=(3, 4, 5, 6), B=2):
    torch.manual_seed(seed)
    ws = [torch.randn(a, b, dtype=torch.float64) * 0.5 for a, b in zip(dims[:-1], dims[1:])]
    xs = [torch.randn(d, B, dtype=torch.float64) for d in dims]
    return xs, ws


@pytest.mark.parametrize("act", ACTS)
def test_step_matches_brute_force_loops(act):
    xs, ws = _tiny(act, seed=11)
    nx, nw, e, _ = O.ipc_step(xs, ws, act=act, alpha=0.05, gamma=0.3)
    bx, bw, be = brute.step([_to_list(v) for v in xs], [_to_list(v) for v in ws], act, 0.05, 0.3)
    for a, b in zip(e, be):
        assert _tol(a, b) < 1e-12
    for a, b in zip(nx, bx):
        assert _tol(a, b) < 1e-12
    for a, b in zip(nw, bw):
        assert _tol(a, b) < 1e-12


def test_several_steps_match_brute_force():
    xs, ws = _tiny("tanh", seed=5, dims=(2, 3, 3, 4), B=3)
    bx, bw = [_to_list(v) for v in xs], [_to_list(v) for v in ws]
    for _ in range(3):
        xs, ws, _e, _m = O.ipc_step(xs, ws, act="tanh", alpha=0.1, gamma=0.5)
        bx, bw, _be = brute.step(bx, bw, "tanh", 0.1, 0.5)
    assert max(_tol(a, b) for a, b in zip(xs, bx)) < 1e-12
    assert max(_tol(a, b) for a, b in zip(ws, bw)) < 1e-12


def test_endpoints_stay_fixed():
    xs, ws = _tiny("tanh", seed=1)
    nx, _, _, _ = O.ipc_step(xs, ws, act="tanh", alpha=0.1, gamma=0.5)
    assert torch.equal(nx[0], xs[0]) and torch.equal(nx[-1], xs[-1])


def test_weight_update_uses_post_update_state():
    # reference.py:53-57: the weight update consumes the just-updated x[l+1].
    xs, ws = _tiny("tanh", seed=2)
    nx, nw, e, _ = O.ipc_step(xs, ws, act="tanh", alpha=0.1, gamma=0.5)
    l = 1
    post = ws[l] + 0.1 * e[l] @ torch.tanh(nx[l + 1]).T
    pre = ws[l] + 0.1 * e[l] @ torch.tanh(xs[l + 1]).T
    assert _tol(nw[l], post) < 1e-14
    assert _tol(nw[l], pre) > 1e-6


def test_special_cases():
    xs, ws = _tiny("sigmoid", seed=3)
    nx, nw, e, _ = O.ipc_step(xs, ws, act="sigmoid", alpha=0.0, gamma=0.0)
    assert all(torch.equal(a, b) for a, b in zip(nx, xs))
    assert all(torch.equal(a, b) for a, b in zip(nw, ws))
    zeros = [torch.zeros_like(w) for w in ws]
    e0 = O.prediction_errors(xs, zeros, "sigmoid")
    assert all(torch.equal(a, b) for a, b in zip(e0, xs[:-1]))
    # E_lower = 0 for every layer => x -= gamma * eps
    x_new, _ = O.infer_update(xs[1], e0[1], ws[0], torch.zeros_like(xs[0]), "sigmoid", 0.25)
    assert _tol(x_new, xs[1] - 0.25 * e0[1]) < 1e-15


def test_weight_delta_is_linear_in_alpha():
    xs, ws = _tiny("gelu", seed=4)
    _, w1, _, _ = O.ipc_step(xs, ws, act="gelu", alpha=1e-3, gamma=0.5)
    _, w2, _, _ = O.ipc_step(xs, ws, act="gelu", alpha=2e-3, gamma=0.5)
    for a, b, w0 in zip(w1, w2, ws):
        assert _tol(2 * (a - w0), b - w0) < 1e-15


def test_rank_b_outer_equals_gemm_sum():
    torch.manual_seed(0)
    w = torch.randn(5, 7, dtype=torch.float64)
    e = torch.randn(5, 3, dtype=torch.float64)
    xu = torch.randn(7, 3, dtype=torch.float64)
    outer = w.clone()
    for b in range(3):
        outer += 0.01 * torch.outer(e[:, b], torch.relu(xu[:, b]))
    assert _tol(O.weight_update(w, e, xu, "relu", 0.01), outer) < 1e-14
    assert _tol(O.weight_update(w, e, torch.relu(xu), "relu", 0.01, recompute=False), outer) < 1e-14


@pytest.mark.parametrize("depth,T", [(3, 2), (4, 4), (6, 4)])
def test_forward_init_wavefront_invariant(depth, T):
    """From the forward init, after t steps eps[l] == 0 exactly for l > t and
    x[l] is untouched for l > t; dW[l] == 0 exactly for l >= T."""
    dims = (10,) + (16,) * depth + (40,)
    ws = O.init_weights(dims, seed=1, init="xavier_uniform")
    x_in, _, y = O.make_batch(dims, 8, seed=1)
    x0 = O.forward_init(x_in, y, ws, "tanh")
    x, w = x0, ws
    for t in range(T):
        e = O.prediction_errors(x, w, "tanh")
        for l in range(t + 1, len(ws)):
            assert torch.count_nonzero(e[l]) == 0
        for l in range(t + 2, len(ws)):
            assert torch.equal(x[l], x0[l])
        x, w, _, _ = O.ipc_step(x, w, act="tanh", alpha=1e-4, gamma=0.5)
    for l in range(len(ws)):
        d = w[l] - ws[l]
        if l >= T:
            assert torch.count_nonzero(d) == 0
        else:
            assert torch.count_nonzero(d) > 0


def test_forward_init_matches_predict_chain():
    dims = (10, 16, 16, 40)
    ws = O.init_weights(dims, seed=2)
    x_in, _, y = O.make_batch(dims, 4, seed=2)
    x = O.forward_init(x_in, y, ws, "relu")
    assert torch.equal(x[0], y)
    assert _tol(x[1], ws[1] @ torch.relu(ws[2] @ torch.relu(x_in))) < 1e-6
    assert _tol(O.predict(ws, x_in, "relu"), ws[0] @ torch.relu(x[1])) < 1e-6


def test_global_rel_err():
    a = [torch.tensor([1.0, 2.0]), torch.tensor([0.0])]
    b = [torch.tensor([1.0, 4.0]), torch.tensor([0.0])]
    assert O.global_rel_err(a, b) == pytest.approx(0.5)
    assert O.global_rel_err([torch.zeros(2)], [torch.zeros(2)]) == 0.0


def test_flops_per_sample_matches_published_derivation():
    # 784->64^d->10: 253,696 / 278,272 / 327,424 flop per sample for d=3/4/6.
    assert O.flops_per_sample((10,) + (64,) * 3 + (784,)) == 253_696
    assert O.flops_per_sample((10,) + (64,) * 4 + (784,)) == 278_272
    assert O.flops_per_sample((10,) + (64,) * 6 + (784,)) == 327_424
    assert O.flops_per_sample((1000,) + (4096,) * 4 + (4096,)) == 393_674_752


SHAPES = [(1, 1, 1), (3, 5, 2), (7, 4, 3), (10, 13, 6)]


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64) * scale


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", SHAPES)
def test_single_kernel_helpers_match_loops(act, M, K, B):
    """The helpers the standalone-kernel GPU tests check against, each against
    the float64 loops on ragged shapes with non-zero errors everywhere
    (a transposed W_lower, a dropped -E term or f' taken of the wrong tensor
    changes these results)."""
    seed = 1000 * M + 10 * K + B
    xu, w, xl = _rand((K, B), seed), _rand((M, K), seed + 1, 0.5), _rand((M, B), seed + 2)
    e, wlo, elo = _rand((M, B), seed + 3), _rand((K, M), seed + 4, 0.5), _rand((K, B), seed + 5)
    got = O.pred_err(xu, w, xl, act)
    assert _tol(got, brute.pred_err(_to_list(xu), _to_list(w), _to_list(xl), act)) < 1e-12
    assert _tol(O.forward_pred(xu, w, act), brute.matmul_act(_to_list(w), _to_list(xu), act)) < 1e-12
    x_new, a_new = O.infer_update(xl, e, wlo, elo, act, 0.375)
    bx, ba = brute.infer_update(_to_list(xl), _to_list(e), _to_list(wlo), _to_list(elo), act, 0.375)
    assert _tol(x_new, bx) < 1e-12 and _tol(a_new, ba) < 1e-12
    a = [[brute.f(act, v) for v in row] for row in _to_list(xu)]
    assert _tol(O.weight_update(w, e, xu, act, 0.01), brute.weight_update(_to_list(w), _to_list(e), a, 0.01)) < 1e-12
    assert _tol(O.weight_update(w, e, torch.tensor(a, dtype=torch.float64), act, 0.01, recompute=False),
                brute.weight_update(_to_list(w), _to_list(e), a, 0.01)) < 1e-12


def test_single_kernel_helpers_special_cases():
    """Closed forms: W = 0 gives E = X_lower; relu of a negative X_upper gives
    E = X_lower; gamma = 0 leaves X; E_lower = 0 gives X - gamma E; a W_lower
    that is not square exposes a transposed read."""
    xu, w, xl = _rand((5, 3), 1), _rand((4, 5), 2), _rand((4, 3), 3)
    assert torch.equal(O.pred_err(xu, torch.zeros_like(w), xl, "tanh"), xl)
    assert torch.equal(O.pred_err(-xu.abs() - 1, w, xl, "relu"), xl)
    e, wlo, elo = _rand((4, 3), 4), _rand((6, 4), 5), _rand((6, 3), 6)
    assert torch.equal(O.infer_update(xl, e, wlo, elo, "silu", 0.0)[0], xl)
    assert _tol(O.infer_update(xl, e, wlo, torch.zeros_like(elo), "silu", 0.5)[0], xl - 0.5 * e) < 1e-15
    with pytest.raises(RuntimeError):
        O.infer_update(xl, e, wlo.T.contiguous(), elo, "silu", 0.5)


def test_global_rel_err_never_reads_nan_as_agreement():
    a = [torch.ones(3), torch.tensor([1.0, float("nan")])]
    b = [torch.ones(3), torch.tensor([1.0, 2.0])]
    assert O.global_rel_err(a, b) == float("inf")
    assert O.global_rel_err(b, a) == float("inf")
    assert O.global_rel_err(b, b) == 0.0


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("T", [1, 3])
def test_run_steps_matches_brute_force_loops(act, T):
    """``run_steps`` (the T-step driver every whole-step GPU test compares
    with) against ``brute.step`` looped T times: a driver that skipped the
    last step, fed back the pre-update W or x, or returned the first step's
    errors instead of the last fails this."""
    xs, ws = _tiny(act, seed=40 + T, dims=(3, 4, 5, 6), B=2)
    gx, gw, ge = O.run_steps(xs, ws, T, act=act, alpha=0.07, gamma=0.4)
    bx, bw = [_to_list(v) for v in xs], [_to_list(v) for v in ws]
    be = None
    for _ in range(T):
        bx, bw, be = brute.step(bx, bw, act, 0.07, 0.4)
    assert max(_tol(a, b) for a, b in zip(gx, bx)) < 1e-12
    assert max(_tol(a, b) for a, b in zip(gw, bw)) < 1e-12
    assert max(_tol(a, b) for a, b in zip(ge, be)) < 1e-12
    # the inputs are not modified in place
    xs2, ws2 = _tiny(act, seed=40 + T, dims=(3, 4, 5, 6), B=2)
    assert all(torch.equal(a, b) for a, b in zip(xs, xs2)) and all(torch.equal(a, b) for a, b in zip(ws, ws2))


def test_run_steps_zero_steps_is_the_identity():
    xs, ws = _tiny("tanh", seed=9)
    gx, gw, ge = O.run_steps(xs, ws, 0, act="tanh", alpha=0.1, gamma=0.5)
    assert ge is None
    assert all(torch.equal(a, b) for a, b in zip(gx, xs)) and all(torch.equal(a, b) for a, b in zip(gw, ws))


@pytest.mark.parametrize("act", ["tanh", "relu"])
def test_step_metrics_and_frozen_weights_match_loops(act):
    """``reference.py:58``: energy = sum over l < L of mean(eps[l]^2) and the
    largest |eps| over the same layers; ``update_weights=False`` still updates
    the states and leaves every W untouched (``reference.py:52``)."""
    xs, ws = _tiny(act, seed=17)
    nx, nw, _e, m = O.ipc_step(xs, ws, act=act, alpha=0.05, gamma=0.3, update_weights=False)
    bx, _bw, be = brute.step([_to_list(v) for v in xs], [_to_list(v) for v in ws], act, 0.05, 0.3)
    energy = sum(sum(v * v for row in el for v in row) / (len(el) * len(el[0])) for el in be)
    biggest = max(abs(v) for el in be for row in el for v in row)
    assert abs(m["energy"] - energy) < 1e-12 and abs(m["max_abs_error"] - biggest) < 1e-12
    assert all(torch.equal(a, b) for a, b in zip(nw, ws))
    assert max(_tol(a, b) for a, b in zip(nx, bx)) < 1e-12


def test_operand_emulation_reduces_to_the_oracle_at_fp32():
    """``oracle/emulate.py`` with fp32 operands rounds nothing and its lo
    terms are exactly zero, so every split gives the oracle's step, forward
    initialisation and T-step run (in float32 arithmetic, the same order of
    operations: bit for bit)."""
    from oracle import emulate as E

    dims = (10, 16, 16, 40)
    ws = O.init_weights(dims, seed=5, init="xavier_uniform")
    x_in, _lab, y = O.make_batch(dims, 6, seed=5)
    x0 = O.forward_init(x_in, y, ws, "tanh")
    for split in (1, 2, 3):
        xe = E.forward_init_operand16(x_in, y, ws, act="tanh", op=torch.float32, split=split)
        assert all(torch.equal(a, b) for a, b in zip(xe[1:], x0[1:]))
        sx, sw, se = E.step_operand16(x0, ws, act="tanh", alpha=1e-2, gamma=0.5, op=torch.float32, split=split)
        ox, ow, oe, _m = O.ipc_step(x0, ws, act="tanh", alpha=1e-2, gamma=0.5)
        assert all(torch.equal(a, b) for a, b in zip(sx, ox))
        assert all(torch.equal(a, b) for a, b in zip(sw, ow))
        assert all(torch.equal(a, b) for a, b in zip(se, oe))
    rx, rw = E.run(E.step_operand16, x0, ws, 3, act="tanh", alpha=1e-2, gamma=0.5, op=torch.float32)
    ox, ow, _oe = O.run_steps(x0, ws, 3, act="tanh", alpha=1e-2, gamma=0.5)
    assert all(torch.equal(a, b) for a, b in zip(rx, ox)) and all(torch.equal(a, b) for a, b in zip(rw, ow))
    # and with 16-bit operands it does round: the emulation is not the oracle there
    bx, _bw, _be = E.step_operand16(x0, ws, act="tanh", alpha=1e-2, gamma=0.5, op=torch.bfloat16)
    assert not all(torch.equal(a, b) for a, b in zip(bx[1:-1], ox[1:-1]))


def test_every_oracle_function_is_exercised():
    """Each public function of ``oracle/ipc_oracle.py`` is called by a test in
    this file, so no oracle function is left without a pin."""
    import inspect
    from pathlib import Path

    src = Path(__file__).read_text()
    names = [n for n, f in inspect.getmembers(O, inspect.isfunction)
             if f.__module__ == O.__name__ and not n.startswith("_")]
    missing = [n for n in names if f"O.{n}(" not in src]
    assert not missing, missing
