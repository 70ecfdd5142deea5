"""Independent float64 pure-Python loops for tiny iPC problems (test infrastructure).

Written from the equations of the reference ``README.md:41-50`` and the
activation definitions of ``src/ipc_tilelang/activations.py:9-29`` with the
``math`` module only (no torch), so that a mistake in ``ipc_oracle`` (a wrong
index, a transposed operand, a dropped term, the wrong phase order) shows up
as a mismatch.  Lists of lists, row-major, ``[rows][cols]``.
"""
from __future__ import annotations

import math


def _sig(v: float) -> float:
    if v >= 0:
        return 1.0 / (1.0 + math.exp(-v))
    ev = math.exp(v)
    return ev / (1.0 + ev)


def f(name: str, v: float) -> float:
    if name == "relu":
        return v if v > 0 else 0.0
    if name == "tanh":
        return math.tanh(v)
    if name == "sigmoid":
        return _sig(v)
    if name == "silu":
        return v * _sig(v)
    if name == "gelu":
        k = math.sqrt(2.0 / math.pi)
        return 0.5 * v * (1.0 + math.tanh(k * (v + 0.044715 * v ** 3)))
    if name == "identity":
        return v
    raise ValueError(name)


def df(name: str, v: float) -> float:
    if name == "relu":
        return 1.0 if v > 0 else 0.0
    if name == "tanh":
        return 1.0 - math.tanh(v) ** 2
    if name == "sigmoid":
        s = _sig(v)
        return s * (1.0 - s)
    if name == "silu":
        s = _sig(v)
        return s + v * s * (1.0 - s)
    if name == "gelu":
        k = math.sqrt(2.0 / math.pi)
        u = k * (v + 0.044715 * v ** 3)
        t = math.tanh(u)
        return 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t * t) * k * (1.0 + 3 * 0.044715 * v * v)
    if name == "identity":
        return 1.0
    raise ValueError(name)


def matmul_act(w, x, act):
    """``W @ f(X)`` by loops."""
    M, K, B = len(w), len(x), len(x[0])
    return [[sum(w[m][k] * f(act, x[k][b]) for k in range(K)) for b in range(B)] for m in range(M)]


def step(x, w, act: str, alpha: float, gamma: float):
    """One step by loops; returns ``(new_x, new_w, eps)``."""
    L = len(w)
    B = len(x[0][0])
    eps = []
    for l in range(L):
        pred = matmul_act(w[l], x[l + 1], act)
        eps.append([[x[l][m][b] - pred[m][b] for b in range(B)] for m in range(len(x[l]))])
    new_x = [[row[:] for row in xl] for xl in x]
    for l in range(1, L):
        d_lo = len(x[l - 1])
        for m in range(len(x[l])):
            for b in range(B):
                sig = sum(w[l - 1][k][m] * eps[l - 1][k][b] for k in range(d_lo))
                new_x[l][m][b] = x[l][m][b] + gamma * (-eps[l][m][b] + df(act, x[l][m][b]) * sig)
    new_w = [[row[:] for row in wl] for wl in w]
    for l in range(L):
        for m in range(len(w[l])):
            for k in range(len(w[l][0])):
                new_w[l][m][k] = w[l][m][k] + alpha * sum(
                    eps[l][m][b] * f(act, new_x[l + 1][k][b]) for b in range(B))
    return new_x, new_w, eps


# ---------------------------------------------------------------------------
# single kernels of the operator API (tilelang_kernels.py:114-349), by loops
# ---------------------------------------------------------------------------
def pred_err(x_upper, w, x_lower, act: str):
    """``E[m][b] = X_lower[m][b] - sum_k W[m][k] f(X_upper[k][b])``."""
    pred = matmul_act(w, x_upper, act)
    return [[x_lower[m][b] - pred[m][b] for b in range(len(x_lower[0]))] for m in range(len(x_lower))]


def infer_update(x, e, w_lower, e_lower, act: str, gamma: float):
    """``X_new[m][b] = X + gamma(-E + f'(X) sum_k W_lower[k][m] E_lower[k][b])``
    with ``W_lower`` of shape ``[K][M]``; returns ``(X_new, f(X_new))``."""
    M, B, K = len(x), len(x[0]), len(e_lower)
    x_new = [[x[m][b] + gamma * (-e[m][b] + df(act, x[m][b]) * sum(w_lower[k][m] * e_lower[k][b] for k in range(K)))
              for b in range(B)] for m in range(M)]
    return x_new, [[f(act, v) for v in row] for row in x_new]


def weight_update(w, e, a, alpha: float):
    """``W[m][k] + alpha sum_b E[m][b] A[k][b]`` (``A`` already activated)."""
    return [[w[m][k] + alpha * sum(e[m][b] * a[k][b] for b in range(len(e[0]))) for k in range(len(w[0]))]
            for m in range(len(w))]
