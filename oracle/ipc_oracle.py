"""Torch-CPU restatement of the reference iPC step (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg use this module, as the checker.  The product package never imports it.

Conventions (reference ``README.md:41-50``, ``src/ipc_tilelang/reference.py:35-59``):

* ``x[0]`` is the fixed one-hot target, ``x[L]`` the fixed input;
* ``W[l]`` has shape ``[d_l, d_{l+1}]`` and maps ``f(x[l+1]) -> x[l]``;
* tensors are feature-major ``[features, batch]``;
* one step is::

      eps[l] = x[l] - W[l] @ f(x[l+1])                          l = 0..L-1
      x[l]  += gamma * (-eps[l] + f'(x[l]) * (W[l-1]^T @ eps[l-1]))   l = 1..L-1
      W[l]  += alpha * eps[l] @ f(x_new[l+1])^T                  l = 0..L-1

  where the state update reads time-t ``x, W, eps`` and the weight update
  reads the just-updated ``x`` (``reference.py:45-57``).

Parity status: ``tests/test_oracle.py`` calls every function here and pins
each one against the independent float64 loops of ``oracle/ipc_brute.py``
(``ipc_step``, ``run_steps`` over one and three steps, the single-kernel
helpers), against ``torch.autograd`` (activation derivatives) and against
closed forms and invariants (forward-init wavefront, gamma=0, alpha=0, W=0,
linearity, phase order, the kaiming / Xavier bounds, the one-hot layout).
``tests/test_oracle.py::test_every_oracle_function_is_exercised`` fails if a
function is added here without a test that calls it.
"""
from __future__ import annotations

import math
from typing import Sequence

import torch

ACTIVATIONS = ("relu", "tanh", "sigmoid", "silu", "gelu", "identity")
_GELU_C = 0.044715
_GELU_K = math.sqrt(2.0 / math.pi)


# ---------------------------------------------------------------------------
# activations (src/ipc_tilelang/activations.py:9-29, tilelang_kernels.py:61-96)
# ---------------------------------------------------------------------------
def act_forward(name: str, x: torch.Tensor) -> torch.Tensor:
    """f(x); follows ``activations.py:9-15``.  ``identity`` is the linear
    activation accepted by ``weight_update_specialization.py:96-102``."""
    if name == "relu":
        return torch.relu(x)
    if name == "tanh":
        return torch.tanh(x)
    if name == "sigmoid":
        return torch.sigmoid(x)
    if name == "silu":
        return torch.nn.functional.silu(x)
    if name == "gelu":
        return torch.nn.functional.gelu(x, approximate="tanh")
    if name == "identity":
        return x
    raise ValueError(f"Unsupported activation: {name!r}")


def act_derivative(name: str, x: torch.Tensor) -> torch.Tensor:
    """f'(x); follows ``activations.py:16-29``.  relu' is the strict ``x > 0``."""
    if name == "relu":
        return (x > 0).to(x.dtype)
    if name == "tanh":
        y = torch.tanh(x)
        return 1 - y * y
    if name == "sigmoid":
        y = torch.sigmoid(x)
        return y * (1 - y)
    if name == "silu":
        s = torch.sigmoid(x)
        return s * (1 + x * (1 - s))
    if name == "gelu":
        u = _GELU_K * (x + _GELU_C * x * x * x)
        t = torch.tanh(u)
        du = _GELU_K * (1 + 3 * _GELU_C * x * x)
        return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * du
    if name == "identity":
        return torch.ones_like(x)
    raise ValueError(f"Unsupported activation: {name!r}")


# ---------------------------------------------------------------------------
# inputs and initialisation
# ---------------------------------------------------------------------------
def one_hot(labels: torch.Tensor, num_classes: int, *, dtype=torch.float32) -> torch.Tensor:
    """``[C, B]`` one-hot targets; follows ``reference.py:12-13``."""
    return torch.nn.functional.one_hot(labels.long(), num_classes=num_classes).to(dtype).T.contiguous()


def init_weights(dims: Sequence[int], *, seed: int = 0, init: str = "kaiming_a_sqrt5",
                 dtype=torch.float32) -> list[torch.Tensor]:
    """Seeded weights drawn in layer order from one CPU generator.

    ``kaiming_a_sqrt5`` follows ``reference.py:15-22`` / ``trainer.py:97-108``
    (``kaiming_uniform_(a=sqrt(5))``: bound ``1/sqrt(d_{l+1})``);
    ``xavier_uniform`` is the initialisation named by the paper-profile
    configurations (bound ``sqrt(6/(d_l+d_{l+1}))``).
    """
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    out = []
    for n_l, n_u in zip(dims[:-1], dims[1:]):
        w = torch.empty((int(n_l), int(n_u)), dtype=torch.float32)
        if init == "kaiming_a_sqrt5":
            torch.nn.init.kaiming_uniform_(w, a=5 ** 0.5, generator=g)
        elif init == "xavier_uniform":
            torch.nn.init.xavier_uniform_(w, generator=g)
        else:
            raise ValueError(f"Unknown init {init!r}")
        out.append(w.to(dtype))
    return out


def make_batch(dims: Sequence[int], batch: int, *, seed: int = 0, input_dist: str = "uniform",
               dtype=torch.float32) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Seeded synthetic batch: input ``[d_L, B]`` (U[0,1] or N(0,1)), labels
    ``[B]`` uniform over ``d_0`` classes, one-hot target ``[d_0, B]``."""
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed) + 7919)
    if input_dist == "uniform":
        x_in = torch.rand((int(dims[-1]), int(batch)), generator=g)
    elif input_dist == "normal":
        x_in = torch.randn((int(dims[-1]), int(batch)), generator=g)
    else:
        raise ValueError(f"Unknown input distribution {input_dist!r}")
    labels = torch.randint(0, int(dims[0]), (int(batch),), generator=g)
    return x_in.to(dtype), labels, one_hot(labels, int(dims[0]), dtype=dtype)


def forward_init(x_input: torch.Tensor, y_target: torch.Tensor, w: Sequence[torch.Tensor],
                 act: str) -> list[torch.Tensor]:
    """Trainer semantics (``trainer.py:509-516``): ``x[L]`` = input, hidden
    ``x[l] = W[l] f(x[l+1])`` from the top down, ``x[0]`` = target."""
    L = len(w)
    x: list[torch.Tensor] = [None] * (L + 1)  # type: ignore[list-item]
    x[L] = x_input.clone()
    for l in reversed(range(L)):
        pred = w[l] @ act_forward(act, x[l + 1])
        x[l] = pred if l > 0 else None  # type: ignore[assignment]
    x[0] = y_target.clone()
    return x


# ---------------------------------------------------------------------------
# the step (reference.py:35-59)
# ---------------------------------------------------------------------------
def prediction_errors(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], act: str) -> list[torch.Tensor]:
    """``eps[l] = x[l] - W[l] @ f(x[l+1])`` for l = 0..L-1 (``reference.py:35-40``)."""
    return [x[l] - w[l] @ act_forward(act, x[l + 1]) for l in range(len(w))]


def ipc_step(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], *, act: str, alpha: float,
             gamma: float, update_weights: bool = True):
    """One iPC step; follows ``reference.py:42-59``.

    Returns ``(new_x, new_w, eps, metrics)``; ``metrics`` holds the
    reference's ``energy`` (sum of per-layer mean squared errors) and
    ``max_abs_error`` over ``eps[0..L-1]``.
    """
    L = len(w)
    e = prediction_errors(x, w, act)
    new_x = [v.clone() for v in x]
    for l in range(1, L):
        signal = w[l - 1].T @ e[l - 1]
        new_x[l] = x[l] + gamma * (-e[l] + act_derivative(act, x[l]) * signal)
    new_w = [v.clone() for v in w]
    if update_weights:
        for l in range(L):
            new_w[l] = w[l] + alpha * (e[l] @ act_forward(act, new_x[l + 1]).T)
    metrics = {
        "energy": float(sum((q.double() ** 2).mean() for q in e)),
        "max_abs_error": float(max(q.abs().max() for q in e)),
    }
    return new_x, new_w, e, metrics


def run_steps(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], steps: int, *, act: str,
              alpha: float, gamma: float):
    """``steps`` consecutive ``ipc_step`` calls; returns ``(x, w, eps_last)``."""
    x = list(x)
    w = list(w)
    e = None
    for _ in range(int(steps)):
        x, w, e, _m = ipc_step(x, w, act=act, alpha=alpha, gamma=gamma)
    return x, w, e


def predict(w: Sequence[torch.Tensor], x_input: torch.Tensor, act: str) -> torch.Tensor:
    """Forward pass ``h = W[l] f(h)`` from the input down (``trainer.py:828-833``)."""
    h = x_input
    for l in reversed(range(len(w))):
        h = w[l] @ act_forward(act, h)
    return h


# ---------------------------------------------------------------------------
# single-kernel semantics (tilelang_kernels.py, weight_update_specialization.py)
# ---------------------------------------------------------------------------
def pred_err(x_upper, w, x_lower, act: str):
    """``E = X_lower - W @ f(X_upper)`` (``tilelang_kernels.py:114-177``)."""
    return x_lower - w @ act_forward(act, x_upper)


def forward_pred(x_upper, w, act: str):
    """``OUT = W @ f(X_upper)`` (forward init ``trainer.py:512-515``, ``predict``)."""
    return w @ act_forward(act, x_upper)


def infer_update(x, e, w_lower, e_lower, act: str, gamma: float):
    """``X + gamma(-E + f'(X) * W_lower^T @ E_lower)``; also returns ``f(X_new)``
    (``tilelang_kernels.py:180-265``).  ``w_lower`` is ``[K, M]``."""
    x_new = x + gamma * (-e + act_derivative(act, x) * (w_lower.T @ e_lower))
    return x_new, act_forward(act, x_new)


def weight_update(w, e, x_upper, act: str, alpha: float, recompute: bool = True):
    """``W + alpha * E @ A^T`` with ``A = f(X_upper)`` (recompute) or the saved
    ``A`` (``tilelang_kernels.py:268-349``).  The rank-B outer-product path
    (``weight_update_specialization.py:63-128``) computes the same sum; the
    reference's ``-alpha`` there is a sign error and the ``+alpha`` of the
    GEMM path and of ``reference.py:57`` is the one restated."""
    a = act_forward(act, x_upper) if recompute else x_upper
    return w + alpha * (e @ a.T)


# ---------------------------------------------------------------------------
# metrics
# ---------------------------------------------------------------------------
def global_rel_err(got: Sequence[torch.Tensor], ref: Sequence[torch.Tensor]) -> float:
    """max over tensors of ``|got - ref|`` divided by max over tensors of ``|ref|``.

    Normalised globally because after T steps from the forward init the top
    layers' weight deltas are exactly zero, which makes a per-layer relative
    error undefined.
    """
    num = 0.0
    den = 0.0
    for g, r in zip(got, ref):
        g64 = g.detach().double().cpu()
        r64 = r.detach().double().cpu()
        if not (bool(torch.isfinite(g64).all()) and bool(torch.isfinite(r64).all())):
            return float("inf")  # a NaN would otherwise drop out of max() and read as agreement
        num = max(num, float((g64 - r64).abs().max()) if g64.numel() else 0.0)
        den = max(den, float(r64.abs().max()) if r64.numel() else 0.0)
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def flops_per_sample(dims: Sequence[int]) -> int:
    """GEMM flops per sample per iPC step: ``2*(2S + S_I)`` with
    ``S = sum d_l d_{l+1}`` (prediction and weight update) and ``S_I`` the
    same sum without the input edge (inference update, l = 1..L-1)."""
    S = sum(int(a) * int(b) for a, b in zip(dims[:-1], dims[1:]))
    S_I = S - int(dims[-2]) * int(dims[-1])
    return 2 * (2 * S + S_I)
