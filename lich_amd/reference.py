"""The reference's pure-PyTorch iPC step as a public API (drop-in for
``ipc_tilelang.reference`` and ``ipc_tilelang.activations``).

Callers of the reference use these names to compute CPU trajectories
(``scripts/validate_reference.py``) and to check kernels; ``python -m
lich_amd.cli reference`` runs that trajectory.  Nothing in the trainer or the
kernel API calls this module: the training path runs only on the HIP library
and has no CPU fallback.

Semantics (``reference.py:12-59``, ``activations.py:6-35``): tensors are
``[features, batch]``; one step computes every prediction error from the
time-t states, updates the hidden states from the time-t errors, and updates
the weights with the updated states; the two end states are clamped to the
given target and input.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import torch

_GELU_K = math.sqrt(2.0 / math.pi)


@dataclass(frozen=True)
class ActivationSpec:
    """f and f' of one activation, evaluated in the tensor's dtype."""

    name: str

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = self.name
        if n == "relu":
            return x.clamp_min(0)
        if n == "tanh":
            return torch.tanh(x)
        if n == "sigmoid":
            return torch.sigmoid(x)
        if n == "silu":
            return x * torch.sigmoid(x)
        if n == "gelu":
            return 0.5 * x * (1.0 + torch.tanh(_GELU_K * (x + 0.044715 * x ** 3)))
        raise ValueError(f"Unsupported activation: {n}")

    def derivative(self, x: torch.Tensor) -> torch.Tensor:
        n = self.name
        if n == "relu":
            return (x > 0).to(x.dtype)  # strict: f'(0) = 0
        if n == "tanh":
            t = torch.tanh(x)
            return 1 - t * t
        if n == "sigmoid":
            s = torch.sigmoid(x)
            return s * (1 - s)
        if n == "silu":
            s = torch.sigmoid(x)
            return s + x * s * (1 - s)
        if n == "gelu":
            u = _GELU_K * (x + 0.044715 * x ** 3)
            t = torch.tanh(u)
            return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * _GELU_K * (1 + 3 * 0.044715 * x * x)
        raise ValueError(f"Unsupported activation: {n}")


def get_activation(name: str) -> ActivationSpec:
    key = str(name).lower()
    if key not in ("relu", "tanh", "sigmoid", "silu", "gelu"):
        raise ValueError(f"Unknown activation {name!r}")
    return ActivationSpec(key)


@dataclass
class ReferenceState:
    x: list[torch.Tensor]
    w: list[torch.Tensor]


def one_hot(labels: torch.Tensor, num_classes: int, *, dtype: torch.dtype) -> torch.Tensor:
    """``[classes, batch]`` one-hot targets."""
    out = torch.zeros((num_classes, labels.numel()), dtype=dtype, device=labels.device)
    out[labels.reshape(-1).long(), torch.arange(labels.numel(), device=labels.device)] = 1
    return out


def init_weights(dims: Sequence[int], *, dtype: torch.dtype, device, seed: int = 0) -> list[torch.Tensor]:
    """``W[l]`` of shape ``[d_l, d_{l+1}]``, kaiming-uniform with ``a = sqrt(5)``,
    drawn in layer order from one generator."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    ws = []
    for rows, cols in zip(dims[:-1], dims[1:]):
        w = torch.empty((int(rows), int(cols)), dtype=dtype, device=device)
        torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5.0), generator=gen)
        ws.append(w)
    return ws


def initialize_state(x_input: torch.Tensor, x_target: torch.Tensor, dims: Sequence[int], *, dtype: torch.dtype,
                     device, seed: int = 0) -> ReferenceState:
    """End states clamped, hidden states zero (the reference's ``initialize_state``;
    its trainer initialises them by a forward prediction instead)."""
    if x_input.ndim != 2 or x_target.ndim != 2:
        raise ValueError("Inputs must be [features,batch]")
    B = int(x_input.shape[1])
    x = [torch.zeros((int(d), B), dtype=dtype, device=device) for d in dims]
    x[0].copy_(x_target)
    x[-1].copy_(x_input)
    return ReferenceState(x=x, w=init_weights(dims, dtype=dtype, device=device, seed=seed))


def prediction_errors(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], act: ActivationSpec):
    """``eps[l] = x[l] - W[l] f(x[l+1])`` for every layer, and the activations
    ``f(x[l])`` (slot 0 holds ``x[0]``); ``eps[L]`` is left unset."""
    L = len(w)
    fx = [x[0]] + [act.forward(x[l]) for l in range(1, L + 1)]
    eps = [x[l] - w[l] @ fx[l + 1] for l in range(L)] + [torch.empty_like(x[L])]
    return eps, fx


def ipc_step(state: ReferenceState, *, act: ActivationSpec, alpha: float, gamma: float, fixed_low: torch.Tensor,
             fixed_high: torch.Tensor, update_weights: bool = True):
    """One iPC step; returns the new state and ``{"energy", "max_abs_error"}``
    over ``eps[0..L-1]``."""
    L = len(state.w)
    eps, _fx = prediction_errors(state.x, state.w, act)
    x = list(state.x)
    new_x = [fixed_low] + [x[l] + gamma * (-eps[l] + act.derivative(x[l]) * (state.w[l - 1].T @ eps[l - 1]))
                           for l in range(1, L)] + [fixed_high]
    new_w = list(state.w)
    if update_weights:
        new_w = [state.w[l] + alpha * (eps[l] @ act.forward(new_x[l + 1]).T) for l in range(L)]
    errs = eps[:L]
    metrics = {"energy": sum((e.float() ** 2).mean() for e in errs).detach(),
               "max_abs_error": torch.stack([e.float().abs().max() for e in errs]).max().detach()}
    return ReferenceState(x=new_x, w=new_w), metrics
