"""CPU emulation of the 16-bit operand design (test infrastructure only).

The HIP path keeps ``x``, ``eps`` and ``W`` in fp32 and rounds only the GEMM
*operands* to fp16/bf16 (``W``, ``f(x)``, ``eps``), accumulating in fp32.
This module applies the same rounding points to the oracle's step so that a
CPU test can confirm, over several seeds, that the design meets the 16-bit
tolerances (states <= 2e-2, weight deltas <= 5e-3, globally normalised)
before any GPU run, and so that GPU tests can compare against a model of the
expected rounding as well as against the fp32 oracle.

It also emulates the reference's all-16-bit *storage* design
(``tilelang_kernels.py:173,320``: ``E = half(x) - half(acc)``,
``W = half(float(W) + alpha*acc)``) to document why that design is not used.
"""
from __future__ import annotations

from typing import Sequence

import torch

from .ipc_oracle import act_derivative, act_forward


def _r(t: torch.Tensor, op: torch.dtype) -> torch.Tensor:
    return t.to(op).to(torch.float32)


def _split(t: torch.Tensor, op: torch.dtype):
    hi = _r(t, op)
    return hi, _r(t - hi, op)


def weight_pair(w: torch.Tensor, op: torch.dtype) -> torch.Tensor:
    """W as a wide plan with weight pairs stores it: float(hi) + float(lo) with
    hi = cvt(W), lo = cvt(W - hi) (about 17 significant bits; the fp32 sum
    rounds once more where lo lies far below hi).  The value is its own pair."""
    hi, lo = _split(w, op)
    return hi + lo


def pred_matmul(w: torch.Tensor, a: torch.Tensor, op: torch.dtype, split: int = 1) -> torch.Tensor:
    """``w @ a`` with 16-bit operands: split 1 rounds both operands once;
    split 2 carries ``w`` as hi + lo terms; split 3 carries both operands as
    hi + lo and keeps hi*hi + lo*hi + hi*lo (the lo*lo term is dropped)."""
    if split == 1:
        return _r(w, op) @ _r(a, op)
    wh, wl = _split(w, op)
    if split == 2:
        ah = _r(a, op)
        return wh @ ah + wl @ ah
    ah, al = _split(a, op)
    return wh @ ah + wl @ ah + wh @ al


def forward_init_operand16(x_input, y_target, w, *, act: str, op: torch.dtype, split: int = 1):
    """Forward initialisation with the same prediction arithmetic as the step."""
    L = len(w)
    x = [None] * (L + 1)
    x[L] = x_input.clone()
    for l in reversed(range(L)):
        p = pred_matmul(w[l], act_forward(act, x[l + 1]), op, split)
        x[l] = p if l > 0 else None
    x[0] = y_target.clone()
    return x


def step_operand16(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], *, act: str, alpha: float,
                   gamma: float, op: torch.dtype, split: int = 1, w_pairs: bool = False):
    """fp32 master x/eps/W; GEMM operands rounded to ``op`` (the prediction
    optionally split, see ``pred_matmul``); fp32 accumulate.  ``w_pairs``: W is
    stored as its hi + lo pair (``weight_pair``) before and after the update."""
    L = len(w)
    if w_pairs:
        w = [weight_pair(v, op) for v in w]
    e = [x[l] - pred_matmul(w[l], act_forward(act, x[l + 1]), op, split) for l in range(L)]
    new_x = [v.clone() for v in x]
    for l in range(1, L):
        sig = _r(w[l - 1], op).T @ _r(e[l - 1], op)
        new_x[l] = x[l] + gamma * (-e[l] + act_derivative(act, x[l]) * sig)
    new_w = [w[l] + alpha * (_r(e[l], op) @ _r(act_forward(act, new_x[l + 1]), op).T) for l in range(L)]
    if w_pairs:
        new_w = [weight_pair(v, op) for v in new_w]
    return new_x, new_w, e


def step_storage16(x: Sequence[torch.Tensor], w: Sequence[torch.Tensor], *, act: str, alpha: float,
                   gamma: float, op: torch.dtype):
    """Everything stored in ``op`` (the reference's fp16 design)."""
    L = len(w)
    xs = [_r(v, op) for v in x]
    ws = [_r(v, op) for v in w]
    e = [_r(_r(xs[l], op) - _r(ws[l] @ _r(act_forward(act, xs[l + 1]), op), op), op) for l in range(L)]
    new_x = [v.clone() for v in xs]
    for l in range(1, L):
        sig = ws[l - 1].T @ e[l - 1]
        new_x[l] = _r(xs[l] + gamma * (-e[l] + act_derivative(act, xs[l]) * sig), op)
    new_w = [_r(ws[l] + alpha * (e[l] @ _r(act_forward(act, new_x[l + 1]), op).T), op) for l in range(L)]
    return new_x, new_w, e


def run(step_fn, x, w, steps: int, **kw):
    x = list(x)
    w = list(w)
    for _ in range(int(steps)):
        x, w, _e = step_fn(x, w, **kw)
    return x, w
