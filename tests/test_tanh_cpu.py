"""The kernels' fp32 tanh (`tanh_f32` in lich_amd/csrc/ipc_device.h) on the CPU.

* Its polynomial coefficients are re-derived here: a weighted least-squares
  fit (iteratively reweighted towards the largest errors) of tanh(a)/a - 1 by
  a degree-4 polynomial in a^2 on [0, 0.55], read back from the header and
  compared within fp32 rounding.
* The evaluation is modelled in float32 (each product and sum rounded, fma
  rounded once, exp2 and the reciprocal correctly rounded) and checked against
  float64 tanh on 2 M points spread over [1e-30, 100]: at most 2 ulp; the
  GPU test (tests/test_gpu_resident.py::test_tanh_within_two_ulp) checks the
  device itself.
"""
import re
from pathlib import Path

import numpy as np

HEADER = Path(__file__).resolve().parents[1] / "lich_amd" / "csrc" / "ipc_device.h"


def _header_constants():
    """The fp32 literals of tanh_f32, in source order."""
    src = HEADER.read_text()
    body = src[src.index("float tanh_f32(float x)"):]
    body = body[:body.index("\n}\n")]
    return [float(v[:-1]) for v in re.findall(r"[-+]?\d+\.\d+f", body)]


def _fit(T=0.55, terms=5):
    n = 4000
    xs = T * (0.5 - 0.5 * np.cos(np.pi * (np.arange(n) + 0.5) / n))
    y = np.tanh(xs) / xs - 1.0
    A = np.stack([xs ** (2 * k) for k in range(1, terms + 1)], axis=1)
    w = np.ones_like(xs)
    for _ in range(30):
        c, *_ = np.linalg.lstsq(A * w[:, None], y * w, rcond=None)
        err = A @ c - y
        w = w * (1 + 4 * np.abs(err) / np.abs(err).max())
    return c, float(np.abs(A @ c - y).max())


def _model(x, c):
    f32 = np.float32
    c = [f32(v) for v in c]

    def fma(a, b, d):
        return (a.astype(np.float64) * b.astype(np.float64) + np.float64(d)).astype(f32)

    with np.errstate(over="ignore", invalid="ignore"):
        a = np.abs(x)
        s = (a * a).astype(f32)
        p = fma(np.full_like(a, c[4]), s, c[3])
        p = fma(p, s, c[2])
        p = fma(p, s, c[1])
        p = fma(p, s, c[0])
        small = fma(a, (s * p).astype(f32), a)
        e = np.exp2((a * f32(2.88539004)).astype(f32).astype(np.float64)).astype(f32)
        r = (1.0 / (e + f32(1)).astype(f32).astype(np.float64)).astype(f32)
        large = fma(np.full_like(r, f32(-2)), r, f32(1))
    return np.copysign(np.where(a < f32(0.55), small, large), x)


def test_coefficients_are_the_fit():
    c, err = _fit()
    assert err < 2e-9
    nums = _header_constants()
    # Horner order in the source: the a^10 coefficient first, the a^2 one last,
    # then 2 log2(e), 1 and the 0.55 threshold
    horner = nums[:5][::-1]
    for fitted, used in zip(c, horner):
        assert abs(fitted - used) <= 1e-7 * abs(fitted), (fitted, used)
    assert abs(nums[5] - 2.0 * np.log2(np.e)) <= 1e-7 * nums[5]
    assert 0.55 in nums


def test_model_within_two_ulp():
    c = [-0.333333194, 0.133326024, -0.0538538583, 0.0210777614, -0.00628247811]
    worst = 0.0
    for lo, hi in ((1e-30, 1e-6), (1e-6, 0.55), (0.5, 2.0), (2.0, 10.0), (10.0, 100.0)):
        b0 = np.float32(lo).view(np.uint32)
        b1 = np.float32(hi).view(np.uint32)
        x = np.linspace(int(b0), int(b1), 400_000).astype(np.uint32).view(np.float32)
        t = _model(x, c)
        ref = np.tanh(x.astype(np.float64))
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        worst = max(worst, float((np.abs(t - ref) / ulp).max()))
    assert worst <= 2.0, worst
    special = _model(np.array([0.0, -0.0, np.inf, -np.inf, np.nan], np.float32), c)
    assert special[0] == 0 and np.signbit(special[1]) and special[2] == 1 and special[3] == -1
    assert np.isnan(special[4])
