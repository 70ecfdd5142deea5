"""CPU evidence for the precision design (no GPU).

The step is emulated with the rounding points of the HIP kernels
(``oracle/emulate.py``) and compared with the fp32 oracle over several seeds,
with the bars the GPU must meet: states <= 2e-2 and weight deltas <= 5e-3
(relative, globally normalised) after T=4 steps.  It also records why the
reference's all-16-bit storage (``tilelang_kernels.py:173,320``) is not used:
it misses the weight-delta bar.
"""
import pytest
import torch

from oracle import emulate as E
from oracle import ipc_oracle as O


def _run(dims, B, seed, op, split, act="tanh", T=4, w_pairs=False, input_dist="uniform"):
    w0 = O.init_weights(dims, seed=seed, init="xavier_uniform")
    x_in, _, y = O.make_batch(dims, B, seed=seed, input_dist=input_dist)
    x = O.forward_init(x_in, y, w0, act)
    xr, wr, _ = O.run_steps(x, w0, T, act=act, alpha=1e-4, gamma=0.5)
    xm = E.forward_init_operand16(x_in, y, w0, act=act, op=op, split=split)
    wm = list(w0)
    for _ in range(T):
        xm, wm, _ = E.step_operand16(xm, wm, act=act, alpha=1e-4, gamma=0.5, op=op, split=split, w_pairs=w_pairs)
    L = len(w0)
    s = O.global_rel_err(xm[1:L], xr[1:L])
    d = O.global_rel_err([wm[l] - w0[l] for l in range(L)], [wr[l] - w0[l] for l in range(L)])
    return s, d


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("op", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("depth", [3, 6])
def test_paper_profile_design_meets_bars(depth, op, seed):
    # the trainer's defaults for narrow tanh nets: split 1 with fp16 operands, 3 with bf16
    split = 1 if op == torch.float16 else 3
    s, d = _run((10,) + (64,) * depth + (784,), 128, seed, op, split=split)
    assert s <= 2e-2 and d <= 5e-3, (s, d)
    if split == 1:
        # with a wide margin: fp16's rounding alone stays ~10x inside the bars
        assert s <= 2e-3 and d <= 1.5e-3, (s, d)


@pytest.mark.parametrize("seed", range(3))
def test_relu_keeps_the_split_with_fp16_operands(seed):
    # relu's f' is a step: unsplit fp16 operands flip it for states near 0 and the flips
    # spread (max-norm state error 3e-2 to 4e-2, weight deltas up to 3.1e-3 at d = 4,
    # as measured on the GPU), so the trainer keeps split 3 for relu, ~40x tighter
    dims = (10,) + (64,) * 4 + (784,)
    s1, d1 = _run(dims, 128, seed, torch.float16, split=1, act="relu")
    s3, d3 = _run(dims, 128, seed, torch.float16, split=3, act="relu")
    assert s3 <= 2e-3 and d3 <= 5e-4, (s3, d3)
    assert s1 > 10 * s3 and d1 > 5 * d3, (s1, s3, d1, d3)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_zero_crossing_derivatives_keep_the_split_with_fp16_operands(act):
    # silu's and gelu's f' cross zero: unsplit fp16 operands take the weight-delta error
    # to 2.1-2.4e-3 at d = 3 (about half the bar) against ~1.3e-4 with split 3; tanh and
    # sigmoid stay at or below 8.4e-4 unsplit, so only they default to split 1
    dims = (10,) + (64,) * 3 + (784,)
    r1 = [_run(dims, 128, seed, torch.float16, split=1, act=act) for seed in range(5)]
    r3 = [_run(dims, 128, seed, torch.float16, split=3, act=act) for seed in range(5)]
    d1, d3 = max(d for _s, d in r1), max(d for _s, d in r3)
    assert d1 > 1.5e-3 and d3 <= 2e-4, (d1, d3)
    for smooth in ("tanh", "sigmoid"):
        assert max(_run(dims, 128, seed, torch.float16, split=1, act=smooth)[1] for seed in range(5)) <= 1e-3


def test_split_reduces_the_prediction_error():
    dims = (10,) + (64,) * 4 + (784,)
    errs = {k: _run(dims, 128, 0, torch.bfloat16, split=k)[1] for k in (1, 2, 3)}
    assert errs[3] < errs[2] < errs[1]


def test_reference_all_16bit_storage_misses_the_weight_delta_bar():
    dims = (10,) + (64,) * 3 + (784,)
    w0 = O.init_weights(dims, seed=0, init="xavier_uniform")
    x_in, _, y = O.make_batch(dims, 128, seed=0)
    x = O.forward_init(x_in, y, w0, "tanh")
    xr, wr, _ = O.run_steps(x, w0, 4, act="tanh", alpha=1e-4, gamma=0.5)
    xs, ws = E.run(E.step_storage16, x, w0, 4, act="tanh", alpha=1e-4, gamma=0.5, op=torch.float16)
    L = len(w0)
    d = O.global_rel_err([ws[l] - w0[l].half().float() for l in range(L)], [wr[l] - w0[l] for l in range(L)])
    assert d > 5e-3


def test_weight_pairs_miss_the_bar_on_small_weight_deltas():
    """Why the wide path keeps an fp32 W master rather than only its bf16 hi + lo
    operand pair (~17 significant bits, which would save the 4-byte fp32 store
    per weight and step): the pair's rounding is ~2^-17 of |W| per update,
    harmless on the wide configuration (max |dW| ~5e-3: 3.3e-3 either way) but
    not where the weight deltas are small against W.  (33, 520, 129, 300, 64),
    silu, B = 100, N(0, 1) inputs: max |dW| is 1.6e-4 and the pair design misses
    the 5e-3 bar (1.27e-2, the value the GPU gave for a build with pairs) while
    the fp32 master stays at 3.1e-3.  The pairs also did not shorten the wide
    weight update on MI355X (323-329 us against 324-326 us)."""
    dims = (33, 520, 129, 300, 64)
    kw = dict(act="silu", input_dist="normal")
    s_f, d_f = _run(dims, 100, 3, torch.bfloat16, split=2, **kw)
    s_p, d_p = _run(dims, 100, 3, torch.bfloat16, split=2, w_pairs=True, **kw)
    assert d_f <= 5e-3 < d_p, (d_f, d_p)
