"""GPU parity of the three kernel families against the CPU oracle.

Tolerances (relative = max|gpu - ref| / max|ref|):
* fp32 storage and operands: <= 1e-5 against the fp32 oracle;
* fp32 storage, fp16/bf16 operands: <= 1e-3 against a float64 model that
  rounds the operands exactly where the kernel does (the residue is fp32
  accumulation order plus rare one-ulp operand flips from device tanh/exp),
  and <= 2e-2 against the fp32 oracle;
* 16-bit storage: the reference's own smoke tolerance (rtol = atol = 2e-2,
  ``scripts/smoke.py:28-66``).
Structural properties are exact: every tile configuration, the grouped
(grid.z) form and the scalar (misaligned) load path give bit-identical
results.
"""
import math

import pytest
import torch

from lich_amd.kernels import (KernelConfig, build_forward, build_inference_update, build_prediction_error,
                              build_weight_update, build_weight_update_outer)
from lich_amd.layer_batching import (build_inference_update_batched, build_prediction_error_batched,
                                     build_weight_update_batched)
from oracle import ipc_oracle as O
from tests.helpers import ACTS, DEV, OPS, gen, randn, rel_err, report, rnd, to_dev

pytestmark = pytest.mark.gpu

SHAPES = [(10, 64, 128), (64, 64, 128), (64, 784, 128), (37, 53, 19), (1, 1, 1), (130, 70, 33), (200, 300, 256)]


def _pe_inputs(M, K, B, seed):
    g = gen(seed)
    return randn((K, B), g), randn((M, K), g, 1 / math.sqrt(K)), randn((M, B), g)


@pytest.mark.parametrize("op", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", SHAPES)
def test_prediction_error(M, K, B, act, op):
    report("pred_err", M=M, K=K, B=B, act=act, op=op)
    xu, w, xl = _pe_inputs(M, K, B, 1000 * M + 7 * K + B)
    e = torch.empty((M, B), device=DEV)
    build_prediction_error(M, K, B, act, "float32", operand_dtype=OPS[op])(to_dev(xu), to_dev(w), to_dev(xl), e)
    torch.cuda.synchronize()
    ref = O.pred_err(xu, w, xl, act)
    if op == "f32":
        assert rel_err(e, ref) <= 1e-5
    else:
        model = xl.double() - rnd(w, OPS[op]).double() @ rnd(O.act_forward(act, xu), OPS[op]).double()
        assert rel_err(e, model) <= 1e-3
        assert rel_err(e, ref) <= 2e-2


def _split_model(w, a, op, split):
    """float64 value of the split 16-bit product (same terms as the kernel)."""
    def parts(t):
        hi = t.to(op).double()
        return hi, (t.double() - hi).to(op).double()
    wh, wl = parts(w)
    if split == 2:
        return wh @ a.to(op).double() + wl @ a.to(op).double()
    ah, al = parts(a)
    return wh @ ah + wl @ ah + wh @ al


@pytest.mark.parametrize("split", [2, 3])
@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ["tanh", "sigmoid", "relu"])
@pytest.mark.parametrize("M,K,B", [(10, 64, 128), (64, 784, 128), (37, 53, 19), (200, 300, 256), (1000, 4096, 64)])
def test_prediction_error_split_operands(M, K, B, act, op, split):
    report("pred_err_split", M=M, K=K, B=B, act=act, op=op, split=split)
    xu, w, xl = _pe_inputs(M, K, B, 77 + M + K)
    e = torch.empty((M, B), device=DEV)
    build_prediction_error(M, K, B, act, "float32", operand_dtype=OPS[op], split=split)(
        to_dev(xu), to_dev(w), to_dev(xl), e)
    out = torch.empty((M, B), device=DEV)
    build_forward(M, K, B, act, "float32", operand_dtype=OPS[op], split=split)(to_dev(xu), to_dev(w), out)
    torch.cuda.synchronize()
    a = O.act_forward(act, xu)
    prod = _split_model(w, a, OPS[op], split)
    # split 3 carries f(X) as hi + lo, so a one-ulp difference between device
    # and host tanh/exp cannot flip a 16-bit rounding; split 2 rounds f(X) once.
    model_tol = 1e-4 if split == 3 else 1e-3
    assert rel_err(e, xl.double() - prod) <= model_tol
    assert rel_err(out, prod) <= model_tol
    ref = O.pred_err(xu, w, xl, act)
    # the split must be closer to fp32 than one rounding of each operand
    bound = 2e-4 if split == 3 else 2e-2
    assert rel_err(e, ref) <= bound
    # forward and prediction share the product bit for bit (the wavefront
    # invariant of the forward initialisation relies on it)
    e2 = torch.empty((M, B), device=DEV)
    build_prediction_error(M, K, B, act, "float32", operand_dtype=OPS[op], split=split)(
        to_dev(xu), to_dev(w), out, e2)
    torch.cuda.synchronize()
    assert torch.count_nonzero(e2) == 0


@pytest.mark.parametrize("op", ["f32", "bf16"])
@pytest.mark.parametrize("act", ["tanh", "sigmoid"])
@pytest.mark.parametrize("M,K,B", [(10, 64, 128), (64, 784, 128), (37, 53, 19)])
def test_forward(M, K, B, act, op):
    report("forward", M=M, K=K, B=B, act=act, op=op)
    xu, w, _ = _pe_inputs(M, K, B, 11)
    out = torch.empty((M, B), device=DEV)
    build_forward(M, K, B, act, "float32", operand_dtype=OPS[op])(to_dev(xu), to_dev(w), out)
    torch.cuda.synchronize()
    ref = O.forward_pred(xu, w, act)
    assert rel_err(out, ref) <= (1e-5 if op == "f32" else 2e-2)


@pytest.mark.parametrize("save", [False, True])
@pytest.mark.parametrize("op", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", [(64, 10, 128), (64, 64, 128), (37, 53, 19), (1, 1, 1), (130, 70, 33),
                                   (300, 200, 256)])
def test_inference_update(M, K, B, act, op, save):
    report("infer", M=M, K=K, B=B, act=act, op=op, save=save)
    g = gen(31 * M + K + 3 * B)
    x, e = randn((M, B), g), randn((M, B), g)
    wl, el = randn((K, M), g, 1 / math.sqrt(K)), randn((K, B), g)
    xd = to_dev(x)
    a_out = torch.empty((M, B), device=DEV) if save else None
    k = build_inference_update(M, K, B, act, "float32", None, 0.5, save, operand_dtype=OPS[op])
    if save:
        k(xd, to_dev(e), to_dev(wl), to_dev(el), a_out)
    else:
        k(xd, to_dev(e), to_dev(wl), to_dev(el))
    torch.cuda.synchronize()
    ref_x, ref_a = O.infer_update(x, e, wl, el, act, 0.5)
    if op == "f32":
        assert rel_err(xd, ref_x) <= 1e-5
        if save:
            assert rel_err(a_out, ref_a) <= 1e-5
    else:
        sig = rnd(wl, OPS[op]).double().T @ rnd(el, OPS[op]).double()
        model = x.double() + 0.5 * (-e.double() + O.act_derivative(act, x.double()) * sig)
        assert rel_err(xd, model) <= 1e-3
        assert rel_err(xd, ref_x) <= 2e-2
        if save:
            assert rel_err(a_out, O.act_forward(act, model)) <= 1e-3


@pytest.mark.parametrize("recompute", [True, False])
@pytest.mark.parametrize("op", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", [(10, 64, 128), (64, 784, 128), (37, 53, 19), (1, 1, 1), (130, 70, 33),
                                   (256, 300, 200)])
def test_weight_update(M, K, B, act, op, recompute):
    report("weight", M=M, K=K, B=B, act=act, op=op, recompute=recompute)
    g = gen(17 * M + 5 * K + B)
    w, e, xu = randn((M, K), g, 1 / math.sqrt(K)), randn((M, B), g), randn((K, B), g)
    src = xu if recompute else O.act_forward(act, xu)
    alpha = 0.1
    wd = to_dev(w)
    build_weight_update(M, K, B, act, "float32", None, alpha, recompute, operand_dtype=OPS[op])(wd, to_dev(e), to_dev(src))
    torch.cuda.synchronize()
    ref = O.weight_update(w, e, xu, act, alpha)
    d_gpu = wd.double().cpu() - w.double()
    d_ref = ref.double() - w.double()
    if op == "f32":
        assert rel_err(d_gpu, d_ref) <= 1e-5
    else:
        model = alpha * (rnd(e, OPS[op]).double() @ rnd(O.act_forward(act, xu), OPS[op]).double().T)
        assert rel_err(d_gpu, model) <= 1e-3
        assert rel_err(d_gpu, d_ref) <= 2e-2


def test_weight_update_small_alpha_fp32():
    # alpha=1e-4 on unit-scale W: the update is below W's own rounding scale, so
    # compare the updated W itself (same fp32 rounding on both sides).
    M, K, B = 64, 784, 128
    g = gen(5)
    w, e, xu = randn((M, K), g), randn((M, B), g), randn((K, B), g)
    wd = to_dev(w)
    build_weight_update(M, K, B, "tanh", "float32", None, 1e-4, True, operand_dtype=torch.float32)(wd, to_dev(e), to_dev(xu))
    torch.cuda.synchronize()
    assert rel_err(wd, O.weight_update(w, e, xu, "tanh", 1e-4)) <= 1e-6


@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid", "identity"])
@pytest.mark.parametrize("B", [1, 4, 8, 16, 32])
@pytest.mark.parametrize("M,K", [(64, 784), (10, 64), (64, 64), (33, 300)])
def test_outer_weight_update(M, K, B, act):
    report("outer", M=M, K=K, B=B, act=act)
    g = gen(M + K + B)
    w, e, xu = randn((M, K), g, 1 / math.sqrt(K)), randn((M, B), g), randn((K, B), g)
    alpha = 0.1
    w_outer, w_gemm = to_dev(w), to_dev(w)
    build_weight_update_outer(M, K, B, act, "float32", alpha, True)(w_outer, to_dev(e), to_dev(xu))
    build_weight_update(M, K, B, act, "float32", None, alpha, True, operand_dtype=torch.float32)(w_gemm, to_dev(e), to_dev(xu))
    torch.cuda.synchronize()
    ref = O.weight_update(w, e, xu, act, alpha)
    d_ref = ref.double() - w.double()
    assert rel_err(w_outer.double().cpu() - w.double(), d_ref) <= 1e-5
    # +alpha sign, same sum as the GEMM path
    assert rel_err(w_outer.double().cpu() - w.double(), w_gemm.double().cpu() - w.double()) <= 1e-5
    if B == 1:
        # rank-1: a single product per element, no accumulation order at all
        assert rel_err(w_outer.double().cpu() - w.double(), w_gemm.double().cpu() - w.double()) <= 1e-6


@pytest.mark.parametrize("op", ["f32", "bf16"])
@pytest.mark.parametrize("M,K,B", [(64, 64, 128), (130, 70, 33), (300, 200, 256)])
def test_every_tile_config_is_bit_identical(M, K, B, op):
    report("tiles", M=M, K=K, B=B, op=op)
    xu, w, xl = _pe_inputs(M, K, B, 3)
    outs = []
    for tile in (0, 1, 2):
        e = torch.empty((M, B), device=DEV)
        build_prediction_error(M, K, B, "tanh", "float32", KernelConfig(tile=tile), operand_dtype=OPS[op])(
            to_dev(xu), to_dev(w), to_dev(xl), e)
        wd = to_dev(w)
        build_weight_update(M, K, B, "tanh", "float32", KernelConfig(tile=tile), 0.1, True, operand_dtype=OPS[op])(
            wd, to_dev(xl), to_dev(xu))
        outs.append((e, wd))
    torch.cuda.synchronize()
    for e, wd in outs[1:]:
        assert torch.equal(e, outs[0][0])
        assert torch.equal(wd, outs[0][1])


def test_misaligned_views_take_the_scalar_path_bit_identically():
    M, K, B = 64, 784, 128
    xu, w, xl = _pe_inputs(M, K, B, 9)

    def shifted(t):
        buf = torch.empty(t.numel() + 1, device=DEV)
        v = buf[1:].view(t.shape)
        v.copy_(t.to(DEV))
        return v

    e1 = torch.empty((M, B), device=DEV)
    e2 = shifted(torch.zeros(M, B))
    k = build_prediction_error(M, K, B, "gelu", "float32", operand_dtype=torch.float32)
    k(to_dev(xu), to_dev(w), to_dev(xl), e1)
    k(shifted(xu), shifted(w), shifted(xl), e2)
    torch.cuda.synchronize()
    assert e2.data_ptr() % 16 != 0
    assert torch.equal(e1, e2)


@pytest.mark.parametrize("op", ["f32", "f16"])
def test_grouped_kernels_equal_singletons(op):
    G, D, B = 3, 64, 128
    g = gen(21)
    xs = randn((G + 1, D, B), g)
    ws = randn((G, D, D), g, 1 / math.sqrt(D))
    cfg = KernelConfig(tile=1)
    opd = OPS[op]
    xs_d, ws_d = to_dev(xs), to_dev(ws)
    # prediction: E[g] = X[g] - W[g] f(X[g+1])
    eb = torch.empty((G, D, B), device=DEV)
    build_prediction_error_batched(D, D, B, G, "tanh", "float32", cfg, operand_dtype=opd)(
        xs_d[1:].contiguous(), ws_d, xs_d[:-1].contiguous(), eb)
    es_single = torch.empty((G, D, B), device=DEV)
    k = build_prediction_error(D, D, B, "tanh", "float32", cfg, operand_dtype=opd)
    for i in range(G):
        k(xs_d[i + 1], ws_d[i], xs_d[i], es_single[i])
    torch.cuda.synchronize()
    assert torch.equal(eb, es_single)
    # inference: X[g+1] += ... with E_lower = E[g]
    e_all = to_dev(randn((G + 1, D, B), g))
    x_b = xs_d[1:].clone()
    build_inference_update_batched(D, D, B, G, "tanh", "float32", cfg, 0.5, False, operand_dtype=opd)(
        x_b, e_all[1:].contiguous(), ws_d, e_all[:-1].contiguous())
    x_s = xs_d[1:].clone()
    ki = build_inference_update(D, D, B, "tanh", "float32", cfg, 0.5, False, operand_dtype=opd)
    for i in range(G):
        ki(x_s[i], e_all[i + 1], ws_d[i], e_all[i])
    torch.cuda.synchronize()
    assert torch.equal(x_b, x_s)
    # weight update
    w_b = ws_d.clone()
    build_weight_update_batched(D, D, B, G, "tanh", "float32", cfg, 0.1, True, operand_dtype=opd)(
        w_b, e_all[:-1].contiguous(), xs_d[1:].contiguous())
    w_s = ws_d.clone()
    kw = build_weight_update(D, D, B, "tanh", "float32", cfg, 0.1, True, operand_dtype=opd)
    for i in range(G):
        kw(w_s[i], e_all[i], xs_d[i + 1])
    torch.cuda.synchronize()
    assert torch.equal(w_b, w_s)


def test_reference_smoke_fp16_storage():
    """The reference's kernel smoke (scripts/smoke.py:10-67) on fp16 storage, relu."""
    torch.manual_seed(0)
    M, K, B = 64, 64, 128
    h = torch.float16
    x_up = torch.randn((K, B), dtype=h).to(DEV)
    w = (torch.randn((M, K), dtype=h) * 0.05).to(DEV)
    x_lo = torch.randn((M, B), dtype=h).to(DEV)
    e = torch.empty_like(x_lo)
    build_prediction_error(M, K, B, "relu", "float16", KernelConfig(64, 128, 16, 128, 2, True, 8, False))(x_up, w, x_lo, e)
    torch.cuda.synchronize()
    ref_e = x_lo.float() - w.float() @ torch.relu(x_up.float())
    torch.testing.assert_close(e.float(), ref_e, rtol=2e-2, atol=2e-2)
    x = x_lo.clone()
    e_low = torch.randn((K, B), dtype=h).to(DEV)
    infer_w = (torch.randn((K, M), dtype=h) * 0.05).to(DEV)
    build_inference_update(M, K, B, "relu", "float16", None, 0.5)(x, e, infer_w, e_low)
    torch.cuda.synchronize()
    ref_x = x_lo.float() + 0.5 * (-e.float() + (x_lo.float() > 0).float() * (infer_w.float().T @ e_low.float()))
    torch.testing.assert_close(x.float(), ref_x, rtol=3e-2, atol=3e-2)
    w2 = w.clone()
    build_weight_update(M, K, B, "relu", "float16", None, 1e-4, True)(w2, e, x_up)
    torch.cuda.synchronize()
    ref_w = w.float() + 1e-4 * e.float() @ torch.relu(x_up.float()).T
    torch.testing.assert_close(w2.float(), ref_w, rtol=2e-2, atol=2e-2)
    # tail M=10
    m2 = 10
    xu2 = torch.randn((K, B), dtype=h).to(DEV)
    ws = (torch.randn((m2, K), dtype=h) * 0.05).to(DEV)
    xs = torch.randn((m2, B), dtype=h).to(DEV)
    es = torch.empty_like(xs)
    build_prediction_error(m2, K, B, "relu", "float16")(xu2, ws, xs, es)
    torch.cuda.synchronize()
    torch.testing.assert_close(es.float(), xs.float() - ws.float() @ torch.relu(xu2.float()), rtol=3e-2, atol=3e-2)
    # saved-activation weight update equals recompute
    w_saved = w.clone()
    build_weight_update(M, K, B, "relu", "float16", None, 1e-4, False)(w_saved, e, torch.relu(x_up).contiguous())
    torch.cuda.synchronize()
    assert torch.equal(w_saved, w2)


@pytest.mark.parametrize("storage", ["float16", "bfloat16"])
def test_16bit_storage_pred_err_rounds_like_reference(storage):
    dt = getattr(torch, storage)
    M, K, B = 64, 784, 128
    xu, w, xl = _pe_inputs(M, K, B, 4)
    xu16, w16, xl16 = xu.to(dt), w.to(dt), xl.to(dt)
    e = torch.empty((M, B), device=DEV, dtype=dt)
    build_prediction_error(M, K, B, "tanh", storage)(xu16.to(DEV), w16.to(DEV), xl16.to(DEV), e)
    torch.cuda.synchronize()
    acc = w16.double() @ torch.tanh(xu16.float()).to(dt).double()
    model = (xl16.float() - acc.float().to(dt).float()).to(dt)
    assert rel_err(e.float(), model.float()) <= 2e-2
