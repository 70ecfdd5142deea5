"""The LDS-DMA kernel (tile IPC_TILE_DMA_256x128) of the standalone 16-bit
storage calls against the generic MFMA kernel and the CPU oracle.

Both kernels round the same 16-bit operands (f applied in fp32, then one
rounding) and feed them to the same v_mfma_f32_32x32x16 instruction in the
same k order with the same epilogue arithmetic, so their results must agree
bit for bit; the LDS-DMA kernel reads some operands through the LDS transpose
read and f(X) through its register path, which this pins.  For the
activations built on exp/tanh the compiler may schedule (and contract into
FMAs) the activation's arithmetic differently in the two kernels: a one-ulp
change of f(x) can flip a 16-bit operand rounding, so those cases are held to
2e-3 of the output's max-norm with at most 1% of the elements differing,
while relu and identity must agree bit for bit.  Against the fp32
oracle the reference smoke tolerance applies (rtol = atol = 2e-2,
``scripts/smoke.py:28-66``, expressed here as a max-norm bound).
"""
import math

import pytest
import torch

from lich_amd.kernels import (KernelConfig, build_forward, build_inference_update, build_prediction_error,
                              build_weight_update)
from lich_amd.layer_batching import (build_inference_update_batched, build_prediction_error_batched,
                                     build_weight_update_batched)
from oracle import ipc_oracle as O
from tests.helpers import ACTS, DEV, OPS, gen, randn, rel_err, report

pytestmark = pytest.mark.gpu

DMA = KernelConfig(tile=3)
GEN = KernelConfig(tile=2)
# (M, K, B): K is the contraction of pred / infer (a multiple of 64); ragged
# M, and B a multiple of 8 but not of the 128-column tile
PI_SHAPES = [(256, 64, 128), (300, 192, 136), (64, 128, 8), (1000, 256, 264)]
# weight update (M, K, B): B is the contraction
W_SHAPES = [(256, 128, 128), (300, 136, 64), (10, 784, 192), (1000, 64, 256)]


def _t(t, op):
    return t.to(device=DEV, dtype=op).contiguous()


def _same(a, b, act):
    diff = float((a != b).float().mean())
    err = rel_err(a.float(), b.float())
    print(f"dma vs generic ({act}): {diff:.2e} of elements differ, rel err {err:.2e}")
    if act in ("relu", "identity"):
        return diff == 0.0
    return err <= 2e-3 and diff <= 1e-2


@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", PI_SHAPES)
def test_dma_prediction_and_forward(M, K, B, act, op):
    report("dma16-pred", M=M, K=K, B=B, act=act, op=op)
    dt = OPS[op]
    g = gen(5 * M + K + B)
    xu, w, xl = randn((K, B), g), randn((M, K), g, 1 / math.sqrt(K)), randn((M, B), g)
    outs = {}
    for name, cfg in (("dma", DMA), ("gen", GEN)):
        e = torch.empty((M, B), device=DEV, dtype=dt)
        f = torch.empty((M, B), device=DEV, dtype=dt)
        build_prediction_error(M, K, B, act, dt, cfg)(_t(xu, dt), _t(w, dt), _t(xl, dt), e)
        build_forward(M, K, B, act, dt, cfg)(_t(xu, dt), _t(w, dt), f)
        outs[name] = (e, f)
    torch.cuda.synchronize()
    assert _same(outs["dma"][0], outs["gen"][0], act)
    assert _same(outs["dma"][1], outs["gen"][1], act)
    ref = O.pred_err(xu.to(dt).float(), w.to(dt).float(), xl.to(dt).float(), act)
    assert rel_err(outs["dma"][0].float(), ref) <= 2e-2


@pytest.mark.parametrize("save", [False, True])
@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", PI_SHAPES)
def test_dma_inference_update(M, K, B, act, op, save):
    report("dma16-infer", M=M, K=K, B=B, act=act, op=op, save=save)
    dt = OPS[op]
    if M % 8:
        M = M + (8 - M % 8)  # W_lower [K, M] is read transposed: its rows must hold a multiple of 8
    g = gen(7 * M + 3 * K + B)
    x, e, wl, el = randn((M, B), g), randn((M, B), g), randn((K, M), g, 1 / math.sqrt(K)), randn((K, B), g)
    res = {}
    for name, cfg in (("dma", DMA), ("gen", GEN)):
        xd = _t(x, dt)
        a = torch.empty((M, B), device=DEV, dtype=dt) if save else None
        build_inference_update(M, K, B, act, dt, cfg, 0.5, save)(xd, _t(e, dt), _t(wl, dt), _t(el, dt), a)
        res[name] = (xd, a)
    torch.cuda.synchronize()
    assert _same(res["dma"][0], res["gen"][0], act)
    if save:
        assert _same(res["dma"][1], res["gen"][1], act)
    xr, ar = O.infer_update(x.to(dt).float(), e.to(dt).float(), wl.to(dt).float(), el.to(dt).float(), act, 0.5)
    assert rel_err(res["dma"][0].float(), xr) <= 2e-2
    if save:
        assert rel_err(res["dma"][1].float(), ar) <= 2e-2


@pytest.mark.parametrize("recompute", [True, False])
@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B", W_SHAPES)
def test_dma_weight_update(M, K, B, act, op, recompute):
    report("dma16-weight", M=M, K=K, B=B, act=act, op=op, recompute=recompute)
    dt = OPS[op]
    g = gen(11 * M + K + 5 * B)
    w, e, xu = randn((M, K), g, 1 / math.sqrt(K)), randn((M, B), g), randn((K, B), g)
    src = xu if recompute else O.act_forward(act, xu)
    res = {}
    for name, cfg in (("dma", DMA), ("gen", GEN)):
        wd = _t(w, dt)
        build_weight_update(M, K, B, act, dt, cfg, 0.01, recompute)(wd, _t(e, dt), _t(src, dt))
        res[name] = wd
    torch.cuda.synchronize()
    assert _same(res["dma"], res["gen"], act)
    a = O.act_forward(act, xu.to(dt).float()) if recompute else src.to(dt).float()
    ref = w.to(dt).float() + 0.01 * (e.to(dt).float() @ a.T)
    assert rel_err(res["dma"].float().cpu() - w.to(dt).float(), ref - w.to(dt).float()) <= 2e-2


@pytest.mark.parametrize("op", ["bf16"])
def test_dma_grouped_equals_singleton(op):
    """Grouped (grid.z) calls run one problem per group on the LDS-DMA kernel."""
    report("dma16-grouped", op=op)
    dt = OPS[op]
    G, M, K, B = 3, 128, 128, 128
    g = gen(3)
    xu, w, xl = randn((G, K, B), g), randn((G, M, K), g, 1 / math.sqrt(K)), randn((G, M, B), g)
    eg = torch.empty((G, M, B), device=DEV, dtype=dt)
    build_prediction_error_batched(M, K, B, G, "tanh", dt, DMA)(_t(xu, dt), _t(w, dt), _t(xl, dt), eg)
    wg = _t(w, dt)
    build_weight_update_batched(M, K, B, G, "tanh", dt, DMA, 0.01, True)(wg, _t(xl, dt), _t(xu, dt))
    for i in range(G):
        e1 = torch.empty((M, B), device=DEV, dtype=dt)
        build_prediction_error(M, K, B, "tanh", dt, DMA)(_t(xu[i], dt), _t(w[i], dt), _t(xl[i], dt), e1)
        w1 = _t(w[i], dt)
        build_weight_update(M, K, B, "tanh", dt, DMA, 0.01, True)(w1, _t(xl[i], dt), _t(xu[i], dt))
        torch.cuda.synchronize()
        assert torch.equal(eg[i], e1)
        assert torch.equal(wg[i], w1)


def test_dma_tile_refused_when_ineligible():
    report("dma16-refuse")
    dt = torch.bfloat16
    # contraction 100 is not a multiple of 64
    k = build_prediction_error(64, 100, 128, "tanh", dt, DMA)
    with pytest.raises(ValueError, match="LDS-DMA"):
        k(torch.zeros((100, 128), device=DEV, dtype=dt), torch.zeros((64, 100), device=DEV, dtype=dt),
          torch.zeros((64, 128), device=DEV, dtype=dt), torch.zeros((64, 128), device=DEV, dtype=dt))
    # fp32 storage
    k = build_prediction_error(64, 64, 128, "tanh", torch.float32, DMA)
    with pytest.raises(ValueError, match="LDS-DMA"):
        k(torch.zeros((64, 128), device=DEV), torch.zeros((64, 64), device=DEV),
          torch.zeros((64, 128), device=DEV), torch.zeros((64, 128), device=DEV))


def _preact(mode):
    from lich_amd import _native as nat
    assert nat.lib().ipc_set_s16_preactivate(mode) == 0


@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M,K,B,G", [(1024, 128, 256, 1), (1088, 1088, 192, 2), (300, 192, 128, 1)])
def test_preactivated_operand_gives_the_register_path_bits(M, K, B, G, act, op):
    """f(X_upper) evaluated once into a caller workspace (mode 1: whenever one
    is given) against the loader's register path (no workspace): prediction,
    forward and the recomputing weight update agree bit for bit, grouped
    (square layers) or not, above and below the automatic threshold."""
    report("dma16-preact", M=M, K=K, B=B, G=G, act=act, op=op)
    dt = OPS[op]
    g = gen(13 * M + K + B + G)
    xu, w, xl = randn((G, K, B), g), randn((G, M, K), g, 1 / math.sqrt(K)), randn((G, M, B), g)
    wk, e = randn((G, M, K), g, 1 / math.sqrt(K)), randn((G, M, B), g)
    res = {}
    try:
        _preact(1)
        for use_ws in (False, True):
            ep = torch.empty((G, M, B), device=DEV, dtype=dt)
            fp = torch.empty((G, M, B), device=DEV, dtype=dt)
            wd = _t(wk, dt)
            if G == 1:
                kp = build_prediction_error(M, K, B, act, dt, DMA)
                kf = build_forward(M, K, B, act, dt, DMA)
                kw = build_weight_update(M, K, B, act, dt, DMA, 0.01, True)
                kp(_t(xu[0], dt), _t(w[0], dt), _t(xl[0], dt), ep[0], workspace=kp.new_workspace() if use_ws else None)
                kf(_t(xu[0], dt), _t(w[0], dt), fp[0], workspace=kf.new_workspace() if use_ws else None)
                kw(wd[0], _t(e[0], dt), _t(xu[0], dt), workspace=kw.new_workspace() if use_ws else None)
            else:
                kp = build_prediction_error_batched(M, K, B, G, act, dt, DMA)
                kw = build_weight_update_batched(M, K, B, G, act, dt, DMA, 0.01, True)
                kp(_t(xu, dt), _t(w, dt), _t(xl, dt), ep, workspace=kp.new_workspace() if use_ws else None)
                kw(wd, _t(e, dt), _t(xu, dt), workspace=kw.new_workspace() if use_ws else None)
            if use_ws and act != "identity":
                assert kp.workspace_bytes == G * K * B * 2 and kw.workspace_bytes == G * K * B * 2
            res[use_ws] = (ep, wd) + ((fp,) if G == 1 else ())  # forward has no grouped form
        torch.cuda.synchronize()
    finally:
        _preact(-1)
    for a, b in zip(res[False], res[True]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ["relu", "tanh"])
@pytest.mark.parametrize("M,K,B,G", [(296, 192, 136, 1), (512, 256, 520, 1), (256, 256, 72, 3)])
def test_transposed_preactivation_matches_the_loader_on_every_tile(M, K, B, G, act, op):
    """With a workspace, the prediction and forward evaluate f(X_upper) once
    and store it transposed ([B][K]), so that the GEMM reads both operands
    k-contiguous: on every LDS-DMA tile configuration (256 x 256 finishes from
    the registers), for ragged batch widths (the transposing pass's edges)
    and grouped calls, the results equal the loader path's bit for bit."""
    from lich_amd import _native as nat

    report("dma16-preact-t", M=M, K=K, B=B, G=G, act=act, op=op)
    dt = OPS[op]
    g = gen(5 * M + 3 * K + B + G)
    xu, w, xl = _t(randn((G, K, B), g), dt), _t(randn((G, M, K), g, 1 / math.sqrt(K)), dt), _t(randn((G, M, B), g), dt)
    try:
        _preact(1)
        for tile in nat.TILE_DMA_TILES:
            cfg = KernelConfig(tile=tile)
            out = {}
            for use_ws in (False, True):
                ep = torch.empty((G, M, B), device=DEV, dtype=dt)
                fp = torch.empty((M, B), device=DEV, dtype=dt)
                if G == 1:
                    kp = build_prediction_error(M, K, B, act, dt, cfg)
                    kp(xu[0], w[0], xl[0], ep[0], workspace=kp.new_workspace() if use_ws else None)
                    kf = build_forward(M, K, B, act, dt, cfg)
                    kf(xu[0], w[0], fp, workspace=kf.new_workspace() if use_ws else None)
                else:
                    kp = build_prediction_error_batched(M, K, B, G, act, dt, cfg)
                    kp(xu, w, xl, ep, workspace=kp.new_workspace() if use_ws else None)
                out[use_ws] = (ep, fp)
            torch.cuda.synchronize()
            assert torch.equal(out[False][0], out[True][0]), tile
            if G == 1:
                assert torch.equal(out[False][1], out[True][1]), tile
    finally:
        _preact(-1)


@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ["relu", "tanh", "identity"])
@pytest.mark.parametrize("M,K,B,G,save", [(296, 192, 136, 1, True), (512, 256, 520, 1, False),
                                          (256, 256, 72, 3, True)])
def test_inference_update_with_transposed_operands_matches_on_every_tile(M, K, B, G, save, act, op):
    """With a workspace, the inference update copies W_lower and E_lower
    transposed ([M][K], [B][K]) and its GEMM reads both operands k-contiguous:
    on every LDS-DMA tile configuration, for ragged shapes and grouped calls,
    X and A_out equal the transposing-read path's bit for bit, and the
    workspace holds (M*K + K*B)*2 bytes per group."""
    from lich_amd import _native as nat

    report("dma16-infer-ws", M=M, K=K, B=B, G=G, save=save, act=act, op=op)
    dt = OPS[op]
    g = gen(11 * M + 5 * K + B + G)
    x0, e = _t(randn((G, M, B), g), dt), _t(randn((G, M, B), g), dt)
    wl, el = _t(randn((G, K, M), g, 1 / math.sqrt(K)), dt), _t(randn((G, K, B), g), dt)
    try:
        _preact(1)
        for tile in nat.TILE_DMA_TILES:
            cfg = KernelConfig(tile=tile)
            out = {}
            for use_ws in (False, True):
                x = x0.clone()
                a = torch.empty((G, M, B), device=DEV, dtype=dt) if save else None
                if G == 1:
                    k = build_inference_update(M, K, B, act, dt, cfg, 0.5, save)
                    k(x[0], e[0], wl[0], el[0], a[0] if save else None,
                      workspace=k.new_workspace() if use_ws else None)
                else:
                    k = build_inference_update_batched(M, K, B, G, act, dt, cfg, 0.5, save)
                    k(x, e, wl, el, a, workspace=k.new_workspace() if use_ws else None)
                if use_ws:
                    assert k.workspace_bytes == G * (M * K + K * B) * 2
                out[use_ws] = (x, a)
            torch.cuda.synchronize()
            assert torch.equal(out[False][0], out[True][0]), tile
            if save:
                assert torch.equal(out[False][1], out[True][1]), tile
    finally:
        _preact(-1)


def test_preactivation_into_a_caller_workspace_under_graph_capture():
    """A captured standalone call with a caller workspace records its
    activation launch and its GEMM (nothing is allocated, so nothing keeps it
    out of the graph); its replays match the direct call bit for bit."""
    report("dma16-preact-graph")
    dt = torch.bfloat16
    M, K, B = 1024, 1024, 1024
    g = gen(17)
    xu, w, xl = _t(randn((K, B), g), dt), _t(randn((M, K), g, 1 / math.sqrt(K)), dt), _t(randn((M, B), g), dt)
    fn = build_prediction_error(M, K, B, "tanh", dt, DMA)
    assert fn.workspace_bytes == K * B * 2  # the automatic rule pre-activates this call
    ws = fn.new_workspace()
    direct = torch.empty((M, B), device=DEV, dtype=dt)
    loader = torch.empty((M, B), device=DEV, dtype=dt)
    captured = torch.empty((M, B), device=DEV, dtype=dt)
    fn(xu, w, xl, direct, workspace=ws)
    fn(xu, w, xl, loader)
    torch.cuda.synchronize()
    assert torch.equal(direct, loader)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(xu, w, xl, captured, workspace=ws)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        fn(xu, w, xl, captured, workspace=ws)
    for _ in range(3):
        captured.zero_()
        ws.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, direct)


def test_default_standalone_calls_allocate_no_device_memory():
    """The standalone calls without a workspace take the loader path at every
    C5 shape and size: the device's free memory is the same before and after
    them (a call that allocated, even from a pool it keeps, would lower it by
    at least its K * B * 2-byte operand)."""
    report("dma16-noalloc")
    dt = torch.bfloat16
    g = gen(23)
    shapes = [(256, 256), (1024, 8192), (4096, 2048), (8192, 2048)]
    tensors = {}
    for n, B in shapes:
        tensors[(n, B)] = (_t(randn((n, B), g), dt), _t(randn((n, n), g, 1 / math.sqrt(n)), dt),
                           _t(randn((n, B), g), dt), torch.empty((n, B), device=DEV, dtype=dt),
                           _t(randn((n, n), g, 1 / math.sqrt(n)), dt))

    def calls(n, B):
        xu, w, xl, e, wk = tensors[(n, B)]
        for act in ("tanh", "relu"):
            kp = build_prediction_error(n, n, B, act, dt, DMA)
            assert n < 1024 or kp.workspace_bytes > 0 or act == "relu"  # would pre-activate given a workspace
            kp(xu, w, xl, e)
            build_forward(n, n, B, act, dt, DMA)(xu, w, e)
            build_weight_update(n, n, B, act, dt, DMA, 1e-4, True)(wk, xl, xu)

    # the same kernels once at a small size first: the runtime's first launch
    # of a kernel may set up its code object and private-segment memory
    calls(256, 256)
    torch.cuda.synchronize()
    free0, _total = torch.cuda.mem_get_info(DEV)
    for n, B in shapes[1:]:
        calls(n, B)
    torch.cuda.synchronize()
    free1, _total = torch.cuda.mem_get_info(DEV)
    print(f"free device memory before {free0} after {free1}", flush=True)
    assert free1 == free0


@pytest.mark.parametrize("op", ["f16", "bf16"])
@pytest.mark.parametrize("act", ["relu", "tanh", "identity"])
@pytest.mark.parametrize("M,K,B", [(296, 192, 136), (1000, 256, 264), (64, 128, 8)])
def test_dma_tile_configurations_agree(M, K, B, act, op):
    """The LDS-DMA tile configurations (the autotuner's search space
    for the standalone calls) add the contraction in the same k order with
    the same epilogue: prediction, forward, inference (with A_out) and both
    weight updates agree with the default configuration bit for bit for relu
    and identity, and within the activation-contraction allowance otherwise.
    (M is a multiple of 8: the inference reads W_lower [K, M] transposed.)"""
    report("dma16-tiles", M=M, K=K, B=B, act=act, op=op)
    dt = OPS[op]
    g = gen(7 * M + 3 * K + B)
    xu, w, xl = _t(randn((K, B), g), dt), _t(randn((M, K), g, 1 / math.sqrt(K)), dt), _t(randn((M, B), g), dt)
    e, wl, el = _t(randn((M, B), g), dt), _t(randn((K, M), g, 1 / math.sqrt(K)), dt), _t(randn((K, B), g), dt)
    # weight update: W [M, Kw], contraction B (a multiple of 64)
    Bw = 128
    ew, xw, w0 = _t(randn((M, Bw), g), dt), _t(randn((K, Bw), g), dt), _t(randn((M, K), g, 1 / math.sqrt(K)), dt)
    res = {}
    from lich_amd import _native as nat

    for tile in nat.TILE_DMA_TILES:
        cfg = KernelConfig(tile=tile)
        ep = torch.empty((M, B), device=DEV, dtype=dt)
        fp = torch.empty((M, B), device=DEV, dtype=dt)
        x, a = xl.clone(), torch.empty((M, B), device=DEV, dtype=dt)
        wr, ws = w0.clone(), w0.clone()
        kp = build_prediction_error(M, K, B, act, dt, cfg)
        assert kp.tile == tile
        kp(xu, w, xl, ep)
        build_forward(M, K, B, act, dt, cfg)(xu, w, fp)
        build_inference_update(M, K, B, act, dt, cfg, 0.5, True)(x, e, wl, el, a)
        build_weight_update(M, K, Bw, act, dt, cfg, 0.01, True)(wr, ew, xw)
        build_weight_update(M, K, Bw, act, dt, cfg, 0.01, False)(ws, ew, xw)
        res[tile] = (ep, fp, x, a, wr, ws)
    torch.cuda.synchronize()
    for tile in nat.TILE_DMA_TILES[1:]:
        for i, (u, v) in enumerate(zip(res[3], res[tile])):
            assert _same(v, u, act), (tile, i)
