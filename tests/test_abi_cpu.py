"""CPU tests of the C ABI and the host-side logic (no GPU, no compute calls).

Every call made here fails host-side validation before any HIP call, which
is exactly what is being tested.
"""
import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from lich_amd import _native as nat

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ipc_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|void|long long|const char\*)\s+(ipc_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(nat.LIB_PATH))
    names = _declared_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    m = re.search(r"#define IPC_ABI_VERSION (\d+)", HEADER.read_text())
    assert nat.lib().ipc_abi_version() == int(m.group(1))


def test_header_constants_match_python():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (IPC_\w+) \(?(-?\d+)\)?", text))
    assert int(consts["IPC_DT_F32"]) == nat.DT_F32 and int(consts["IPC_DT_BF16"]) == nat.DT_BF16
    assert int(consts["IPC_ACT_TANH"]) == nat.ACT_CODES["tanh"]
    assert int(consts["IPC_ACT_GELU"]) == nat.ACT_CODES["gelu"]
    assert int(consts["IPC_ERR_STATE"]) == nat.ERR_STATE
    assert int(consts["IPC_TILE_COUNT"]) == nat.TILE_COUNT


L = None


def _lib():
    return nat.lib()


P = 4096  # a fake, aligned, non-null address; never dereferenced (validation fails first)


@pytest.mark.parametrize("args,code,needle", [
    ((None, P, P, P, 64, 64, 128, 1, 0, 0, 1, 2, -1, None), nat.ERR_NULL, "x_upper"),
    ((P, P, P, P, 0, 64, 128, 1, 0, 0, 1, 2, -1, None), nat.ERR_SHAPE, "dimensions"),
    ((P, P, P, P, 64, 64, 128, 0, 0, 0, 1, 2, -1, None), nat.ERR_SHAPE, "groups"),
    ((P, P, P, P, 64, 64, 128, 1, 7, 0, 1, 2, -1, None), nat.ERR_DTYPE, "storage"),
    ((P, P, P, P, 64, 64, 128, 1, 1, 2, 1, 2, -1, None), nat.ERR_DTYPE, "16-bit"),
    ((P, P, P, P, 64, 64, 128, 1, 0, 0, 1, 9, -1, None), nat.ERR_ACT, "activation"),
    ((P, P, P, P, 64, 64, 128, 1, 0, 0, 1, 2, 7, None), nat.ERR_CONFIG, "tile"),
    ((P + 2, P, P, P, 64, 64, 128, 1, 0, 0, 1, 2, -1, None), nat.ERR_ALIGN, "aligned"),
    ((P, P, P, P, 1 << 20, 1 << 20, 128, 1, 0, 0, 1, 2, -1, None), nat.ERR_SHAPE, "too large"),
])
def test_pred_err_validation(args, code, needle):
    assert _lib().ipc_pred_err(*args) == code
    assert needle in nat.last_error()


def test_other_entry_points_validate():
    lib = _lib()
    assert lib.ipc_forward(P, P, None, 10, 64, 128, 1, 0, 0, 1, 1, -1, None) == nat.ERR_NULL
    assert lib.ipc_infer_update(P, P, P, None, None, 64, 10, 128, 1, 0.5, 0, 0, 2, -1, None) == nat.ERR_NULL
    assert lib.ipc_infer_update(P, P, P, P, P + 1, 64, 10, 128, 1, 0.5, 0, 0, 2, -1, None) == nat.ERR_ALIGN
    assert lib.ipc_weight_update(P, P, P, 64, 64, -1, 1, 1e-4, 1, 0, 0, 2, -1, None) == nat.ERR_SHAPE
    assert lib.ipc_weight_update_outer(P, P, P, 64, 64, 33, 1, 1e-4, 1, 0, 2, None) == nat.ERR_SHAPE
    assert "B <= 32" in nat.last_error()
    assert lib.ipc_weight_update_outer(P, P, P, 64, 64, 8, 1, 1e-4, 1, 0, 11, None) == nat.ERR_ACT


def test_plan_validation():
    lib = _lib()
    h = ctypes.c_void_p()
    dims = (ctypes.c_int * 4)(10, 64, 64, 784)
    assert lib.ipc_plan_create(None, 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.ERR_NULL
    assert lib.ipc_plan_create(ctypes.byref(h), 3, None, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.ERR_NULL
    assert lib.ipc_plan_create(ctypes.byref(h), 0, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.ERR_SHAPE
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 5, -1) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 64, 0, 0, 1, 2, 1e-4, 0.5, 1, 1, -1) == nat.ERR_SHAPE
    bad = (ctypes.c_int * 4)(10, 0, 64, 784)
    assert lib.ipc_plan_create(ctypes.byref(h), 3, bad, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.ERR_SHAPE
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:
        # stepping an unbound plan is a state error, not a crash
        assert lib.ipc_plan_step(h, 1, None) == nat.ERR_STATE
        assert lib.ipc_plan_forward_init(h, None) == nat.ERR_STATE
        assert lib.ipc_plan_launch_count(h) == 0
        arr = (ctypes.c_void_p * 4)(P, P, P, P)
        assert lib.ipc_plan_bind(h, None, arr, arr, None, P) == nat.ERR_NULL
        arr_bad = (ctypes.c_void_p * 4)(P, None, P, P)
        assert lib.ipc_plan_bind(h, arr_bad, arr, arr, None, P) == nat.ERR_NULL
        assert "x[1]" in nat.last_error()
        # a narrow fp32 net runs the whole-step kernel, which needs a workspace
        assert lib.ipc_plan_fused(h) == 1 and lib.ipc_plan_workspace_bytes(h) > 0
        assert lib.ipc_plan_bind(h, arr, arr, arr, None, None) == nat.ERR_NULL
        assert "workspace" in nat.last_error()
        # binding validates every pointer first; a fused plan then raises the
        # kernel's dynamic-LDS limit, the one HIP call of bind (fails without a GPU)
        rc = lib.ipc_plan_bind(h, arr, arr, arr, None, P)
        assert rc == (nat.IPC_OK if torch.cuda.is_available() else nat.ERR_LAUNCH)
        if rc == nat.IPC_OK:
            assert lib.ipc_plan_launch_count(h) == 1
    finally:
        lib.ipc_plan_destroy(h)
    # fused off: one multi-layer launch per phase, no workspace
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, 0) == nat.IPC_OK
    try:
        assert lib.ipc_plan_fused(h) == 0 and lib.ipc_plan_workspace_bytes(h) == 0
        arr = (ctypes.c_void_p * 4)(P, P, P, P)
        assert lib.ipc_plan_bind(h, arr, arr, arr, None, None) == nat.IPC_OK
        assert lib.ipc_plan_launch_count(h) == 3
    finally:
        lib.ipc_plan_destroy(h)
    # forcing the whole-step kernel on a wide net is a configuration error
    wide = (ctypes.c_int * 3)(1000, 4096, 4096)
    assert lib.ipc_plan_create(ctypes.byref(h), 2, wide, 1024, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, 1) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 2, wide, 1024, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    assert lib.ipc_plan_fused(h) == 0
    lib.ipc_plan_destroy(h)
    # 16-bit storage never takes the whole-step kernel
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 1, 1, 1, 2, 1e-4, 0.5, 1, 0, 1) == nat.ERR_CONFIG
    assert lib.ipc_plan_step(None, 1, None) == nat.ERR_NULL
    lib.ipc_plan_destroy(None)  # no-op


def _wide_layout_bytes(dims, B, split2):
    """The wide path's workspace layout restated: 256 bytes, then one 256-byte
    aligned 16-bit buffer per operand copy, rows and columns padded to 64:
    W hi [and lo] and its transpose (for l < L-1), f(x[l]) and its transpose
    for l = 1..L, eps[l] for l < L and its transpose for l < L-1, then the
    partial products of a k-split prediction of layer 0.  A split-2 net whose
    every contraction d_{l+1} is a multiple of 64 keeps no W hi / lo copies:
    its prediction reads the fp32 W itself."""
    pad = lambda v, m: (v + m - 1) // m * m  # noqa: E731
    L = len(dims) - 1
    direct = split2 and all(d % 64 == 0 for d in dims[1:])
    total = 256

    def add(rows, cols):
        nonlocal total
        total += pad(pad(rows, 64) * pad(cols, 64) * 2, 256)

    for l in range(L):
        if not direct:
            add(dims[l], dims[l + 1])
            if split2:
                add(dims[l], dims[l + 1])
        if l <= L - 2:
            add(dims[l + 1], dims[l])
    for l in range(1, L + 1):
        add(dims[l], B)
        add(B, dims[l])
    for l in range(L):
        add(dims[l], B)
        if l <= L - 2:
            add(B, dims[l])
    # fp32 partial products of a k-split layer-0 prediction: as many [d_0][B]
    # slices as keep all of layer 0's prediction tiles within 512 slices and
    # each slice a multiple of 64 long (at most 16)
    bm, bn = (128, 256) if split2 else (256, 128)
    t0 = -(-dims[0] // bm) * -(-B // bn)
    for sl in (16, 8, 4, 2):
        if sl * t0 <= 512 and pad(dims[1], 64) % (sl * 64) == 0:
            total += pad(sl * dims[0] * B * 4, 256)
            break
    return total


def test_plan_path_selection_and_wide_workspace():
    lib = _lib()
    h = ctypes.c_void_p()
    wide = (ctypes.c_int * 4)(1000, 4096, 4096, 4096)
    # AUTO on a wide fp32-master / bf16-operand net with split 2 takes the wide path
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:
        assert lib.ipc_plan_path(h) == nat.PATH_WIDE and lib.ipc_plan_fused(h) == 0
        assert lib.ipc_plan_workspace_bytes(h) == _wide_layout_bytes((1000, 4096, 4096, 4096), 1024, True)
        assert lib.ipc_plan_sync(h, None) == nat.ERR_STATE  # unbound
        arr = (ctypes.c_void_p * 4)(P, P, P, P)
        assert lib.ipc_plan_bind(h, arr, arr, arr, None, None) == nat.ERR_NULL
        assert "workspace" in nat.last_error()
        assert lib.ipc_plan_bind(h, arr, arr, arr, None, P + 16) == nat.ERR_ALIGN
        # every contraction is whole 64-k steps: the prediction reads W itself (16-byte rows)
        wmis = (ctypes.c_void_p * 4)(P, P + 4, P, P)
        assert lib.ipc_plan_bind(h, arr, arr, wmis, None, P) == nat.ERR_ALIGN
        assert "W[1]" in nat.last_error()
    finally:
        lib.ipc_plan_destroy(h)
    # a split-2 net with a contraction off the 64-k grid keeps the W hi / lo copies
    ragged2 = (10, 300, 200, 784)
    r2 = (ctypes.c_int * 4)(*ragged2)
    assert lib.ipc_plan_create(ctypes.byref(h), 3, r2, 128, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, 2) == nat.IPC_OK
    try:
        assert lib.ipc_plan_workspace_bytes(h) == _wide_layout_bytes(ragged2, 128, True)
        assert _wide_layout_bytes(ragged2, 128, True) > _wide_layout_bytes(ragged2, 128, False)
    finally:
        lib.ipc_plan_destroy(h)
    # split 1 drops the W_lo copies; ragged sizes pad rows and columns to 64
    ragged = (7, 130, 65, 257)
    rd = (ctypes.c_int * 4)(*ragged)
    assert lib.ipc_plan_create(ctypes.byref(h), 3, rd, 37, 0, 1, 1, 1, 1e-4, 0.5, 1, 0, 2) == nat.IPC_OK
    try:
        assert lib.ipc_plan_path(h) == nat.PATH_WIDE
        assert lib.ipc_plan_workspace_bytes(h) == _wide_layout_bytes(ragged, 37, False)
    finally:
        lib.ipc_plan_destroy(h)
    # the wide path is refused for fp32 operands, split 3, the outer-product update and 16-bit storage
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, 2) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 2, 3, 2, 1e-4, 0.5, 1, 0, 2) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 8, 0, 2, 2, 2, 1e-4, 0.5, 1, 1, 2) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 2, 2, 1, 2, 1e-4, 0.5, 1, 0, 2) == nat.ERR_CONFIG
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, 3) == nat.ERR_CONFIG
    # AUTO with split 3 falls back to the phased path (no workspace)
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 2, 3, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:
        assert lib.ipc_plan_path(h) == nat.PATH_PHASED and lib.ipc_plan_workspace_bytes(h) == 0
    finally:
        lib.ipc_plan_destroy(h)
    # a narrow net keeps a whole-step kernel under AUTO: the layer-resident one
    # for 16-bit operands and for fp32 operands whose blocks fit the LDS (B = 8
    # here, with the rank-B update), the column-block one when asked for or
    # for fp32 at B = 128
    narrow = (ctypes.c_int * 4)(10, 64, 64, 784)
    for operand, B, path, want in ((1, 128, -1, nat.PATH_RESIDENT), (1, 128, 1, nat.PATH_NARROW),
                                   (0, 128, -1, nat.PATH_NARROW), (0, 8, -1, nat.PATH_RESIDENT)):
        assert lib.ipc_plan_create(ctypes.byref(h), 3, narrow, B, 0, operand, 3, 2, 1e-4, 0.5, 1, 2, path) == nat.IPC_OK
        try:
            assert lib.ipc_plan_path(h) == want and lib.ipc_plan_fused(h) == 1
        finally:
            lib.ipc_plan_destroy(h)
    assert lib.ipc_plan_path(None) == -1


def _resident_ws_bytes(dims, B, recompute, esize=2):
    """Restated workspace of a layer-resident plan: the column kernel's
    barrier words and f(x) buffers, then 512 bytes of flags (step flags, the
    cache generation, the workgroups' cache slots) and the
    double-buffered exchange of 16x16 tiles (1 KiB each): eps[l] for
    l = 1..L-2, W[l]^T eps[l] for l = 0..L-2 (three buffers for l = L-2, which
    the top chunks read one step late), and one partial product per
    128-column chunk of the top layer (and one more for the next launch's
    first step); then the chunks' input images."""
    L = len(dims) - 1
    n = 256
    if recompute:
        n += sum((dims[l] * B * 4 + 255) // 256 * 256 for l in range(1, L + 1))
    n = (n + 255) // 256 * 256 + 512

    def tiles(d):
        return -(-d // 16) * -(-B // 16)

    for l in range(L - 1):
        if l >= 1:
            n += 2 * tiles(dims[l]) * 1024
        n += (3 if l + 2 == L else 2) * tiles(dims[l + 1]) * 1024
    C = -(-dims[L] // 128)
    n += (2 * (C + 1) + C) * tiles(dims[L - 1]) * 1024   # the partials, chunk 0's summed eps[L-1], the next ones
    # then, per top chunk, its cached f(x[L]) operands as laid out in LDS
    # (16-bit, split 3: hi and lo [B16][K32+8], hi [K16][B32+8]; fp32: [B16][K16+4]
    # and [K16][B16+4]), 256-byte aligned
    r = lambda v, m: -(-v // m) * m  # noqa: E731
    K = min(dims[L], 128)
    if esize == 2:
        image = r((2 * r(B, 16) * (r(K, 32) + 8) + r(K, 16) * (r(B, 32) + 8)) * 2, 256)
    else:
        image = r((r(B, 16) * (r(K, 16) + 4) + r(K, 16) * (r(B, 16) + 4)) * 4, 256)
    return r(n, 256) + C * image


@pytest.mark.parametrize("dims,B,recompute,operand", [
    ((10, 64, 64, 64, 64, 64, 64, 784), 128, 1, 2),
    ((10, 64, 784), 128, 0, 2),
    ((7, 33, 48, 130), 40, 1, 2),
    ((3, 64, 100), 17, 1, 2),
    ((10, 64, 64, 64, 64, 784), 8, 1, 0),
    ((7, 33, 48, 130), 40, 0, 0),
    ((10, 64, 784), 64, 1, 0),
])
def test_resident_plan_workspace(dims, B, recompute, operand):
    lib = _lib()
    h = ctypes.c_void_p()
    L = len(dims) - 1
    d = (ctypes.c_int * (L + 1))(*dims)
    assert lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, operand, 3, 2, 1e-4, 0.5, recompute, 0, 3) == nat.IPC_OK
    try:
        assert lib.ipc_plan_path(h) == nat.PATH_RESIDENT
        assert lib.ipc_plan_workspace_bytes(h) == _resident_ws_bytes(dims, B, recompute, 4 if operand == 0 else 2)
    finally:
        lib.ipc_plan_destroy(h)


@pytest.mark.parametrize("dims,B,operand,split,wmode,why", [
    ((10, 64, 64, 784), 128, 0, 1, 0, "fp32 operand blocks beyond the LDS"),
    ((10, 64, 64, 784), 256, 1, 3, 0, "batch above 128"),
    ((10, 128, 64, 784), 128, 1, 3, 0, "hidden width above 64"),
    ((10, 784), 128, 1, 3, 0, "a single layer"),
    ((10, 64, 64, 784), 8, 1, 3, 2, "rank-B outer-product weight update"),
    ((10, 64, 64, 784), 128, 1, 2, 0, "split 2"),
])
def test_resident_path_refuses_ineligible_nets(dims, B, operand, split, wmode, why):
    lib = _lib()
    h = ctypes.c_void_p()
    L = len(dims) - 1
    d = (ctypes.c_int * (L + 1))(*dims)
    rc = lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, operand, split, 2, 1e-4, 0.5, 1, wmode, 3)
    assert rc == nat.ERR_CONFIG, why
    assert "layer-resident" in nat.last_error()
    # AUTO then picks another path
    if lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, operand, split, 2, 1e-4, 0.5, 1, wmode, -1) == nat.IPC_OK:
        try:
            assert lib.ipc_plan_path(h) != nat.PATH_RESIDENT
        finally:
            lib.ipc_plan_destroy(h)


def test_check_maps_codes_to_exceptions():
    _lib().ipc_pred_err(None, P, P, P, 64, 64, 128, 1, 0, 0, 1, 2, -1, None)
    with pytest.raises(ValueError, match="x_upper is NULL"):
        nat.check(nat.ERR_NULL)
    with pytest.raises(nat.IPCNativeError):
        nat.check(nat.ERR_LAUNCH)
    nat.check(nat.IPC_OK)


def test_device_check_refuses_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(nat.IPCNativeError):
        nat.device_arch(0)


def test_kernel_config_tile_mapping():
    from lich_amd.kernels import KernelConfig
    assert KernelConfig().tile_id() == -1
    assert KernelConfig(64, 128, 16, 128, 2, True, 8, False).tile_id() == 1  # reference scripts' config
    assert KernelConfig(128, 128).tile_id() == 2
    assert KernelConfig(32, 32).tile_id() == 0
    assert KernelConfig(tile=0).tile_id() == 0
    with pytest.raises(ValueError):
        KernelConfig(tile=9).tile_id()


def test_builders_validate_arguments_on_host():
    from lich_amd.kernels import build_prediction_error, build_weight_update_outer
    with pytest.raises(ValueError):
        build_prediction_error(64, 64, 128, "softplus", "float32")
    with pytest.raises(ValueError):
        build_prediction_error(64, 64, 128, "tanh", "float16", operand_dtype="bfloat16")
    with pytest.raises(ValueError):
        build_prediction_error(0, 64, 128, "tanh", "float32")
    with pytest.raises(ValueError):
        build_weight_update_outer(64, 64, 64, "tanh", "float32")
    k = build_prediction_error(64, 64, 128, "tanh", "float32")
    with pytest.raises(ValueError, match="device tensor"):
        k(torch.zeros(64, 128), torch.zeros(64, 64), torch.zeros(64, 128), torch.zeros(64, 128))


def test_find_internal_square_groups_matches_reference_semantics():
    from lich_amd.layer_batching import LayerBatchGroup, find_internal_square_groups as f
    d6 = (10,) + (64,) * 6 + (784,)
    assert f(d6, max_group_count=2) == (LayerBatchGroup(1, 2, 64), LayerBatchGroup(4, 5, 64))
    assert f(d6, max_group_count=5) == (LayerBatchGroup(1, 5, 64),)
    assert f((10,) + (64,) * 4 + (784,), max_group_count=3) == (LayerBatchGroup(1, 3, 64),)
    assert f((10, 64, 784), max_group_count=2) == ()
    assert f(d6, max_group_count=1) == ()
    g = LayerBatchGroup(1, 3, 64)
    assert g.count == 3 and g.state_count == 4 and g.state_indices == (1, 2, 3, 4)


def test_batched_builders_require_square_groups():
    from lich_amd.layer_batching import build_prediction_error_batched
    with pytest.raises(ValueError):
        build_prediction_error_batched(64, 64, 128, 1, "tanh", "float32")
    with pytest.raises(ValueError):
        build_prediction_error_batched(64, 32, 128, 2, "tanh", "float32")


def test_small_b_policy_reader(tmp_path):
    from lich_amd.weight_update_specialization import SmallBWeightPolicy
    p = tmp_path / "policy.json"
    p.write_text(json.dumps({"entries": [
        {"M": 64, "K": 784, "B": 4, "activation": "relu", "dtype": "float16", "backend": "outer"},
        {"M": 64, "K": 64, "B": 4, "backend": "bogus"},
        {"K": 1},
    ]}))
    pol = SmallBWeightPolicy(p)
    assert pol.backend(M=64, K=784, B=4, activation="relu", dtype=torch.float16) == "outer"
    assert pol.backend(M=64, K=64, B=4, activation="relu", dtype=torch.float16) == "gemm"


def test_product_init_matches_oracle_init():
    from lich_amd.trainer import init_weights_cpu
    from oracle.ipc_oracle import init_weights
    dims = (10, 64, 64, 784)
    for init in ("kaiming_a_sqrt5", "xavier_uniform"):
        for a, b in zip(init_weights_cpu(dims, seed=5, init=init), init_weights(dims, seed=5, init=init)):
            assert torch.equal(a, b)


def test_prepare_batch_layout():
    from lich_amd.trainer import prepare_batch
    imgs = torch.rand(5, 1, 28, 28)
    labels = torch.tensor([3, 1, 4, 1, 5])
    x, y = prepare_batch(imgs, labels, device="cpu", dtype=torch.float32, num_classes=10)
    assert x.shape == (784, 5) and y.shape == (10, 5)
    assert torch.equal(x[:, 2], imgs[2].flatten())
    assert y[:, 0].argmax() == 3 and float(y.sum()) == 5


def test_trainer_refuses_cpu_device():
    from lich_amd.trainer import HipIPC, IPCConfig
    with pytest.raises(ValueError):
        HipIPC(IPCConfig(dims=(10, 64, 784)), device="cpu")


def test_health_entry_points_validate_arguments():
    lib = _lib()
    assert lib.ipc_plan_check(None, None) == nat.ERR_NULL
    assert lib.ipc_plan_set_spin_limit(None, 0) == nat.ERR_NULL
    assert lib.ipc_set_coresident_limit(-1) == nat.ERR_CONFIG
    dims = (ctypes.c_int * 4)(10, 64, 64, 784)
    h = ctypes.c_void_p()
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:
        assert lib.ipc_plan_check(h, None) == nat.ERR_STATE  # unbound: nothing to check yet
        assert lib.ipc_plan_set_spin_limit(h, 0) == nat.IPC_OK
        assert lib.ipc_plan_set_spin_limit(h, -1) == nat.IPC_OK
    finally:
        lib.ipc_plan_destroy(h)


def test_resident_plan_refused_when_its_workgroups_cannot_run_at_once():
    """A device that holds fewer workgroups at once than a layer-resident
    launch starts (modelled with the co-resident limit hook): an explicit
    resident plan fails with IPC_ERR_CONFIG, an AUTO plan takes the column
    kernel.  Without a device (this container) the capacity is unknown and the
    choice is the usual one."""
    lib = _lib()
    d6 = (ctypes.c_int * 8)(10, 64, 64, 64, 64, 64, 64, 784)
    h = ctypes.c_void_p()
    try:
        assert lib.ipc_set_coresident_limit(8) == nat.IPC_OK
        rc = lib.ipc_plan_create(ctypes.byref(h), 7, d6, 128, 0, 1, 3, 2, 1e-4, 0.5, 1, 0, nat.PATH_RESIDENT)
        assert rc == nat.ERR_CONFIG and "co-resident" in nat.last_error()
        assert lib.ipc_plan_create(ctypes.byref(h), 7, d6, 128, 0, 1, 3, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
        assert lib.ipc_plan_path(h) == nat.PATH_NARROW
        lib.ipc_plan_destroy(h)
        assert lib.ipc_set_coresident_limit(64) == nat.IPC_OK
        assert lib.ipc_plan_create(ctypes.byref(h), 7, d6, 128, 0, 1, 3, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
        assert lib.ipc_plan_path(h) == nat.PATH_RESIDENT
        lib.ipc_plan_destroy(h)
    finally:
        assert lib.ipc_set_coresident_limit(0) == nat.IPC_OK
    assert lib.ipc_plan_create(ctypes.byref(h), 7, d6, 128, 0, 1, 3, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    assert lib.ipc_plan_path(h) == nat.PATH_RESIDENT
    lib.ipc_plan_destroy(h)


def test_graph_entry_points_validate_arguments():
    lib = _lib()
    assert lib.ipc_plan_graph_capture(None, 4) == nat.ERR_NULL
    assert lib.ipc_plan_graph_launch(None, 1, None) == nat.ERR_NULL
    assert lib.ipc_plan_graph_steps(None) == 0
    dims = (ctypes.c_int * 4)(10, 64, 64, 784)
    h = ctypes.c_void_p()
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:
        assert lib.ipc_plan_graph_capture(h, 4) == nat.ERR_STATE  # unbound
        assert lib.ipc_plan_graph_launch(h, 1, None) == nat.ERR_STATE  # nothing captured
        assert "no captured graph" in nat.last_error()
        assert lib.ipc_plan_graph_steps(h) == 0
    finally:
        lib.ipc_plan_destroy(h)


def test_noalloc_entry_point_validates_on_the_host():
    lib = _lib()
    d = (ctypes.c_int * 4)(10, 64, 64, 784)
    arr = (ctypes.c_void_p * 4)(P, P, P, P)
    args = (3, d, 128, arr, arr, arr, nat.DT_F16, 3, 2, 1e-4, 0.5, 0)
    assert lib.ipc_steps_noalloc(3, None, 128, arr, arr, arr, nat.DT_F16, 3, 2, 1e-4, 0.5, 0, 1, None) == nat.ERR_NULL
    assert lib.ipc_steps_noalloc(*args[:3], None, arr, arr, *args[6:], 1, None) == nat.ERR_NULL
    assert lib.ipc_steps_noalloc(*args, -1, None) == nat.ERR_SHAPE
    wide = (ctypes.c_int * 3)(1000, 4096, 4096)
    assert lib.ipc_steps_noalloc(2, wide, 1024, arr, arr, arr, nat.DT_BF16, 2, 2, 1e-4, 0.5, 0, 1, None) == nat.ERR_CONFIG
    # the f(x) buffers of B = 4096 exceed the 8 MiB static scratch: refused before any HIP call
    assert lib.ipc_steps_noalloc(3, d, 4096, arr, arr, arr, nat.DT_F16, 3, 2, 1e-4, 0.5, 0, 1, None) == nat.ERR_SHAPE
    assert "scratch" in nat.last_error()
    # zero steps of an acceptable net: validated, nothing enqueued
    assert lib.ipc_steps_noalloc(*args, 0, None) == nat.IPC_OK


def test_wide_tile_configurations_are_selectable_before_bind():
    lib = _lib()
    assert lib.ipc_plan_wide_config_count(0, nat.SPLIT_W) == 2 and lib.ipc_plan_wide_config_count(0, 1) == 2
    assert lib.ipc_plan_wide_config_count(1, 1) == 4 and lib.ipc_plan_wide_config_count(2, 1) == 5
    assert lib.ipc_plan_wide_config_count(0, nat.SPLIT_WX) == 0 and lib.ipc_plan_wide_config_count(7, 1) == 0
    assert lib.ipc_plan_set_wide_config(None, 0, 0, 0, -1) == nat.ERR_NULL
    dims = (ctypes.c_int * 4)(10, 64, 64, 784)
    h = ctypes.c_void_p()
    assert lib.ipc_plan_create(ctypes.byref(h), 3, dims, 128, 0, 0, 1, 2, 1e-4, 0.5, 1, 0, -1) == nat.IPC_OK
    try:  # not a wide plan
        assert lib.ipc_plan_set_wide_config(h, 0, 0, 0, -1) == nat.ERR_CONFIG
    finally:
        lib.ipc_plan_destroy(h)
    wide = (ctypes.c_int * 4)(1000, 4096, 4096, 4096)
    assert lib.ipc_plan_create(ctypes.byref(h), 3, wide, 1024, 0, 2, 2, 2, 1e-4, 0.5, 1, 0, nat.PATH_WIDE) == nat.IPC_OK
    try:
        base = lib.ipc_plan_workspace_bytes(h)
        assert lib.ipc_plan_set_wide_config(h, 2, 0, 0, -1) == nat.ERR_CONFIG   # split-2 prediction has 0..1
        assert lib.ipc_plan_set_wide_config(h, 0, 0, 5, -1) == nat.ERR_CONFIG   # weight has 0..4
        assert lib.ipc_plan_set_wide_config(h, 0, 0, 0, 3) == nat.ERR_CONFIG    # not a power of two
        assert lib.ipc_plan_set_wide_config(h, -1, 1, 2, 8) == nat.IPC_OK
        assert lib.ipc_plan_workspace_bytes(h) == base                          # same prediction tile
        # the 128 x 128 prediction tile: twice the output tiles of layer 0, half the slices
        assert lib.ipc_plan_set_wide_config(h, 1, 0, 0, -1) == nat.IPC_OK
        assert lib.ipc_plan_workspace_bytes(h) < base
    finally:
        lib.ipc_plan_destroy(h)


def test_s16_preactivate_hook_validates_its_mode():
    lib = _lib()
    assert lib.ipc_set_s16_preactivate(2) == nat.ERR_CONFIG and "pre-activation" in nat.last_error()
    assert lib.ipc_set_s16_preactivate(-2) == nat.ERR_CONFIG
    for mode in (0, 1, -1):
        assert lib.ipc_set_s16_preactivate(mode) == nat.IPC_OK


def test_s16_preactivation_rule():
    """The automatic rule: exp-based activations from M >= 1024 and K*B >= 2^20,
    relu from M >= 4096 and K*B >= 2^22, never identity; the inference update
    (which copies its operands transposed) from M*K >= 2^26 and K*B >= 2^26,
    whatever the activation; mode 0 turns it off, mode 1 on.  The workspace
    sizes follow: K*B*2 per group, (M*K + K*B)*2 for the inference update."""
    lib = _lib()
    tanh, relu, ident = nat.act_code("tanh"), nat.act_code("relu"), nat.act_code("identity")
    q = lib.ipc_s16_preactivates
    assert q(0, tanh, 1024, 1024, 1024) == 1 and q(2, tanh, 1024, 1024, 1024) == 1
    assert q(0, tanh, 1023, 1024, 1024) == 0 and q(0, tanh, 1024, 1024, 512) == 0
    assert q(0, relu, 4096, 4096, 1024) == 1 and q(0, relu, 2048, 4096, 2048) == 0
    assert q(0, relu, 4096, 1024, 2048) == 0
    assert q(0, ident, 8192, 8192, 8192) == 0
    assert q(1, tanh, 8192, 8192, 8192) == 1 and q(1, ident, 8192, 8192, 8192) == 1
    assert q(1, relu, 8192, 8192, 4096) == 0 and q(1, tanh, 4096, 8192, 8192) == 0
    wb = lib.ipc_s16_workspace_bytes
    assert wb(0, tanh, 1024, 1024, 1024, 3) == 3 * 1024 * 1024 * 2
    assert wb(1, relu, 8192, 8192, 8192, 2) == 2 * (8192 * 8192 + 8192 * 8192) * 2
    assert wb(1, relu, 4096, 4096, 2048, 1) == 0 and wb(0, ident, 8192, 8192, 8192, 1) == 0
    try:
        assert lib.ipc_set_s16_preactivate(0) == nat.IPC_OK and q(0, tanh, 8192, 8192, 8192) == 0
        assert lib.ipc_set_s16_preactivate(1) == nat.IPC_OK and q(0, relu, 8, 64, 8) == 1
    finally:
        lib.ipc_set_s16_preactivate(-1)


def test_split2_problem_without_lo_operand_is_refused_on_the_host():
    """A split-2 LDS-DMA kernel that does not split the fp32 W itself loads a
    lo block next to every W block; a problem without that operand would read
    through a null pointer on every workgroup (a GPU memory fault, not an error
    code).  Every launch checks each problem on the host first, before its
    first HIP call, for the prediction and the forward initialisation alike."""
    lib = _lib()
    P, I, W, F = 0, 1, 2, 3
    chk = lib.ipc_wide_problem_check
    for phase in (P, F):
        assert chk(phase, 2, 0, 0, 4096, 1) == nat.ERR_CONFIG, phase
        assert "refused" in nat.last_error()
        assert chk(phase, 2, 0, 1, 4096, 1) == nat.IPC_OK   # lo operand passed
        assert chk(phase, 2, 1, 0, 4096, 1) == nat.IPC_OK   # the kernel splits the fp32 W itself
        assert chk(phase, 1, 0, 0, 4096, 1) == nat.IPC_OK   # unsplit: no lo operand read
    for phase in (I, W):
        assert chk(phase, 1, 0, 0, 1024, 1) == nat.IPC_OK
    # k-split slices are whole 64-k steps
    assert chk(P, 2, 1, 0, 4096, 8) == nat.IPC_OK
    assert chk(P, 2, 1, 0, 4096, 128) == nat.ERR_CONFIG
    assert chk(P, 1, 0, 0, 4160, 2) == nat.ERR_CONFIG
    assert chk(7, 1, 0, 0, 64, 1) == nat.ERR_CONFIG


def test_resident_row_blocks_are_a_plan_option():
    """ipc_plan_set_resident_rows: 16, 32 (the default) or 64 rows of the top
    layer per workgroup on a layer-resident plan, before bind; other sizes,
    other paths and nets whose blocks do not fit are refused and leave the
    plan as it was.  The exchange records are per 16-row tile, so the
    workspace does not depend on the size."""
    lib = _lib()
    dims, B = (10,) + (64,) * 6 + (784,), 128
    L = len(dims) - 1
    d = (ctypes.c_int * (L + 1))(*dims)
    h = ctypes.c_void_p()
    assert lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, nat.DT_F16, 1, 2, 1e-4, 0.5, 1, 0, 3) == nat.IPC_OK
    try:
        ws = lib.ipc_plan_workspace_bytes(h)
        assert lib.ipc_plan_resident_rows(h) == 32
        for rows in (16, 64, 32, -1):
            assert lib.ipc_plan_set_resident_rows(h, rows) == nat.IPC_OK, nat.last_error()
            assert lib.ipc_plan_resident_rows(h) == (32 if rows == -1 else rows)
            assert lib.ipc_plan_workspace_bytes(h) == ws
        assert lib.ipc_plan_set_resident_rows(h, 48) == nat.ERR_CONFIG and "16, 32 or 64" in nat.last_error()
        assert lib.ipc_plan_resident_rows(h) == 32
    finally:
        lib.ipc_plan_destroy(h)
    assert lib.ipc_plan_set_resident_rows(None, 16) == nat.ERR_NULL
    # a column-kernel plan has no row blocks
    assert lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, nat.DT_F16, 1, 2, 1e-4, 0.5, 1, 0, 1) == nat.IPC_OK
    try:
        assert lib.ipc_plan_set_resident_rows(h, 16) == nat.ERR_CONFIG and lib.ipc_plan_resident_rows(h) == 0
    finally:
        lib.ipc_plan_destroy(h)
    # split 3 with 64-row blocks of a 784-wide input: the block's operands exceed the LDS
    assert lib.ipc_plan_create(ctypes.byref(h), L, d, B, 0, nat.DT_BF16, 3, 2, 1e-4, 0.5, 1, 0, 3) == nat.IPC_OK
    try:
        rc = lib.ipc_plan_set_resident_rows(h, 64)
        assert rc in (nat.IPC_OK, nat.ERR_CONFIG)
        assert lib.ipc_plan_resident_rows(h) == (64 if rc == nat.IPC_OK else 32)
    finally:
        lib.ipc_plan_destroy(h)


def test_dma_tile_ids_are_refused_where_the_dma_kernel_cannot_run():
    """The LDS-DMA tile ids need 16-bit storage and a contraction of
    whole 64-k steps; asked for otherwise they are an error, never a silent
    fallback; an id past the table is unknown."""
    lib = _lib()
    for tile in nat.TILE_DMA_TILES:
        rc = lib.ipc_pred_err(P, P, P, P, 64, 64, 128, 1, nat.DT_F32, nat.DT_F32, 1, 2, tile, None)
        assert rc == nat.ERR_CONFIG and "LDS-DMA" in nat.last_error()
        rc = lib.ipc_pred_err(P, P, P, P, 64, 100, 128, 1, nat.DT_BF16, nat.DT_BF16, 1, 2, tile, None)
        assert rc == nat.ERR_CONFIG and "LDS-DMA" in nat.last_error()
    assert lib.ipc_pred_err(P, P, P, P, 64, 64, 128, 1, nat.DT_BF16, nat.DT_BF16, 1, 2, nat.TILE_COUNT, None) == \
        nat.ERR_CONFIG
