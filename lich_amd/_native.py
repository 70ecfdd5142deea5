"""ctypes binding of ``libipc_hip.so`` (the C ABI of ``include/ipc_hip.h``).

The library is built in-tree by ``lich_amd.build``.  It links the HIP runtime
by soname, so torch is imported first and its already-loaded HIP runtime is
the one the library binds to.  There is no fallback: if the library is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_longlong, c_void_p
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "libipc_hip.so"

# status codes (include/ipc_hip.h)
IPC_OK = 0
ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ACT, ERR_ALIGN, ERR_DEVICE, ERR_LAUNCH, ERR_CONFIG, ERR_STATE, ERR_TIMEOUT = (
    -1, -2, -3, -4, -5, -6, -7, -8, -9, -10)

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
ACT_CODES = {"identity": 0, "linear": 0, "relu": 1, "tanh": 2, "sigmoid": 3, "silu": 4, "gelu": 5}
TILE_AUTO = -1
TILE_DMA = 3
TILE_DMA_TILES = (3, 4, 5, 6)  # LDS-DMA kernel: 256 x 128, 128 x 256, 128 x 128, 256 x 256
TILE_COUNT = 7
WMODE = {"gemm": 0, "outer": 1, "auto": 2}
SPLIT_NONE, SPLIT_W, SPLIT_WX = 1, 2, 3
PATH_AUTO, PATH_PHASED, PATH_NARROW, PATH_WIDE, PATH_RESIDENT = -1, 0, 1, 2, 3
# plan path option (IPCConfig.fused): the IPC_PATH_* codes; "off"/"on" are the
# IPC_FUSED_* spellings of phased / narrow
FUSED = {"auto": PATH_AUTO, "off": PATH_PHASED, "phased": PATH_PHASED, "on": PATH_NARROW, "narrow": PATH_NARROW,
         "wide": PATH_WIDE, "resident": PATH_RESIDENT}
PATH_NAMES = {PATH_PHASED: "phased", PATH_NARROW: "narrow", PATH_WIDE: "wide", PATH_RESIDENT: "resident"}

_DTYPE_CODES = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}


class IPCNativeError(RuntimeError):
    """A HIP-side failure reported by the library (launch or device errors)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[ipc_hip {code}] {message}")
        self.code = code


def dtype_code(dtype) -> int:
    if isinstance(dtype, str):
        dtype = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
                 "fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}.get(dtype, dtype)
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise ValueError(f"Unsupported dtype {dtype!r}; expected float32, float16 or bfloat16") from exc


def act_code(name: str) -> int:
    try:
        return ACT_CODES[str(name).lower()]
    except KeyError as exc:
        raise ValueError(f"Unsupported activation {name!r}") from exc


_lib = None


def _declare(lib):
    vp, i, f = c_void_p, c_int, c_float
    sig = {
        "ipc_abi_version": ([], i),
        "ipc_last_error": ([], c_char_p),
        "ipc_device_check": ([i, c_char_p, i], i),
        "ipc_pred_err": ([vp, vp, vp, vp, i, i, i, i, i, i, i, i, i, vp], i),
        "ipc_forward": ([vp, vp, vp, i, i, i, i, i, i, i, i, i, vp], i),
        "ipc_infer_update": ([vp, vp, vp, vp, vp, i, i, i, i, f, i, i, i, i, vp], i),
        "ipc_weight_update": ([vp, vp, vp, i, i, i, i, f, i, i, i, i, i, vp], i),
        "ipc_weight_update_outer": ([vp, vp, vp, i, i, i, i, f, i, i, i, vp], i),
        "ipc_pred_err_ws": ([vp, vp, vp, vp, i, i, i, i, i, i, i, i, i, vp, c_longlong, vp], i),
        "ipc_forward_ws": ([vp, vp, vp, i, i, i, i, i, i, i, i, i, vp, c_longlong, vp], i),
        "ipc_weight_update_ws": ([vp, vp, vp, i, i, i, i, f, i, i, i, i, i, vp, c_longlong, vp], i),
        "ipc_infer_update_ws": ([vp, vp, vp, vp, vp, i, i, i, i, f, i, i, i, i, vp, c_longlong, vp], i),
        "ipc_s16_workspace_bytes": ([i, i, i, i, i, i], c_longlong),
        "ipc_plan_create": ([POINTER(vp), i, POINTER(c_int), i, i, i, i, i, f, f, i, i, i], i),
        "ipc_plan_fused": ([vp], i),
        "ipc_plan_path": ([vp], i),
        "ipc_plan_set_tiles": ([vp, i, i, i], i),
        "ipc_plan_workspace_bytes": ([vp], c_longlong),
        "ipc_plan_bind": ([vp, POINTER(vp), POINTER(vp), POINTER(vp), POINTER(vp), vp], i),
        "ipc_plan_step": ([vp, i, vp], i),
        "ipc_plan_forward_init": ([vp, vp], i),
        "ipc_plan_sync": ([vp, vp], i),
        "ipc_plan_phase": ([vp, i, i, vp], i),
        "ipc_plan_launch_count": ([vp], i),
        "ipc_plan_check": ([vp, vp], i),
        "ipc_plan_set_spin_limit": ([vp, i], i),
        "ipc_plan_wide_config_count": ([i, i], i),
        "ipc_plan_set_wide_config": ([vp, i, i, i, i], i),
        "ipc_plan_set_resident_rows": ([vp, i], i),
        "ipc_plan_resident_rows": ([vp], i),
        "ipc_set_coresident_limit": ([i], i),
        "ipc_set_s16_preactivate": ([i], i),
        "ipc_s16_preactivates": ([i, i, i, i, i], i),
        "ipc_wide_problem_check": ([i, i, i, i, i, i], i),
        "ipc_noalloc_check": ([vp], i),
        "ipc_noalloc_set_spin_limit": ([i], i),
        "ipc_plan_graph_capture": ([vp, i], i),
        "ipc_plan_graph_launch": ([vp, i, vp], i),
        "ipc_plan_graph_steps": ([vp], i),
        "ipc_steps_noalloc": ([i, POINTER(c_int), i, POINTER(vp), POINTER(vp), POINTER(vp), i, i, i, f, f, i, i, vp],
                              i),
        "ipc_plan_destroy": ([vp], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def lib():
    """The loaded library (loads it on first use; raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -m lich_amd.build or __graft_entry__.build()); there is no CPU fallback")
        _lib = _declare(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def last_error() -> str:
    msg = lib().ipc_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    """Raise for a non-zero status: argument errors as ValueError (as the
    reference's builders and TileLang adapter do), HIP failures as
    IPCNativeError."""
    if rc == IPC_OK:
        return
    msg = last_error()
    if rc in (ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ACT, ERR_ALIGN, ERR_CONFIG):
        raise ValueError(f"[ipc_hip {rc}] {msg}")
    raise IPCNativeError(rc, msg)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream, read at call time so that calls
    made under ``torch.cuda.graph`` land on the capture stream.  torch's raw
    accessor returns the same handle without building a Stream object (about
    3 us less per call on MI355X, which a whole-step replay's wall time
    carries before its first launch)."""
    if _raw_stream is not None:
        if device is None:
            index = torch.cuda.current_device()
        elif isinstance(device, int):
            index = device
        elif isinstance(device, torch.device) and device.index is not None:
            index = device.index
        else:
            index = torch.device(device).index
            if index is None:
                index = torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def device_arch(device_index: int = 0) -> str:
    buf = ctypes.create_string_buffer(64)
    rc = lib().ipc_device_check(int(device_index), buf, 64)
    arch = buf.value.decode()
    check(rc)
    return arch
