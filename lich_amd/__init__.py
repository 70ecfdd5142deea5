"""lich_amd: MI355X-native (gfx950) iPC training step.

Hand-written HIP kernels behind the C ABI of ``include/ipc_hip.h``
(``libipc_hip.so``, built in-tree by ``lich_amd.build``), with a Python host
surface that mirrors the reference's ``ipc_tilelang`` package: kernel
builders (``lich_amd.kernels``), layer batching, the small-batch weight
update, the trainer (``IPCConfig``, ``HipIPC``/``TileLangIPC``,
``prepare_batch``) and graph capture.
"""
from .kernels import (KernelConfig, build_forward, build_inference_update, build_prediction_error,
                      build_weight_update, build_weight_update_outer)
from .trainer import HipIPC, IPCConfig, TileLangIPC, prepare_batch

__all__ = [
    "KernelConfig", "build_prediction_error", "build_inference_update", "build_weight_update",
    "build_weight_update_outer", "build_forward", "IPCConfig", "HipIPC", "TileLangIPC", "prepare_batch",
]
__version__ = "0.1.0"
