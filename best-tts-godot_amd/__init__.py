"""MI355X (gfx950) tensor-op layer for the quantized Kokoro-82M graph.

The package mirrors the reference's per-op interface,
``RefRuntime.dispatch(op, node_input, node_output, attrs, env)``
(tools/ref_runtime.py:428-668), on top of libkk: hand-written HIP kernels
behind a C ABI (include/kk.h) loaded with ctypes.  There is no CPU path:
importing works without a GPU, but every op needs libkk and a device.

The directory name is not a Python identifier; import it with
``importlib.import_module("best-tts-godot_amd")``.
"""
from . import _lib  # noqa: F401
from .dispatch import dispatch, to_device, to_host  # noqa: F401
from .tensor import (DeviceTensor, device_count, dispatch_count, init, pool_stats,  # noqa: F401
                     pool_trim, sync)
from . import ops  # noqa: F401

__all__ = ["dispatch", "to_device", "to_host", "DeviceTensor", "init", "sync",
           "pool_stats", "pool_trim", "device_count", "dispatch_count", "ops"]
