"""Capability registry mirroring comfy-kitchen's op dispatch.

Reference behaviour (roblennon/mac-kernels-public): ops are looked up with
``registry.get_implementation(func_name, backend=None, kwargs=None)`` (bench/te_encode.py:82-90,
bench/review_layer_load.py:136-158); a backend that does not declare an opt-in keyword (the
``lora_*`` family) is skipped, and when no backend accepts the call the registry raises
``NoCapableBackendError(func_name, {backend: reason})`` (tests/test_lora_sidepath.py:274-296).
A disabled backend keeps its capabilities listed (docs/upstream/comfyui-mps-kitchen-formats.md:18).
ComfyUI maps capabilities to formats: int8_linear -> int8_tensorwise, w4a8_int8_linear ->
asym_w4a8_int8 / w6a8_int8 (docs/upstream/comfyui-mps-kitchen-formats.md:13-15).
"""
from __future__ import annotations

import os

from . import ops
from .exceptions import NoCapableBackendError

# func name -> (callable, keyword arguments the backend accepts beyond the plain signature)
_HIP = {
    "int8_linear": (ops.int8_linear, {"lora_down", "lora_up", "lora_scale"}),
    "w4a8_int8_linear": (ops.w4a8_int8_linear, {"lora_down", "lora_up", "lora_scale"}),
    "gguf_linear": (ops.gguf_linear, {"lora_down", "lora_up", "lora_scale"}),
    "dequantize_gguf": (ops.dequantize_gguf, set()),
    "dequantize_int8_convrot_weight": (ops.dequantize_int8_convrot_weight, set()),
    "dequantize_w4a8_int8_weight": (ops.dequantize_w4a8_int8_weight, set()),
    "quantize_int8_rowwise": (ops.quantize_int8_rowwise, set()),
}
_OPT_IN = {"lora_down", "lora_up", "lora_scale", "correction"}

FORMATS = {"int8_linear": ("int8_tensorwise",), "w4a8_int8_linear": ("asym_w4a8_int8", "w6a8_int8"),
           "gguf_linear": ("gguf",)}


class Registry:
    def __init__(self):
        self.backends = {"hip": _HIP}

    def capabilities(self, backend="hip"):
        return sorted(self.backends[backend])

    def enabled(self, backend="hip"):
        return os.environ.get("QLIN_DISABLE", "0") in ("", "0")

    def get_implementation(self, func_name, backend=None, kwargs=None):
        reasons = {}
        names = [backend] if backend else list(self.backends)
        for name in names:
            table = self.backends.get(name)
            if table is None:
                reasons[name] = "unknown backend"
                continue
            if not self.enabled(name):
                reasons[name] = "disabled by QLIN_DISABLE"
                continue
            if func_name not in table:
                reasons[name] = "capability not provided"
                continue
            fn, accepted = table[func_name]
            used = {k for k, v in (kwargs or {}).items() if k in _OPT_IN and v is not None}
            missing = used - accepted
            if missing:
                reasons[name] = f"does not accept {sorted(missing)}"
                continue
            return fn
        raise NoCapableBackendError(func_name, reasons)


registry = Registry()
