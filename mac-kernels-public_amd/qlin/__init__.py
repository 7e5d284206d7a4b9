"""qlin: packed-weight quantized linear ops for AMD MI355X (gfx950).

Drop-in for comfy-kitchen's packed-weight linear family (roblennon/mac-kernels-public): INT8 with
ConvRot rotation (weight-only, fp16 MFMA), W4A8 / W6A8 (AsymW4A8Int8 storage, int8 MFMA on
per-token int8 activations) and the GGUF block formats Q4_0..Q6_K, IQ4_NL, IQ4_XS (weight-only,
decoded inside the kernels).  Everything runs in libqlin.so (HIP, C ABI in include/qlin.h).
"""
from .autograd import int8_linear_grad_input, int8_linear_trainable, w4a8_linear_grad_input, w4a8_linear_trainable
from .exceptions import NoCapableBackendError, QlinError
from .gguf import GGUF_TYPES, gguf_type_id
from .layouts import AsymW4A8Int8Layout, QuantizedTensor, TensorWiseINT8Layout
from .loader import PackedLinear, gguf_header, load_gguf, load_safetensors, quantized_linears, safetensors_header
from .ops import (
    dequantize_gguf,
    dequantize_int8,
    dequantize_int8_convrot_weight,
    dequantize_w4a8_int8_weight,
    gguf_linear,
    int8_linear,
    quantize_int8_rowwise,
    w4a8_int8_grid,
    w4a8_int8_linear,
)
from .registry import registry

__all__ = [
    "NoCapableBackendError", "QlinError", "GGUF_TYPES", "gguf_type_id", "dequantize_gguf", "dequantize_int8",
    "dequantize_int8_convrot_weight", "dequantize_w4a8_int8_weight", "gguf_linear", "int8_linear",
    "quantize_int8_rowwise", "w4a8_int8_grid", "w4a8_int8_linear", "registry", "PackedLinear", "gguf_header",
    "load_gguf", "load_safetensors", "quantized_linears", "safetensors_header", "int8_linear_grad_input",
    "int8_linear_trainable", "w4a8_linear_grad_input", "w4a8_linear_trainable", "AsymW4A8Int8Layout",
    "QuantizedTensor", "TensorWiseINT8Layout",
]
