"""Carriers of the packed operands, with comfy-kitchen's layout names and fields.

The reference passes packed weights around as ``QuantizedTensor(qdata, layout_name, params)`` and
takes them apart with ``<Layout>.get_plain_tensors(weight)`` before calling the linear ops
(roblennon/mac-kernels-public tests/test_training_packed.py:54-66, train/train_lora.py:197-223,
bench/bench_lora_fused_rank.py:38-44):

  TensorWiseINT8Layout.Params(scale, orig_dtype, orig_shape, convrot, convrot_groupsize)
      get_plain_tensors(w) -> (qdata, scale)
  AsymW4A8Int8Layout.Params(scale, s_channel, codebook, correction, group_size, convrot_groupsize,
                            orig_dtype, orig_shape, transposed)       (scale is s_rel)
      get_plain_tensors(w) -> (qdata, s_rel, s_channel, correction, codebook)

These classes hold the tensors as given (no copy, no conversion) and route ``dequantize()`` and
``linear()`` to this package's ops, so the packed storage never changes.  They are plain Python
carriers, not torch tensor subclasses: code that needs a Module parameter keeps the qdata tensor
and the carrier side by side.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

import torch

from .exceptions import NoCapableBackendError


class TensorWiseINT8Layout:
    """Per-output-channel INT8 codes, optionally in the ConvRot-rotated basis."""

    @dataclass
    class Params:
        scale: torch.Tensor
        orig_dtype: Any = torch.bfloat16
        orig_shape: Optional[tuple] = None
        convrot: bool = False
        convrot_groupsize: int = 256

    @staticmethod
    def get_plain_tensors(w: "QuantizedTensor"):
        return w._qdata, w._params.scale

    @staticmethod
    def dequantize(w: "QuantizedTensor"):
        from .ops import dequantize_int8_convrot_weight
        p = w._params
        out = dequantize_int8_convrot_weight(w._qdata, p.scale, p.convrot_groupsize if p.convrot else 0)
        return out.to(p.orig_dtype)

    @staticmethod
    def linear(x, w: "QuantizedTensor", bias=None, out_dtype=None, **kw):
        from .ops import int8_linear
        p = w._params
        return int8_linear(x, w._qdata, p.scale, bias, out_dtype, convrot=p.convrot,
                           convrot_groupsize=p.convrot_groupsize, **kw)


class AsymW4A8Int8Layout:
    """4-bit (codebook or uniform) or 6-bit codes on a per-group int8 grid, per-channel scale."""

    @dataclass
    class Params:
        scale: torch.Tensor                       # s_rel [N, K / group_size]
        s_channel: torch.Tensor
        codebook: Optional[torch.Tensor] = None
        correction: Optional[torch.Tensor] = None
        group_size: int = 16
        convrot_groupsize: int = 256
        orig_dtype: Any = torch.bfloat16
        orig_shape: Optional[tuple] = None
        transposed: bool = False

    @staticmethod
    def get_plain_tensors(w: "QuantizedTensor"):
        p = w._params
        return w._qdata, p.scale, p.s_channel, p.correction, p.codebook

    @staticmethod
    def _check(p):
        if p.transposed:
            raise NoCapableBackendError("w4a8_int8_linear", {"hip": "transposed storage is not implemented"})

    @staticmethod
    def dequantize(w: "QuantizedTensor"):
        from .ops import dequantize_w4a8_int8_weight
        p = w._params
        AsymW4A8Int8Layout._check(p)
        out = dequantize_w4a8_int8_weight(w._qdata, p.scale, p.s_channel, p.codebook, p.correction, p.group_size,
                                          p.convrot_groupsize)
        return out.to(p.orig_dtype)

    @staticmethod
    def linear(x, w: "QuantizedTensor", bias=None, out_dtype=None, **kw):
        from .ops import w4a8_int8_linear
        p = w._params
        AsymW4A8Int8Layout._check(p)
        return w4a8_int8_linear(x, w._qdata, p.scale, p.s_channel, p.codebook, p.correction, bias, p.group_size,
                                p.convrot_groupsize, out_dtype, **kw)


LAYOUTS = {"TensorWiseINT8Layout": TensorWiseINT8Layout, "AsymW4A8Int8Layout": AsymW4A8Int8Layout}


@dataclass
class QuantizedTensor:
    """qdata plus its layout name and parameters (the reference's QuantizedTensor(qdata, layout,
    params)).  `_layout_cls` is the layout's name, as the reference's trainer compares it."""
    _qdata: torch.Tensor
    _layout_cls: str
    _params: Any = field(default=None)

    def __post_init__(self):
        if self._layout_cls not in LAYOUTS:
            raise ValueError(f"unknown layout {self._layout_cls!r}; expected one of {sorted(LAYOUTS)}")

    @property
    def layout(self):
        return LAYOUTS[self._layout_cls]

    @property
    def shape(self):
        p = self._params
        if p is not None and p.orig_shape is not None:
            return torch.Size(p.orig_shape)
        n = self._qdata.shape[0]
        if self._layout_cls == "TensorWiseINT8Layout":
            return torch.Size((n, self._qdata.shape[1]))
        return torch.Size((n, p.scale.shape[1] * p.group_size))

    @property
    def dtype(self):
        return self._params.orig_dtype

    @property
    def device(self):
        return self._qdata.device

    def dequantize(self):
        return self.layout.dequantize(self)


def linear(x, weight, bias=None, out_dtype=None, **kw):
    """F.linear over a QuantizedTensor weight through the packed-weight op of its layout; any
    LoRA / residual keywords pass through."""
    if not isinstance(weight, QuantizedTensor):
        raise TypeError("weight must be a QuantizedTensor")
    return weight.layout.linear(x, weight, bias, out_dtype, **kw)
