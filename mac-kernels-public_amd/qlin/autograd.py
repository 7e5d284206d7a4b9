"""Frozen-weight training on packed bases: the input gradient of the quantized linears and the
autograd wrappers that use it.

Mirrors comfy-kitchen's MPS training entry points as roblennon/mac-kernels-public calls them:
  - int8_linear_grad_input(dy, qdata, scale, convrot, convrot_groupsize, out_dtype=None)
    (bench/bench_int8_backward.py:15, 52);
  - int8_linear_trainable(x, qdata, scale, bias, convrot, convrot_groupsize) and
    w4a8_linear_trainable(x, qdata, s_rel, s_channel, codebook, correction, bias, group_size,
    convrot_groupsize) (train/train_lora.py:187-188, 210, 221-223; tests/test_training_packed.py:22-36).
The wrappers' forward is the quantized linear; their backward gives the activation gradient
dx = dy W only (the codes, scales and bias are frozen: docs/upstream/comfy-kitchen-mps-followups.md:17).
"""
import torch

from . import _lib
from .exceptions import NoCapableBackendError
from .ops import (_FLOAT, _as_2d, _bits_of, _check_device, _disabled, _srel_desc, _workspace, int8_linear,
                  w4a8_int8_linear)


def _grad_out(dy2, lead, k, out_dtype, dy):
    dt = out_dtype or dy.dtype
    if dt not in _FLOAT:
        raise NoCapableBackendError("grad_input", {"hip": f"out_dtype {dt} unsupported"})
    return torch.empty((dy2.shape[0], k), dtype=dt, device=dy.device), lead + (k,)


def int8_linear_grad_input(dy, qdata, scale, convrot=False, convrot_groupsize=256, out_dtype=None):
    """dx = dy @ W with W = rotate(q * scale), the INT8 weight in the original basis."""
    op = "int8_linear_grad_input"
    _disabled(op)
    _check_device(op, dy, qdata, scale)
    if dy.dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"dy dtype {dy.dtype} unsupported"})
    n, k = qdata.shape
    dy2, lead = _as_2d(dy, n)
    dx, shape = _grad_out(dy2, lead, k, out_dtype, dy)
    if dy2.shape[0] == 0 or k == 0:
        return dx.reshape(shape)
    if n == 0:
        return dx.zero_().reshape(shape)
    s = scale.reshape(-1) if scale.numel() in (1, n) else scale
    g = int(convrot_groupsize) if convrot else 0
    ws = _workspace(_lib.OP_INT8_GRAD_INPUT, dy2.shape[0], n, k, 0, dy2)
    st = _lib.load().qlin_int8_linear_grad_input(_lib.desc(dy2), _lib.desc(qdata), _lib.desc(s), g, _lib.desc(dx),
                                                 ws.data_ptr(), ws.numel(), _lib.stream_of(dy.device))
    _lib.check(st, op)
    return dx.reshape(shape)


def w4a8_linear_grad_input(dy, qdata, s_rel, s_channel, codebook=None, correction=None, group_size=16,
                           convrot_groupsize=256, out_dtype=None):
    """dx = dy @ W with W = dequantize_w4a8_int8_weight(...), the weight in the original basis."""
    op = "w4a8_linear_grad_input"
    _disabled(op)
    if correction is not None:
        raise NoCapableBackendError(op, {"hip": "the asymmetric `correction` variant is not implemented"})
    _check_device(op, dy, qdata, s_rel, s_channel, codebook)
    if dy.dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"dy dtype {dy.dtype} unsupported"})
    bits, k = _bits_of(qdata, s_rel, group_size)
    n = qdata.shape[0]
    dy2, lead = _as_2d(dy, n)
    dx, shape = _grad_out(dy2, lead, k, out_dtype, dy)
    if dy2.shape[0] == 0 or k == 0:
        return dx.reshape(shape)
    if n == 0:
        return dx.zero_().reshape(shape)
    q = qdata if qdata.dtype in (torch.int8, torch.uint8) else qdata.view(torch.int8)
    cb = None if codebook is None else codebook.to(torch.float32).contiguous()
    sch = s_channel.reshape(-1).to(torch.float32).contiguous()
    ws = _workspace(_lib.OP_W4A8_GRAD_INPUT, dy2.shape[0], n, k, bits, dy2)
    st = _lib.load().qlin_w4a8_linear_grad_input(_lib.desc(dy2), _lib.desc(q), _srel_desc(s_rel), _lib.desc(sch),
                                                 _lib.desc(cb), _lib.desc(dx), bits, int(group_size),
                                                 int(convrot_groupsize or 0), ws.data_ptr(), ws.numel(),
                                                 _lib.stream_of(dy.device))
    _lib.check(st, op)
    return dx.reshape(shape)


class _Int8Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, qdata, scale, bias, convrot, convrot_groupsize):
        ctx.save_for_backward(qdata, scale)
        ctx.conf = (bool(convrot), int(convrot_groupsize), x.dtype)
        return int8_linear(x, qdata, scale, bias, convrot=convrot, convrot_groupsize=convrot_groupsize)

    @staticmethod
    def backward(ctx, dy):
        qdata, scale = ctx.saved_tensors
        convrot, g, x_dtype = ctx.conf
        dx = None
        if ctx.needs_input_grad[0]:
            dx = int8_linear_grad_input(dy.contiguous(), qdata, scale, convrot, g, out_dtype=x_dtype)
        return dx, None, None, None, None, None


class _W4A8Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, qdata, s_rel, s_channel, codebook, bias, group_size, convrot_groupsize):
        ctx.save_for_backward(qdata, s_rel, s_channel, codebook)
        ctx.conf = (int(group_size), int(convrot_groupsize), x.dtype)
        return w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, None, bias, group_size, convrot_groupsize)

    @staticmethod
    def backward(ctx, dy):
        qdata, s_rel, s_channel, codebook = ctx.saved_tensors
        gs, g, x_dtype = ctx.conf
        dx = None
        if ctx.needs_input_grad[0]:
            dx = w4a8_linear_grad_input(dy.contiguous(), qdata, s_rel, s_channel, codebook, None, gs, g,
                                        out_dtype=x_dtype)
        return dx, None, None, None, None, None, None, None


def int8_linear_trainable(x, qdata, scale, bias=None, convrot=False, convrot_groupsize=256):
    """int8_linear with an activation gradient (the weight, scale and bias stay frozen)."""
    return _Int8Linear.apply(x, qdata, scale, bias, convrot, convrot_groupsize)


def w4a8_linear_trainable(x, qdata, s_rel, s_channel, codebook=None, correction=None, bias=None, group_size=16,
                          convrot_groupsize=256):
    """w4a8_int8_linear with an activation gradient (the packed weight and bias stay frozen)."""
    if correction is not None:
        raise NoCapableBackendError("w4a8_linear_trainable", {"hip": "the asymmetric `correction` variant is not implemented"})
    return _W4A8Linear.apply(x, qdata, s_rel, s_channel, codebook, bias, group_size, convrot_groupsize)
