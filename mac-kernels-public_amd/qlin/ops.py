"""Packed-weight linear ops on MI355X, with comfy-kitchen's names, argument order and defaults.

Reference interface (roblennon/mac-kernels-public; the implementations live in un-vendored
comfy-kitchen forks, the call sites below pin the API):
  int8_linear       bench/bench_ck01_int8.py:57, bench/bench_lora_sidepath_kernel.py:77
  w4a8_int8_linear  bench/bench_w4a8_linear.py:82-83, bench/bench_lora_fused_rank.py:42-44
  gguf_linear       docs/research/2026-10-03-gguf-on-metal.md:85, bench/bench_gguf_linear.py:120
  dequantize_*      bench/bench_ck01_int8.py:49, tests/test_training_packed.py:25-26

Every op runs on the HIP library through the C ABI on the current torch stream and returns a new
tensor.  Inputs are read-only and packed weights are never copied.  A call the kernels do not
implement raises NoCapableBackendError (the reference registry's decline), never a silent
approximation.
"""
from __future__ import annotations

import os

import torch

from . import _lib
from .exceptions import NoCapableBackendError, QlinError
from .gguf import GGUF_TYPES, gguf_type_id

# The eager entry points of csrc/torch_ops.cpp (qlin/_qlin_torch.so): plain linears (no LoRA, no
# residual) go from Python to the C ABI in one C++ call.  Every other call, and every call when the
# module is not built, takes the ctypes route below; both run the same kernels through the same
# C ABI.
try:
    from . import _qlin_torch as _FAST
except ImportError:  # pragma: no cover - only when the module was not built
    _FAST = None
if _FAST is not None:
    _FAST.set_gguf_types({tid: (qk, ts) for tid, qk, ts in GGUF_TYPES.values()})
    _FastError = _FAST.QlinStatusError


def _fast_error(op, e):
    """The exception ops raise for a status the C++ entry point reported as "<status>:<message>"."""
    status, _, msg = str(e).partition(":")
    status = int(status)
    if status == _lib.QLIN_EUNSUPPORTED:
        return NoCapableBackendError(op, {"hip": msg})
    if status in (_lib.QLIN_EINVAL, _lib.QLIN_EWORKSPACE):
        return ValueError(f"{op}: {msg}")
    return QlinError(f"{op}: {msg}")

_FLOAT = (torch.float16, torch.bfloat16, torch.float32)

# os.environ keeps its encoded copy in a dict on POSIX; reading that is ~8x cheaper than
# os.environ.get and still sees every change made through os.environ.
_ENV_DATA = getattr(os.environ, "_data", None) if os.name == "posix" else None


def env_disabled() -> bool:
    """QLIN_DISABLE set to anything but "" or "0" (read at every call)."""
    if _ENV_DATA is not None:
        v = _ENV_DATA.get(b"QLIN_DISABLE")
        return v is not None and v not in (b"", b"0")
    return os.environ.get("QLIN_DISABLE", "0") not in ("", "0")


def _disabled(op):
    if env_disabled():
        raise NoCapableBackendError(op, {"hip": "disabled by QLIN_DISABLE"})


def _lora_args(op, lora_down, lora_up, lora_scale, n, k):
    """Validated (down [R, K], up [N, R], scale) or None.  lora_scale None means 1.0; a scale
    without both factors is rejected (the reference passes the three together)."""
    if lora_down is None and lora_up is None:
        if lora_scale is not None:
            raise ValueError(f"{op}: lora_scale given without lora_down / lora_up")
        return None
    if lora_down is None or lora_up is None:
        raise ValueError(f"{op}: lora_down and lora_up go together")
    if lora_down.dim() != 2 or lora_up.dim() != 2:
        raise ValueError(f"{op}: lora_down must be [R, K] and lora_up [N, R]")
    r = lora_down.shape[0]
    if lora_down.shape[1] != k or tuple(lora_up.shape) != (n, r):
        raise ValueError(f"{op}: lora_down {tuple(lora_down.shape)} / lora_up {tuple(lora_up.shape)} "
                         f"do not fit K={k}, N={n}")
    for t in (lora_down, lora_up):
        if t.dtype not in _FLOAT:
            raise NoCapableBackendError(op, {"hip": f"lora dtype {t.dtype} unsupported"})
    scale = 1.0 if lora_scale is None else float(lora_scale)
    return lora_down, lora_up, scale


def _base_out(lora, y, residual=None):
    """Where the base linear writes: y itself, or an fp32 buffer when a residual follows or LoRA
    meets a 16-bit y, so that the base, LoRA and residual terms are added in fp32 and rounded once
    into y (as the reference's single fp32 sum, docs/upstream/comfy-kitchen-mps-backend.md:52-56)."""
    if y.numel() == 0 or (residual is None and (lora is None or y.dtype == torch.float32)):
        return y
    return torch.empty(y.shape, dtype=torch.float32, device=y.device)


def _residual_args(op, residual, residual_scale, shape, n):
    """Validated residual [.., N] (flattened to [M, N]) and residual_scale [N] (or None)."""
    if residual is None:
        if residual_scale is not None:
            raise ValueError(f"{op}: residual_scale given without residual")
        return None
    if tuple(residual.shape) != tuple(shape):
        raise ValueError(f"{op}: residual has shape {tuple(residual.shape)}, the output is {tuple(shape)}")
    for t in (residual, residual_scale):
        if t is not None and t.dtype not in _FLOAT:
            raise NoCapableBackendError(op, {"hip": f"residual dtype {t.dtype} unsupported"})
    r = residual.reshape(-1, n)
    if r.shape[0] > 1 and (r.stride(1) != 1 or r.stride(0) < n):
        r = r.contiguous()
    rs = None
    if residual_scale is not None:
        if residual_scale.numel() != n:
            raise ValueError(f"{op}: residual_scale has {residual_scale.numel()} elements, expected {n}")
        rs = residual_scale.reshape(n).contiguous()
    return r, rs


def _finish(op, lora, res, x2, y, yb):
    """After the base linear wrote yb: the LoRA term, then the residual epilogue, into y."""
    if res is None:
        _apply_lora(op, lora, x2, y, yb)
        return
    _apply_lora(op, lora, x2, yb, yb)  # in place on the fp32 base
    r, rs = res
    _check_device(op, r, rs)
    st = _lib.load().qlin_residual_epilogue(_lib.desc(yb), _lib.desc(r), _lib.desc(rs), _lib.desc(y),
                                            _lib.stream_of(y.device))
    _lib.check(st, op)


def _lora_operands(op, lora):
    down, up, scale = lora
    _check_device(op, down, up)
    if down.stride(-1) != 1:
        down = down.contiguous()
    if up.stride(-1) != 1:
        up = up.contiguous()
    return down, up, scale


def _fused_lora(op, lora, res, x2, run):
    """Runs the linear with the LoRA term in its GEMM epilogue when no residual follows: `run(down, up,
    scale)` returns the entry point's status.  True when it ran; False when the entry point declined
    (QLIN_EUNSUPPORTED: the rows take a kernel without the fused term), and the caller runs the
    plain linear and the separate LoRA kernels."""
    if lora is None or res is not None:
        return False
    st = run(*_lora_operands(op, lora))
    if st == _lib.QLIN_EUNSUPPORTED:
        return False
    _lib.check(st, op)
    return True


def _apply_lora(op, lora, x2, y, base=None):
    """y = dtype(base + scale * (x2 @ down^T) @ up^T) on the GPU after the base linear; `base` is the
    fp32 buffer from _base_out, or y itself (updated in place)."""
    if lora is None or y.numel() == 0:
        return
    down, up, scale = _lora_operands(op, lora)
    r = down.shape[0]
    ws = _workspace(_lib.OP_LORA, x2.shape[0], up.shape[0], x2.shape[1], r, x2)
    L = _lib.load()
    if base is None or base is y:
        st = L.qlin_lora_apply(_lib.desc(x2), _lib.desc(down), _lib.desc(up), scale, _lib.desc(y), ws.data_ptr(),
                               ws.numel(), _lib.stream_of(x2.device))
    else:
        st = L.qlin_lora_apply_base(_lib.desc(x2), _lib.desc(down), _lib.desc(up), scale, _lib.desc(base),
                                    _lib.desc(y), ws.data_ptr(), ws.numel(), _lib.stream_of(x2.device))
    _lib.check(st, op)


def _check_device(op, *tensors):
    dev = -1
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise NoCapableBackendError(op, {"hip": f"tensor on {t.device}, the kernels need a ROCm device"})
        d = t.get_device()
        if dev < 0:
            dev = d
        elif d != dev:
            raise ValueError(f"{op}: tensors on different devices (cuda:{dev}, cuda:{d})")


def _as_2d(x: torch.Tensor, k: int):
    sh = x.shape
    if sh[-1] != k:
        raise ValueError(f"x has {sh[-1]} input features, the weight has {k}")
    lead = tuple(sh[:-1])
    x2 = x if len(sh) == 2 else x.reshape(-1, k)
    if x2.shape[0] > 1 and x2.stride(1) != 1:
        x2 = x2.contiguous()
    if x2.shape[0] > 1 and x2.stride(0) < k:
        x2 = x2.contiguous()
    if x2.data_ptr() % 16:  # storage offset that breaks 128-bit loads: take an aligned copy
        x2 = x2.clone(memory_format=torch.contiguous_format)
    return x2, lead


def _out(x2, lead, n, out_dtype, x):
    dt = out_dtype or x.dtype
    if dt not in _FLOAT:
        raise NoCapableBackendError("linear", {"hip": f"out_dtype {dt} unsupported"})
    y = torch.empty((x2.shape[0], n), dtype=dt, device=x.device)
    return y, lead + (n,)


_WS_SIZES: dict = {}


def _workspace(op, m, n, k, param, x2, stream=None):
    """The per-stream workspace for one call (sizes cached per shape; the C ABI computes them).  With
    the C++ module the buffer comes from its cache, which its own calls use too (the current stream
    of x2's device is the stream every op here runs on)."""
    key = (op, m, n, k, param, x2.dtype)
    nbytes = _WS_SIZES.get(key)
    if nbytes is None:
        if len(_WS_SIZES) > 4096:
            _WS_SIZES.clear()
        nbytes = _WS_SIZES[key] = _lib.load().qlin_workspace_size(op, m, n, k, param, _lib._TORCH_DT[x2.dtype])
    if _FAST is not None:
        return _FAST.workspace(nbytes, x2)
    return _lib.workspace(nbytes, x2.device, _lib.stream_of(x2.device) if stream is None else stream)


def _shaped(y, shape):
    return y if len(shape) == 2 else y.reshape(shape)


def _f32_1d(t):
    """t flattened to a contiguous fp32 vector (t itself when it already is one)."""
    if t.dim() == 1 and t.dtype == torch.float32 and t.is_contiguous():
        return t
    return t.reshape(-1).to(torch.float32).contiguous()


def _bias(bias, n):
    if bias is None:
        return None
    if bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} elements, expected {n}")
    return bias if bias.dim() == 1 and bias.is_contiguous() else bias.reshape(n).contiguous()


# ------------------------------------------------------------------------------------------------
# INT8 (+ ConvRot) weight-only
# ------------------------------------------------------------------------------------------------

def int8_linear(x, qdata, scale, bias=None, out_dtype=None, *, convrot=False, convrot_groupsize=256,
                lora_down=None, lora_up=None, lora_scale=None, residual=None, residual_scale=None):
    """y = rot(x) @ (qdata * scale)^T + bias.  qdata int8 [N, K] (rotated basis when convrot),
    scale [N] / [N, 1] / scalar (fp32 or fp16).  fp16 MFMA, fp32 accumulate.  With `residual`
    ([.., N]): y = residual + residual_scale * (linear + bias + LoRA), one rounding."""
    op = "int8_linear"
    _disabled(op)
    if _FAST is not None and lora_down is None and lora_up is None and lora_scale is None and residual is None \
            and residual_scale is None:
        try:
            return _FAST.int8_linear(x, qdata, scale, bias, out_dtype, int(convrot_groupsize) if convrot else 0)
        except _FastError as e:
            raise _fast_error(op, e) from None
    _check_device(op, x, qdata, scale, bias)
    if qdata.dtype != torch.int8 or qdata.dim() != 2:
        raise NoCapableBackendError(op, {"hip": "qdata must be a 2-D int8 tensor"})
    if x.dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"x dtype {x.dtype} unsupported"})
    n, k = qdata.shape
    lora = _lora_args(op, lora_down, lora_up, lora_scale, n, k)
    x2, lead = _as_2d(x, k)
    y, shape = _out(x2, lead, n, out_dtype, x)
    res = _residual_args(op, residual, residual_scale, shape, n)
    if x2.shape[0] == 0 or n == 0:
        return y.reshape(shape)
    g = int(convrot_groupsize) if convrot else 0
    s = scale if scale.dim() == 1 or scale.numel() not in (1, n) else scale.reshape(-1)
    b = _bias(bias, n)
    L = _lib.load()
    m = x2.shape[0]
    stream = _lib.stream_of(x.device)
    if m > 16 and lora is not None:
        def run(down, up, lscale):
            wsl = _workspace(_lib.OP_INT8_LINEAR_LORA, m, n, k, down.shape[0], x2, stream)
            return L.qlin_int8_linear_lora(_lib.desc(x2), _lib.desc(qdata), _lib.desc(s), _lib.desc(b), _lib.desc(y), g,
                                           _lib.desc(down), _lib.desc(up), lscale, wsl.data_ptr(), wsl.numel(), stream)
        if _fused_lora(op, lora, res, x2, run):
            return _shaped(y, shape)
    if res is not None and lora is None:  # the residual joins the linear's epilogue (or its own kernel)
        r, rs = res
        _check_device(op, r, rs)
        ws = _workspace(_lib.OP_INT8_LINEAR_RESIDUAL, m, n, k, g, x2, stream)
        st = L.qlin_int8_linear_residual(_lib.desc(x2), _lib.desc(qdata), _lib.desc(s), _lib.desc(b), _lib.desc(r),
                                         _lib.desc(rs), _lib.desc(y), g, ws.data_ptr(), ws.numel(), stream)
        _lib.check(st, op)
        return _shaped(y, shape)
    ws = _workspace(_lib.OP_INT8_LINEAR, m, n, k, g, x2, stream)
    yb = _base_out(lora, y, res)
    st = L.qlin_int8_linear(_lib.desc(x2), _lib.desc(qdata), _lib.desc(s), _lib.desc(b), _lib.desc(yb), g,
                            ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, op)
    _finish(op, lora, res, x2, y, yb)
    return _shaped(y, shape)


def dequantize_int8(qdata, scale):
    """float32 q * scale[n] (the rotated basis for ConvRot weights), bit-exact."""
    return dequantize_int8_convrot_weight(qdata, scale, 0)


def dequantize_int8_convrot_weight(qdata, scale, convrot_groupsize=256):
    """Original-basis float32 weight rotate(q * scale) (0 = no rotation)."""
    op = "dequantize_int8"
    _check_device(op, qdata, scale)
    n, k = qdata.shape
    out = torch.empty((n, k), dtype=torch.float32, device=qdata.device)
    s = scale.reshape(-1) if scale.numel() in (1, n) else scale
    st = _lib.load().qlin_dequantize_int8(_lib.desc(qdata), _lib.desc(s), _lib.desc(out), int(convrot_groupsize),
                                          _lib.stream_of(qdata.device))
    _lib.check(st, op)
    return out


# ------------------------------------------------------------------------------------------------
# W4A8 / W6A8 (AsymW4A8Int8 storage), A8 int8 GEMM
# ------------------------------------------------------------------------------------------------

def _srel_desc(s_rel):
    if s_rel.dtype == torch.float8_e4m3fn:
        return _lib.desc(s_rel.view(torch.uint8), _lib.DT_E4M3)
    if s_rel.dtype in (torch.float16, torch.bfloat16, torch.float32):
        return _lib.desc(s_rel)
    raise NoCapableBackendError("w4a8_int8_linear", {"hip": f"s_rel dtype {s_rel.dtype} unsupported"})


def _bits_of(qdata, s_rel, group_size):
    k = s_rel.shape[1] * group_size
    bits = (qdata.shape[1] * 8) // k
    if bits not in (4, 6) or qdata.shape[1] * 8 != bits * k:
        raise ValueError(f"qdata [{qdata.shape[0]}, {qdata.shape[1]}] does not hold 4- or 6-bit codes for K={k}")
    return bits, k


def w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook=None, correction=None, bias=None, group_size=16,
                     convrot_groupsize=256, out_dtype=None, *, lora_down=None, lora_up=None, lora_scale=None,
                     residual=None, residual_scale=None):
    """A8 linear: per-token int8 activations (quantize_int8_rowwise of the rotated x), int8 MFMA
    against the int8 weight grid, y = acc * sx[m] * s_channel[n] + bias (then LoRA and residual as
    for int8_linear)."""
    op = "w4a8_int8_linear"
    _disabled(op)
    if correction is not None:
        raise NoCapableBackendError(op, {"hip": "the asymmetric `correction` variant is not implemented"})
    if _FAST is not None and lora_down is None and lora_up is None and lora_scale is None and residual is None \
            and residual_scale is None:
        try:
            return _FAST.w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, bias, int(group_size),
                                          int(convrot_groupsize or 0), out_dtype)
        except _FastError as e:
            raise _fast_error(op, e) from None
    _check_device(op, x, qdata, s_rel, s_channel, codebook, bias)
    if x.dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"x dtype {x.dtype} unsupported"})
    bits, k = _bits_of(qdata, s_rel, group_size)
    n = qdata.shape[0]
    lora = _lora_args(op, lora_down, lora_up, lora_scale, n, k)
    x2, lead = _as_2d(x, k)
    y, shape = _out(x2, lead, n, out_dtype, x)
    res = _residual_args(op, residual, residual_scale, shape, n)
    if x2.shape[0] == 0 or n == 0:
        return _shaped(y, shape)
    q = qdata if qdata.dtype in (torch.int8, torch.uint8) else qdata.view(torch.int8)
    cb = None if codebook is None else _f32_1d(codebook)
    sch = _f32_1d(s_channel)
    b = _bias(bias, n)
    L = _lib.load()
    m = x2.shape[0]
    stream = _lib.stream_of(x.device)
    # above the small-M kernel's 32 rows the C ABI fuses the term where it decodes the weight grid
    # once, and declines elsewhere
    if m > 32 and lora is not None:
        def run(down, up, lscale):
            wsl = _workspace(_lib.OP_W4A8_LINEAR_LORA, m, n, k, down.shape[0] | int(group_size) << 16, x2, stream)
            return L.qlin_w4a8_linear_lora(_lib.desc(x2), _lib.desc(q), _srel_desc(s_rel), _lib.desc(sch), _lib.desc(cb),
                                           _lib.desc(b), _lib.desc(y), bits, int(group_size), int(convrot_groupsize or 0),
                                           _lib.desc(down), _lib.desc(up), lscale, wsl.data_ptr(), wsl.numel(), stream)
        if _fused_lora(op, lora, res, x2, run):
            return _shaped(y, shape)
    if res is not None and lora is None:  # the residual joins the linear's epilogue (or its own kernel)
        r, rs = res
        _check_device(op, r, rs)
        ws = _workspace(_lib.OP_W4A8_LINEAR_RESIDUAL, m, n, k, bits | int(group_size) << 8, x2, stream)
        st = L.qlin_w4a8_linear_residual(_lib.desc(x2), _lib.desc(q), _srel_desc(s_rel), _lib.desc(sch), _lib.desc(cb),
                                         _lib.desc(b), _lib.desc(r), _lib.desc(rs), _lib.desc(y), bits, int(group_size),
                                         int(convrot_groupsize or 0), ws.data_ptr(), ws.numel(), stream)
        _lib.check(st, op)
        return _shaped(y, shape)
    ws = _workspace(_lib.OP_W4A8_LINEAR, m, n, k, bits | int(group_size) << 8, x2, stream)
    yb = _base_out(lora, y, res)
    st = L.qlin_w4a8_linear(_lib.desc(x2), _lib.desc(q), _srel_desc(s_rel), _lib.desc(sch), _lib.desc(cb),
                            _lib.desc(b), _lib.desc(yb), bits, int(group_size), int(convrot_groupsize or 0),
                            ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, op)
    _finish(op, lora, res, x2, y, yb)
    return _shaped(y, shape)


def dequantize_w4a8_int8_weight(qdata, s_rel, s_channel, codebook=None, correction=None, group_size=16,
                                convrot_groupsize=256, output_dtype=torch.float32):
    """Packed storage -> weight in the original basis (rotated back per ConvRot group)."""
    op = "dequantize_w4a8_int8_weight"
    if correction is not None:
        raise NoCapableBackendError(op, {"hip": "the asymmetric `correction` variant is not implemented"})
    _check_device(op, qdata, s_rel, s_channel, codebook)
    bits, k = _bits_of(qdata, s_rel, group_size)
    n = qdata.shape[0]
    out = torch.empty((n, k), dtype=torch.float32, device=qdata.device)
    cb = None if codebook is None else codebook.to(torch.float32).contiguous()
    sch = s_channel.reshape(-1).to(torch.float32).contiguous()
    st = _lib.load().qlin_dequantize_w4a8(_lib.desc(qdata), _srel_desc(s_rel), _lib.desc(sch), _lib.desc(cb),
                                          _lib.desc(out), bits, int(group_size), int(convrot_groupsize or 0),
                                          _lib.stream_of(qdata.device))
    _lib.check(st, op)
    return out if output_dtype == torch.float32 else out.to(output_dtype)


def w4a8_int8_grid(qdata, s_rel, codebook=None, group_size=16):
    """The int8 weight grid w8 [N, K] the A8 GEMM multiplies (bit-exact decode)."""
    op = "w4a8_int8_grid"
    _check_device(op, qdata, s_rel, codebook)
    bits, k = _bits_of(qdata, s_rel, group_size)
    n = qdata.shape[0]
    out = torch.empty((n, k), dtype=torch.int8, device=qdata.device)
    cb = None if codebook is None else codebook.to(torch.float32).contiguous()
    ones = torch.ones(n, dtype=torch.float32, device=qdata.device)
    st = _lib.load().qlin_dequantize_w4a8(_lib.desc(qdata), _srel_desc(s_rel), _lib.desc(ones), _lib.desc(cb),
                                          _lib.desc(out), bits, int(group_size), 0, _lib.stream_of(qdata.device))
    _lib.check(st, op)
    return out


def quantize_int8_rowwise(x, convrot_groupsize=0, return_rotated=False):
    """Per-token A8 quantization on the GPU: (q int8 [M, K], scale fp32 [M, 1]) of rot(x),
    with the reference's arithmetic in x's dtype."""
    op = "quantize_int8_rowwise"
    _check_device(op, x)
    k = x.shape[-1]
    x2, lead = _as_2d(x, k)
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    xr = torch.empty((m, k), dtype=x.dtype, device=x.device) if return_rotated else None
    if m:
        st = _lib.load().qlin_quantize_act_int8(_lib.desc(x2), _lib.desc(q), _lib.desc(s), int(convrot_groupsize),
                                                _lib.desc(xr), _lib.stream_of(x.device))
        _lib.check(st, op)
    q = q.reshape(lead + (k,))
    s = s.reshape(lead + (1,))
    if return_rotated:
        return q, s, xr.reshape(lead + (k,))
    return q, s


# ------------------------------------------------------------------------------------------------
# GGUF
# ------------------------------------------------------------------------------------------------

def gguf_linear(x, weight, qtype, shape, bias=None, out_dtype=None, lora_down=None, lora_up=None, lora_scale=None,
                *, residual=None, residual_scale=None):
    """y = x @ W^T + bias with W [N, K] decoded from GGUF blocks of `qtype` (ggml type id or name).
    `weight` is the tensor's raw bytes (uint8, [N, K/qk*ts] or flat).  LoRA and residual as for
    int8_linear."""
    op = "gguf_linear"
    _disabled(op)
    tid = gguf_type_id(qtype)
    n, k = int(shape[0]), int(shape[1])
    if _FAST is not None and lora_down is None and lora_up is None and lora_scale is None and residual is None \
            and residual_scale is None:
        try:
            return _FAST.gguf_linear(x, weight, tid, n, k, bias, out_dtype)
        except _FastError as e:
            raise _fast_error(op, e) from None
    _check_device(op, x, weight, bias)
    lora = _lora_args(op, lora_down, lora_up, lora_scale, n, k)
    if weight.dtype != torch.uint8:
        raise NoCapableBackendError(op, {"hip": "weight must be the uint8 block bytes"})
    if not weight.is_contiguous():
        raise NoCapableBackendError(op, {"hip": "weight bytes must be contiguous"})
    _, qk, ts = GGUF_TYPES_BY_ID[tid]
    if weight.numel() != n * k // qk * ts:
        raise ValueError(f"weight has {weight.numel()} bytes, expected {n * k // qk * ts} for {shape}")
    if x.dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"x dtype {x.dtype} unsupported"})
    x2, lead = _as_2d(x, k)
    y, oshape = _out(x2, lead, n, out_dtype, x)
    res = _residual_args(op, residual, residual_scale, oshape, n)
    if x2.shape[0] == 0 or n == 0:
        return _shaped(y, oshape)
    b = _bias(bias, n)
    stream = _lib.stream_of(x.device)
    m = x2.shape[0]
    if m > 16 and lora is not None:
        def run(down, up, lscale):
            wsl = _workspace(_lib.OP_GGUF_LINEAR_LORA, m, n, k, tid | down.shape[0] << 8, x2, stream)
            return _lib.load().qlin_gguf_linear_lora(_lib.desc(x2), weight.data_ptr(), tid, n, k, _lib.desc(b),
                                                     _lib.desc(y), _lib.desc(down), _lib.desc(up), lscale,
                                                     wsl.data_ptr(), wsl.numel(), stream)
        if _fused_lora(op, lora, res, x2, run):
            return _shaped(y, oshape)
    if res is not None and lora is None:  # the residual joins the linear's epilogue (or its own kernel)
        r, rs = res
        _check_device(op, r, rs)
        ws = _workspace(_lib.OP_GGUF_LINEAR_RESIDUAL, x2.shape[0], n, k, tid, x2, stream)
        st = _lib.load().qlin_gguf_linear_residual(_lib.desc(x2), weight.data_ptr(), tid, n, k, _lib.desc(b), _lib.desc(r),
                                                   _lib.desc(rs), _lib.desc(y), ws.data_ptr(), ws.numel(), stream)
        _lib.check(st, op)
        return _shaped(y, oshape)
    ws = _workspace(_lib.OP_GGUF_LINEAR, x2.shape[0], n, k, tid, x2, stream)
    yb = _base_out(lora, y, res)
    st = _lib.load().qlin_gguf_linear(_lib.desc(x2), weight.data_ptr(), tid, n, k, _lib.desc(b), _lib.desc(yb),
                                      ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, op)
    _finish(op, lora, res, x2, y, yb)
    return _shaped(y, oshape)


def dequantize_gguf(weight, qtype, shape, out_dtype=torch.float32):
    """Decode GGUF block bytes to a dense [N, K] tensor; float32 is bit-exact with gguf-py."""
    op = "dequantize_gguf"
    tid = gguf_type_id(qtype)
    n, k = int(shape[0]), int(shape[1])
    _, qk, ts = GGUF_TYPES_BY_ID[tid]
    # the kernel decodes N*K/qk whole blocks from a raw pointer: check the buffer before any launch
    if weight.dtype != torch.uint8:
        raise NoCapableBackendError(op, {"hip": "weight must be the uint8 block bytes"})
    if not weight.is_contiguous():
        raise NoCapableBackendError(op, {"hip": "weight bytes must be contiguous"})
    if n < 0 or k < 0 or (n * k) % qk:
        raise ValueError(f"{op}: shape {tuple(shape)} is not a whole number of {qk}-value blocks")
    if weight.numel() != n * k // qk * ts:
        raise ValueError(f"weight has {weight.numel()} bytes, expected {n * k // qk * ts} for {tuple(shape)}")
    if out_dtype not in _FLOAT:
        raise NoCapableBackendError(op, {"hip": f"out_dtype {out_dtype} unsupported"})
    _check_device(op, weight)
    out = torch.empty((n, k), dtype=out_dtype, device=weight.device)
    if out.numel() == 0:
        return out
    st = _lib.load().qlin_dequantize_gguf(weight.data_ptr(), tid, n, k, _lib.desc(out), _lib.stream_of(weight.device))
    _lib.check(st, op)
    return out


GGUF_TYPES_BY_ID = {v[0]: (name, v[1], v[2]) for name, v in GGUF_TYPES.items()}
