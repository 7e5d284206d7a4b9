"""ctypes binding of libqlin.so (include/qlin.h).

The library is built in-tree by ``mac-kernels-public_amd/build_lib.py``.  Loading fails loudly
when it is missing: there is no CPU or eager fallback in this package.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading

import torch

from .exceptions import NoCapableBackendError, QlinError

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqlin.so")

QLIN_OK, QLIN_EUNSUPPORTED, QLIN_EINVAL, QLIN_EHIP, QLIN_EWORKSPACE = 0, 1, 2, 3, 4
DT_F32, DT_F16, DT_BF16, DT_I8, DT_U8, DT_I32, DT_E4M3 = 0, 1, 2, 3, 4, 5, 6
OP_INT8_LINEAR, OP_W4A8_LINEAR, OP_GGUF_LINEAR, OP_LORA, OP_INT8_GRAD_INPUT, OP_W4A8_GRAD_INPUT = 0, 1, 2, 3, 4, 5
OP_INT8_LINEAR_LORA, OP_W4A8_LINEAR_LORA = 6, 7
OP_INT8_LINEAR_RESIDUAL, OP_W4A8_LINEAR_RESIDUAL, OP_GGUF_LINEAR_RESIDUAL = 8, 9, 10
OP_GGUF_LINEAR_LORA = 11

_TORCH_DT = {
    torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.int8: DT_I8,
    torch.uint8: DT_U8, torch.int32: DT_I32, torch.float8_e4m3fn: DT_E4M3,
}

# Every symbol include/qlin.h declares.
EXPORTS = (
    "qlin_version", "qlin_status_string", "qlin_last_error", "qlin_workspace_size", "qlin_query",
    "qlin_int8_linear", "qlin_w4a8_linear", "qlin_gguf_linear", "qlin_gguf_linear_noalloc", "qlin_dequantize_gguf",
    "qlin_dequantize_int8", "qlin_dequantize_w4a8", "qlin_quantize_act_int8", "qlin_lora_apply", "qlin_lora_apply_base",
    "qlin_residual_epilogue", "qlin_int8_linear_lora", "qlin_w4a8_linear_lora",
    "qlin_int8_linear_grad_input", "qlin_w4a8_linear_grad_input",
    "qlin_int8_linear_residual", "qlin_w4a8_linear_residual", "qlin_gguf_linear_residual",
    "qlin_gguf_linear_lora",
)


class QlinTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


_lib = None


def load():
    """Load libqlin.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise QlinError(f"{LIB_PATH} is missing: build it with mac-kernels-public_amd/build_lib.py "
                        "(the HIP library is the only implementation; there is no fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    T = ctypes.c_void_p  # the address of a qlin_tensor (see desc)
    sigs = {
        "qlin_version": (I, []),
        "qlin_status_string": (ctypes.c_char_p, [I]),
        "qlin_last_error": (ctypes.c_char_p, []),
        "qlin_workspace_size": (SZ, [I, I64, I64, I64, I, I]),
        "qlin_query": (I, [I, I64, I64, I64, I, I, I]),
        "qlin_int8_linear": (I, [T, T, T, T, T, I, P, SZ, P]),
        "qlin_w4a8_linear": (I, [T, T, T, T, T, T, T, I, I, I, P, SZ, P]),
        "qlin_int8_linear_lora": (I, [T, T, T, T, T, I, T, T, ctypes.c_float, P, SZ, P]),
        "qlin_w4a8_linear_lora": (I, [T, T, T, T, T, T, T, I, I, I, T, T, ctypes.c_float, P, SZ, P]),
        "qlin_gguf_linear": (I, [T, P, I, I64, I64, T, T, P, SZ, P]),
        "qlin_gguf_linear_lora": (I, [T, P, I, I64, I64, T, T, T, T, ctypes.c_float, P, SZ, P]),
        "qlin_int8_linear_residual": (I, [T, T, T, T, T, T, T, I, P, SZ, P]),
        "qlin_w4a8_linear_residual": (I, [T, T, T, T, T, T, T, T, T, I, I, I, P, SZ, P]),
        "qlin_gguf_linear_residual": (I, [T, P, I, I64, I64, T, T, T, T, P, SZ, P]),
        "qlin_gguf_linear_noalloc": (I, [T, P, I, I64, I64, T, T, P]),
        "qlin_dequantize_gguf": (I, [P, I, I64, I64, T, P]),
        "qlin_dequantize_int8": (I, [T, T, T, I, P]),
        "qlin_dequantize_w4a8": (I, [T, T, T, T, T, I, I, I, P]),
        "qlin_quantize_act_int8": (I, [T, T, T, I, T, P]),
        "qlin_lora_apply": (I, [T, T, T, ctypes.c_float, T, P, SZ, P]),
        "qlin_lora_apply_base": (I, [T, T, T, ctypes.c_float, T, T, P, SZ, P]),
        "qlin_residual_epilogue": (I, [T, T, T, T, P]),
        "qlin_int8_linear_grad_input": (I, [T, T, T, I, T, P, SZ, P]),
        "qlin_w4a8_linear_grad_input": (I, [T, T, T, T, T, T, I, I, I, P, SZ, P]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


# qlin_tensor {void* data; int32 dtype; int32 ndim; int64 shape[4]; int64 stride[4]}: 80 bytes.
_DESC = struct.Struct("=Qii8q")
assert _DESC.size == ctypes.sizeof(QlinTensor)
_DESC_SLOTS = 32
_PACK = _DESC.pack_into
_tls = threading.local()


def desc(t: torch.Tensor | None, dtype_override: int | None = None):
    """Address of a qlin_tensor descriptor of a torch tensor (None -> NULL).  Descriptors are
    packed into a per-thread ring of 32 slots, so one is valid until 32 more have been made on the
    same thread: build them right before the call that reads them."""
    if t is None:
        return None
    try:
        ring = _tls.ring
    except AttributeError:
        buf = ctypes.create_string_buffer(_DESC.size * _DESC_SLOTS)
        ring = _tls.ring = [buf, ctypes.addressof(buf), 0]
    i = ring[2]
    ring[2] = (i + 1) % _DESC_SLOTS
    dt = _TORCH_DT[t.dtype] if dtype_override is None else dtype_override
    sh = t.shape
    nd = len(sh)
    off = _DESC.size * i
    if nd == 2:
        st = t.stride()
        _PACK(ring[0], off, t.data_ptr(), dt, 2, sh[0], sh[1], 0, 0, st[0], st[1], 0, 0)
    elif nd == 1:
        _PACK(ring[0], off, t.data_ptr(), dt, 1, sh[0], 0, 0, 0, t.stride(0), 0, 0, 0)
    elif nd == 0:
        _PACK(ring[0], off, t.data_ptr(), dt, 1, 1, 0, 0, 0, 1, 0, 0, 0)
    elif nd <= 4:
        st = t.stride()
        pad = (0,) * (4 - nd)
        _PACK(ring[0], off, t.data_ptr(), dt, nd, *sh, *pad, *st, *pad)
    else:
        raise ValueError("at most 4 dims")
    return ring[1] + off


def stream_of(device: torch.device) -> int:
    """The raw handle of the current stream of `device`."""
    idx = device.index
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


_ws_cache: dict = {}


def workspace(nbytes: int, device: torch.device, stream: int) -> torch.Tensor:
    """A device byte buffer of at least `nbytes` for one call on `stream`.  Outside graph capture
    one buffer per (device, stream) is kept and grown, so eager calls do not allocate: calls on one
    stream run in order, so they can share it.  During capture every call gets its own tensor from
    the graph's pool."""
    nbytes = max(int(nbytes), 1)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, stream)
    w = _ws_cache.get(key)
    if w is None or w.numel() < nbytes:
        w = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws_cache[key] = w
    return w


def release_workspaces() -> None:
    """Drop the cached per-stream workspaces (their memory returns to torch's allocator)."""
    _ws_cache.clear()
    try:
        from . import _qlin_torch
    except ImportError:  # pragma: no cover
        return
    _qlin_torch.release_workspaces()


def check(status: int, op: str):
    if status == QLIN_OK:
        return
    msg = load().qlin_last_error().decode(errors="replace")
    if status == QLIN_EUNSUPPORTED:
        raise NoCapableBackendError(op, {"hip": msg})
    if status in (QLIN_EINVAL, QLIN_EWORKSPACE):
        raise ValueError(f"{op}: {msg}")
    raise QlinError(f"{op}: {msg}")
