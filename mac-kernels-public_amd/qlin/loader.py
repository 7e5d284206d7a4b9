"""Packed weights from disk to HBM, unchanged.

Two on-disk formats carry this path's weights:
  - safetensors as ComfyUI stores quantized linears (roblennon/mac-kernels-public
    tests/test_mps_pread_load.py:24-28, tests/test_h3_scale_ownership.py:24-29,
    bench/wan_int8_convert.py:57-77): per layer `weight` (I8 codes or packed W4/W6 bytes),
    `weight_scale` (INT8) or `weight_s_rel` / `weight_s_channel` / `weight_codebook` (W4A8, W6A8),
    and `comfy_quant`, a U8 tensor holding the layer's JSON config;
  - GGUF (header layout as read by bench/gguf_headers.py:80-110): ggml blocks stored as they are
    decoded by the kernels, with `comfy.gguf.orig_shape.<name>` giving the torch shape of tensors
    whose rows straddle blocks (docs/research/2026-10-03-gguf-on-metal.md:38).

Every tensor's bytes go from the file to device memory without decoding or repacking: the file
is read with pread into two pinned host buffers in turn, and each filled buffer is copied to the
device asynchronously while the next one is read.  `comfy_quant` config tensors stay on the host,
where the layer builder reads them (tests/test_mps_pread_load.py:21, :36).  The file is only read.
"""
from __future__ import annotations

import json
import math
import os
import struct
from dataclasses import dataclass, field

import torch

from .exceptions import NoCapableBackendError
from .gguf import GGUF_NAMES, GGUF_TYPES

CHUNK = 32 << 20  # bytes per pinned staging buffer (two are used)

# safetensors dtype names (the format's header strings) -> torch dtypes
ST_DTYPES = {
    "BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "I16": torch.int16, "I32": torch.int32,
    "I64": torch.int64, "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32,
    "F64": torch.float64, "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2,
}
ST_HEADER_MAX = 100 << 20


# --------------------------------------------------------------------------- byte transfer

class _Reader:
    """pread-based copies of file byte ranges into tensors; device destinations go through two
    pinned buffers so that reading one chunk overlaps the host-to-device copy of the other."""

    def __init__(self, path, chunk=CHUNK):
        self.fd = os.open(path, os.O_RDONLY)
        self.size = os.fstat(self.fd).st_size
        self.chunk = int(chunk)
        self.bufs = None
        self.events = [None, None]
        self.turn = 0

    def close(self):
        if self.bufs is not None:
            for ev in self.events:
                if ev is not None:
                    ev.synchronize()
        os.close(self.fd)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _pread_into(self, mv, offset):
        done = 0
        while done < len(mv):
            got = os.preadv(self.fd, [mv[done:]], offset + done)
            if got <= 0:
                raise ValueError(f"unexpected end of file at byte {offset + done}")
            done += got

    def pread(self, offset, n) -> bytes:
        if offset < 0 or offset + n > self.size:
            raise ValueError(f"byte range [{offset}, {offset + n}) is outside the file ({self.size} bytes)")
        out = bytearray(n)
        self._pread_into(memoryview(out), offset)
        return bytes(out)

    def into(self, dst: torch.Tensor, offset: int):
        """Fill the contiguous tensor `dst` with the file bytes at `offset`."""
        n = dst.numel() * dst.element_size()
        if offset < 0 or offset + n > self.size:
            raise ValueError(f"byte range [{offset}, {offset + n}) is outside the file ({self.size} bytes)")
        if n == 0:
            return
        flat = dst.view(-1).view(torch.uint8)
        if dst.device.type == "cpu":
            self._pread_into(memoryview(flat.numpy()), offset)
            return
        if self.bufs is None:
            size = min(self.chunk, max(n, 1 << 20))
            self.bufs = [torch.empty(size, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
            self.views = [memoryview(b.numpy()) for b in self.bufs]
        stream = torch.cuda.current_stream(dst.device)
        pos = 0
        size = self.bufs[0].numel()
        while pos < n:
            i = self.turn
            self.turn ^= 1
            if self.events[i] is not None:
                self.events[i].synchronize()  # the buffer's previous copy has left it
            m = min(size, n - pos)
            self._pread_into(self.views[i][:m], offset + pos)
            flat[pos:pos + m].copy_(self.bufs[i][:m], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
            self.events[i] = ev
            pos += m


def _device(device):
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


# --------------------------------------------------------------------------- safetensors

def safetensors_header(path):
    """(tensor entries {name: {"dtype", "shape", "data_offsets"}}, metadata dict, data start byte).

    Layout: an 8-byte little-endian header length, the JSON header, then the data; offsets are
    relative to the data start.  Entries are checked: known dtype, in-bounds and consistent
    offsets, no overlaps."""
    with _Reader(path) as r:
        if r.size < 8:
            raise ValueError(f"{path}: not a safetensors file (too short)")
        (hlen,) = struct.unpack("<Q", r.pread(0, 8))
        if hlen > ST_HEADER_MAX or 8 + hlen > r.size:
            raise ValueError(f"{path}: header length {hlen} is invalid")
        header = json.loads(r.pread(8, hlen).decode("utf-8"))
        size = r.size
    if not isinstance(header, dict):
        raise ValueError(f"{path}: header is not a JSON object")
    meta = header.pop("__metadata__", None) or {}
    start = 8 + hlen
    spans = []
    for name, e in header.items():
        dt, shape, (a, b) = e.get("dtype"), e.get("shape"), e.get("data_offsets", (None, None))
        if dt not in ST_DTYPES:
            raise ValueError(f"{path}: tensor {name} has unsupported dtype {dt}")
        nbytes = math.prod(shape) * torch.empty((), dtype=ST_DTYPES[dt]).element_size()
        if not (isinstance(a, int) and isinstance(b, int)) or b - a != nbytes or a < 0 or start + b > size:
            raise ValueError(f"{path}: tensor {name} has data_offsets {a, b} for {nbytes} bytes")
        spans.append((a, b, name))
    spans.sort()
    for (a0, b0, n0), (a1, b1, n1) in zip(spans, spans[1:]):
        if a1 < b0:
            raise ValueError(f"{path}: tensors {n0} and {n1} overlap")
    return header, meta, start


def load_safetensors(path, device="cuda", return_metadata=False, keys=None, chunk=CHUNK):
    """{name: tensor} with every tensor's bytes copied unchanged to `device` (`comfy_quant` config
    tensors stay on the host).  Mirrors comfy.utils.load_torch_file(path, device,
    return_metadata) for safetensors files (tests/test_mps_pread_load.py:36-43)."""
    header, meta, start = safetensors_header(path)
    dev = _device(device)
    want = set(header) if keys is None else set(keys)
    missing = want - set(header)
    if missing:
        raise KeyError(f"{path}: no tensors {sorted(missing)}")
    out = {}
    with _Reader(path, chunk) as r:
        # file order, so the reads are sequential
        for name, e in sorted(header.items(), key=lambda kv: kv[1]["data_offsets"][0]):
            if name not in want:
                continue
            on = torch.device("cpu") if name.endswith("comfy_quant") else dev
            t = torch.empty(e["shape"], dtype=ST_DTYPES[e["dtype"]], device=on)
            r.into(t, start + e["data_offsets"][0])
            out[name] = t
    return (out, meta) if return_metadata else out


# --------------------------------------------------------------------------- packed linear layers

@dataclass
class PackedLinear:
    """One quantized linear layer as stored: `kind` is "int8", "w4a8" (4- or 6-bit) or "gguf";
    `tensors` are the plain operands (the layout's get_plain_tensors view) and `params` the
    layer's config.  Calling it runs the matching qlin op."""
    kind: str
    out_features: int
    in_features: int
    tensors: dict
    params: dict = field(default_factory=dict)
    bias: torch.Tensor | None = None

    def __call__(self, x, out_dtype=None, lora_down=None, lora_up=None, lora_scale=None):
        from . import ops
        t, p = self.tensors, self.params
        lora = dict(lora_down=lora_down, lora_up=lora_up, lora_scale=lora_scale)
        if self.kind == "int8":
            return ops.int8_linear(x, t["qdata"], t["scale"], self.bias, out_dtype, convrot=p["convrot"],
                                   convrot_groupsize=p["convrot_groupsize"], **lora)
        if self.kind == "w4a8":
            return ops.w4a8_int8_linear(x, t["qdata"], t["s_rel"], t["s_channel"], t.get("codebook"), None, self.bias,
                                        p["group_size"], p["convrot_groupsize"], out_dtype, **lora)
        if self.kind == "gguf":
            if self.in_features % GGUF_TYPES[p["qtype"]][1]:
                raise NoCapableBackendError("gguf_linear", {"hip": "rows straddle GGUF blocks (use dequantize)"})
            return ops.gguf_linear(x, t["data"], p["qtype"], (self.out_features, self.in_features), self.bias,
                                   out_dtype, **lora)
        raise ValueError(f"unknown layer kind {self.kind}")

    def dequantize(self, out_dtype=torch.float32):
        """The weight in the original basis, [out_features, in_features]."""
        from . import ops
        t, p = self.tensors, self.params
        if self.kind == "int8":
            g = p["convrot_groupsize"] if p["convrot"] else 0
            return ops.dequantize_int8_convrot_weight(t["qdata"], t["scale"], g).to(out_dtype)
        if self.kind == "w4a8":
            return ops.dequantize_w4a8_int8_weight(t["qdata"], t["s_rel"], t["s_channel"], t.get("codebook"), None,
                                                   p["group_size"], p["convrot_groupsize"], out_dtype)
        return ops.dequantize_gguf(t["data"], p["qtype"], (self.out_features, self.in_features), out_dtype)


W4A8_FORMATS = {"asym_w4a8_int8": 4, "w6a8_int8": 6}


def _config(t):
    return json.loads(bytes(t.cpu().numpy().tobytes()).decode("utf-8"))


def quantized_linears(state):
    """{layer prefix: PackedLinear} for every layer of a loaded state dict that carries a
    `comfy_quant` config: "int8_tensorwise" (`weight` I8 [N, K], `weight_scale`; config keys
    convrot, convrot_groupsize) or "asym_w4a8_int8" / "w6a8_int8" (`weight` [N, K*bits/8],
    `weight_s_rel` [N, K/group_size], `weight_s_channel` [N], optional `weight_codebook` [16];
    config keys group_size, convrot_groupsize).  The tensors are the loaded ones (no copies)."""
    out = {}
    for key in state:
        if not key.endswith("comfy_quant"):
            continue
        prefix = key[: -len("comfy_quant")]
        name = prefix.rstrip(".")
        conf = _config(state[key])
        fmt = conf.get("format")
        w = state.get(prefix + "weight")
        if w is None:
            raise ValueError(f"{name}: comfy_quant without a weight")
        bias = state.get(prefix + "bias")
        if fmt == "int8_tensorwise":
            if w.dtype != torch.int8 or w.dim() != 2:
                raise ValueError(f"{name}: int8_tensorwise weight must be I8 [N, K], got {w.dtype} {tuple(w.shape)}")
            scale = state[prefix + "weight_scale"]
            params = {"convrot": bool(conf.get("convrot", False)),
                      "convrot_groupsize": int(conf.get("convrot_groupsize", 256))}
            out[name] = PackedLinear("int8", w.shape[0], w.shape[1], {"qdata": w, "scale": scale}, params, bias)
        elif fmt in W4A8_FORMATS:
            s_rel, s_ch = state[prefix + "weight_s_rel"], state[prefix + "weight_s_channel"]
            gs = int(conf.get("group_size", 16))
            n, k = w.shape[0], s_rel.shape[1] * gs
            bits = W4A8_FORMATS[fmt]
            if w.dim() != 2 or w.shape[1] * 8 != k * bits:
                raise ValueError(f"{name}: {fmt} weight {tuple(w.shape)} does not hold {bits}-bit codes for K={k}")
            t = {"qdata": w, "s_rel": s_rel, "s_channel": s_ch}
            if prefix + "weight_codebook" in state:
                t["codebook"] = state[prefix + "weight_codebook"]
            if conf.get("correction") is not None or prefix + "weight_correction" in state:
                raise NoCapableBackendError("w4a8_int8_linear", {"hip": f"{name}: the `correction` variant is not implemented"})
            params = {"group_size": gs, "convrot_groupsize": int(conf.get("convrot_groupsize", 256)), "bits": bits}
            out[name] = PackedLinear("w4a8", n, k, t, params, bias)
        else:
            raise NoCapableBackendError("quantized_linears", {"hip": f"{name}: format {fmt!r} is not supported"})
    return out


# --------------------------------------------------------------------------- GGUF

GGUF_MAGIC = b"GGUF"
# GGUF metadata value types: id -> struct format (8 = string, 9 = array)
GGUF_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
# ggml float types kept as plain tensors: id -> (torch dtype, bytes)
GGML_FLOAT = {0: torch.float32, 1: torch.float16, 30: torch.bfloat16}


@dataclass
class GGUFTensorInfo:
    name: str
    dims: list          # ggml order: dims[0] is the contiguous (row) dimension
    ggml_type: int
    offset: int         # from the data start
    nbytes: int
    shape: tuple        # torch shape: reversed dims, or comfy.gguf.orig_shape.<name>


class _Cursor:
    def __init__(self, data, path):
        self.data, self.pos, self.path = data, 0, path

    def take(self, n):
        if self.pos + n > len(self.data):
            raise EOFError
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self):
        return self.take(self.u64()).decode("utf-8")

    def value(self, vtype):
        if vtype in GGUF_SCALARS:
            fmt = GGUF_SCALARS[vtype]
            return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        if vtype == 8:
            return self.string()
        if vtype == 9:
            etype, n = self.u32(), self.u64()
            return [self.value(etype) for _ in range(n)]
        raise ValueError(f"{self.path}: unknown GGUF value type {vtype}")


def _gguf_nbytes(ggml_type, nelem, name):
    if ggml_type in GGML_FLOAT:
        return nelem * torch.empty((), dtype=GGML_FLOAT[ggml_type]).element_size()
    if ggml_type in GGUF_NAMES:
        _, qk, ts = GGUF_TYPES[GGUF_NAMES[ggml_type]]
        if nelem % qk:
            raise ValueError(f"tensor {name}: {nelem} values is not a whole number of {qk}-value blocks")
        return nelem // qk * ts
    raise NoCapableBackendError("load_gguf", {"hip": f"tensor {name}: ggml type {ggml_type} is not supported"})


def gguf_header(path, max_header=64 << 20):
    """(version, {key: value}, [GGUFTensorInfo], data start byte) of a GGUF v2/v3 file.

    Layout: magic "GGUF", u32 version, u64 tensor count, u64 key/value count, the key/value pairs
    (u64-length string key, u32 type, value), the tensor infos (name, u32 rank, u64 dims, u32 ggml
    type, u64 offset), then the data at the next multiple of general.alignment (default 32)."""
    with _Reader(path) as r:
        head = r.pread(0, min(r.size, max_header))
        size = r.size
    c = _Cursor(head, path)
    try:
        if c.take(4) != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file")
        version = c.u32()
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version} is not supported")
        n_tensors, n_kv = c.u64(), c.u64()
        kv = {}
        for _ in range(n_kv):
            key = c.string()
            kv[key] = c.value(c.u32())
        raw = []
        for _ in range(n_tensors):
            name = c.string()
            dims = [c.u64() for _ in range(c.u32())]
            raw.append((name, dims, c.u32(), c.u64()))
    except EOFError:
        raise ValueError(f"{path}: truncated GGUF header") from None
    align = int(kv.get("general.alignment", 32))
    if align <= 0 or align & (align - 1):
        raise ValueError(f"{path}: general.alignment {align} is not a power of two")
    start = (c.pos + align - 1) // align * align
    infos = []
    for name, dims, qt, off in raw:
        nelem = math.prod(dims)
        nbytes = _gguf_nbytes(qt, nelem, name)
        if off % align or start + off + nbytes > size:
            raise ValueError(f"{path}: tensor {name} at offset {off} ({nbytes} bytes) is misplaced")
        orig = kv.get("comfy.gguf.orig_shape." + name)
        shape = tuple(int(d) for d in orig) if orig is not None else tuple(int(d) for d in reversed(dims))
        if math.prod(shape) != nelem:
            raise ValueError(f"{path}: orig_shape {shape} of {name} does not hold {nelem} values")
        infos.append(GGUFTensorInfo(name, dims, qt, off, nbytes, shape))
    return version, kv, infos, start


def load_gguf(path, device="cuda", keys=None, chunk=CHUNK):
    """({name: tensor or PackedLinear}, {key: value}).  Float tensors (F32, F16, BF16) come back
    as plain tensors of their torch shape; block-quantized 2-D tensors as PackedLinear("gguf")
    whose `data` is the raw block bytes on `device` ([N, row bytes] when rows are whole blocks,
    flat otherwise) and whose shape is the torch shape (orig_shape when the file records one)."""
    _, kv, infos, start = gguf_header(path)
    dev = _device(device)
    want = None if keys is None else set(keys)
    out = {}
    with _Reader(path, chunk) as r:
        for info in sorted(infos, key=lambda i: i.offset):
            if want is not None and info.name not in want:
                continue
            if info.ggml_type in GGML_FLOAT:
                t = torch.empty(info.shape, dtype=GGML_FLOAT[info.ggml_type], device=dev)
                r.into(t, start + info.offset)
                out[info.name] = t
                continue
            qtype = GGUF_NAMES[info.ggml_type]
            _, qk, ts = GGUF_TYPES[qtype]
            shape = info.shape if len(info.shape) == 2 else (math.prod(info.shape[:-1]), info.shape[-1])
            n, k = shape
            data = torch.empty((n, k // qk * ts) if k % qk == 0 else (info.nbytes,), dtype=torch.uint8, device=dev)
            r.into(data, start + info.offset)
            out[info.name] = PackedLinear("gguf", n, k, {"data": data}, {"qtype": qtype, "shape": info.shape})
    if want is not None and want - set(out):
        raise KeyError(f"{path}: no tensors {sorted(want - set(out))}")
    return out, kv
