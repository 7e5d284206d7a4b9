"""A minimal GGUF v3 writer for tests, byte by byte from the file layout the reference's header
reader walks (roblennon/mac-kernels-public bench/gguf_headers.py:80-110): magic "GGUF", u32
version, u64 tensor count, u64 key/value count, key/value pairs (u64-length UTF-8 key, u32 value
type, value), tensor infos (name, u32 rank, u64 dims in ggml order, u32 ggml type, u64 offset
from the data start), zero padding to general.alignment, then the tensor data, each tensor at an
aligned offset."""
import struct

# value type ids of the GGUF key/value section
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v, etype=None):
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        return struct.pack("<IQ", etype, len(v)) + b"".join(_value(etype, e) for e in v)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, kv, tensors, alignment=32):
    """kv: [(key, vtype, value[, element type for arrays])]; tensors: [(name, ggml dims, ggml type,
    data bytes)].  Returns {name: absolute byte offset of its data}."""
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for item in kv:
        key, vtype, value = item[:3]
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, value, item[3] if len(item) > 3 else None)
    offsets, off = [], 0
    for name, dims, qtype, data in tensors:
        offsets.append(off)
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", qtype, off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    start = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(off)
    for (name, dims, qtype, data), o in zip(tensors, offsets):
        body[o:o + len(data)] = data
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)) + bytes(body))
    return {t[0]: start + o for t, o in zip(tensors, offsets)}
