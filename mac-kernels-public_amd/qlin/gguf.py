"""GGUF block-type table (ggml type id, values per block, bytes per block).

Mirrors the type table the reference's gguf backend exposes as ``GGUF_TYPES[name] = (type_id,
qk, type_size)`` (roblennon/mac-kernels-public bench/bench_gguf_linear.py:70, 90).  The ids are
ggml's ``enum ggml_type`` (Q8_0 = 8 and Q4_K = 12 are pinned at modal/weight_error_app.py:84);
block sizes follow docs/research/2026-10-03-gguf-on-metal.md:18-29.
"""
GGUF_TYPES = {
    "Q4_0": (2, 32, 18), "Q4_1": (3, 32, 20), "Q5_0": (6, 32, 22), "Q5_1": (7, 32, 24),
    "Q8_0": (8, 32, 34), "Q2_K": (10, 256, 84), "Q3_K": (11, 256, 110), "Q4_K": (12, 256, 144),
    "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210), "IQ4_NL": (20, 32, 18), "IQ4_XS": (23, 256, 136),
}
GGUF_NAMES = {v[0]: k for k, v in GGUF_TYPES.items()}


def gguf_type_id(qtype) -> int:
    """Accept a ggml type id, a type name ('Q4_K') or an enum with .value / .name."""
    if isinstance(qtype, str):
        key = qtype.upper()
        if key not in GGUF_TYPES:
            raise ValueError(f"unknown GGUF type {qtype}")
        return GGUF_TYPES[key][0]
    if hasattr(qtype, "value"):
        qtype = qtype.value
    tid = int(qtype)
    if tid not in GGUF_NAMES:
        from .exceptions import NoCapableBackendError
        raise NoCapableBackendError("gguf_linear", {"hip": f"ggml type {tid} is not supported"})
    return tid


def row_bytes(qtype, k: int) -> int:
    _, qk, ts = GGUF_TYPES[GGUF_NAMES[gguf_type_id(qtype)]]
    return k // qk * ts
