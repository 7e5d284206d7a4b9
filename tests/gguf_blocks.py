"""Random legal GGUF blocks for the GPU tests: test-input generation, not part of the package.

The reference benchmarks its GGUF linear on blocks of uniformly random bytes whose fp16 scale
fields are overwritten with small positive values, so that the decoded weights have |w| of about
0.02-0.05 (bench/bench_gguf_linear.py:34-40, 69-78).  Every byte pattern is a legal block in
these formats, so only the scale fields need care.
"""
import numpy as np

from qlin.gguf import GGUF_NAMES, GGUF_TYPES, gguf_type_id

# Per format: byte offsets of its fp16 scale fields inside a block (d, and dmin where the format
# has one) and the scale magnitude drawn there.
SCALE_FIELDS = {
    "Q4_0": ((0,), 5e-3), "Q4_1": ((0, 2), 3e-3), "Q5_0": ((0,), 2.5e-3), "Q5_1": ((0, 2), 1.5e-3),
    "Q8_0": ((0,), 3e-4), "Q2_K": ((80, 82), 1e-3), "Q3_K": ((108,), 2e-4), "Q4_K": ((0, 2), 5e-5),
    "Q5_K": ((0, 2), 2.5e-5), "Q6_K": ((208,), 3e-5), "IQ4_NL": ((0,), 3e-4), "IQ4_XS": ((0,), 1e-5),
}


def random_gguf_blocks(qtype, n, k, seed=0):
    """uint8 block bytes for an [n, k] weight of `qtype` ([n, row bytes], or flat when k is not a
    whole number of blocks): random bytes, then |N(m, m)| fp16 values in the scale fields."""
    name = GGUF_NAMES[gguf_type_id(qtype)]
    qk, block_bytes = GGUF_TYPES[name][1:]
    blocks = n * k // qk
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(blocks, block_bytes), dtype=np.uint8)
    offsets, m = SCALE_FIELDS[name]
    for off in offsets:
        field = np.abs(m + m * rng.standard_normal(blocks)).astype(np.float16)
        raw[:, off:off + 2] = field.view(np.uint8).reshape(blocks, 2)
    if k % qk:
        return raw.reshape(-1)
    return raw.reshape(n, (k // qk) * block_bytes)
