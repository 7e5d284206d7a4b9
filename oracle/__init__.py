"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE, never the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package.  It restates the reference's codecs (roblennon/mac-kernels-public,
``modal/weight_error_app.py:88-339``, ``modal/modal_app.py:30-50``,
``docs/research/2026-10-03-gguf-on-metal.md:18-36``) in plain C (``qlin_oracle.c``, built by
``oracle/Makefile`` into ``liboracle_qlin.so``) with numpy wrappers.  The quantizers that make packed
test inputs live in the product's host layer (``qlin/quantize.py``) and are pinned by the same golden
vectors.

Parity pins (checked in tests/test_oracle_*.py):
  * GGUF Q8_0 / Q4_K decode ........ reference golden deq sha256 (bit-exact)
  * INT8 rowwise quant + decode .... reference golden q/scale/deq sha256 (bit-exact)
  * W4A8 / W6A8 int8-grid decode ... reference golden raw q/s_rel/s_channel/codebook, decoded and
                                     rotated, against the golden deq (sha256 or 1-ulp tolerance)
  * Q4_0 ........................... closed form of modal/modal_app.py:42-50, brute force
  * Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K, Q6_K: written formulas only, checked with known-answer
    blocks built by hand in the tests (parity otherwise unpinned by reference vectors)
  * IQ4_NL / IQ4_XS ................ parity unpinned (the reference holds neither table nor
                                     vectors); known-answer blocks check the layout only
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_qlin.so")
_lib = None

# ggml type ids (enum ggml_type) -> (name, values per block, bytes per block)
GGUF_TYPES = {
    "Q4_0": (2, 32, 18), "Q4_1": (3, 32, 20), "Q5_0": (6, 32, 22), "Q5_1": (7, 32, 24),
    "Q8_0": (8, 32, 34), "Q2_K": (10, 256, 84), "Q3_K": (11, 256, 110), "Q4_K": (12, 256, 144),
    "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210), "IQ4_NL": (20, 32, 18), "IQ4_XS": (23, 256, 136),
}
GGUF_BY_ID = {v[0]: k for k, v in GGUF_TYPES.items()}


def build(force: bool = False) -> str:
    """Compile the C restatement (make -C oracle)."""
    if force or not os.path.exists(_LIB_PATH) or (
            os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "qlin_oracle.c"))):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        sigs = {
            "qlo_gguf_dequantize": (I, [I, P, I64, P]),
            "qlo_gguf_dequantize_range": (I, [I, P, I64, I64, P]),
            "qlo_gguf_block_info": (I, [I, P, P]),
            "qlo_dequantize_int8": (None, [P, P, I64, I64, P]),
            "qlo_quantize_int8_rowwise_f32": (None, [P, I64, I64, P, P]),
            "qlo_quantize_int8_rowwise_f16": (None, [P, I64, I64, P, P]),
            "qlo_quantize_int8_rowwise_bf16": (None, [P, I64, I64, P, P]),
            "qlo_rotate_f32": (I, [P, I64, I64, I, P]),
            "qlo_rotate_f16": (I, [P, I64, I64, I, P]),
            "qlo_hadamard_sign": (I, [I, I, I]),
            "qlo_hadamard_valid": (I, [I]),
            "qlo_unpack_codes": (None, [P, I64, I64, I, P]),
            "qlo_w4a8_int8_grid": (None, [P, P, P, I64, I64, I, I, P]),
            "qlo_linear_f64": (None, [P, P, P, I64, I64, I64, P]),
            "qlo_int8_gemm_i64": (None, [P, P, I64, I64, I64, P]),
            "qlo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "qlo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "qlo_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
            "qlo_f32_to_e4m3": (ctypes.c_uint8, [ctypes.c_float]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# --- scalar formats --------------------------------------------------------------------------

def e4m3_to_f32(raw: np.ndarray) -> np.ndarray:
    """float8_e4m3fn bit patterns (uint8) -> float32, exact."""
    raw = np.asarray(raw, dtype=np.uint8)
    table = np.array([lib().qlo_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return table[raw]


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> float8_e4m3fn bits, round to nearest even (torch's cast semantics)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().qlo_f32_to_e4m3
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint8).reshape(x.shape)


# --- GGUF ------------------------------------------------------------------------------------

def gguf_type_id(qtype) -> int:
    if isinstance(qtype, str):
        return GGUF_TYPES[qtype.upper()][0]
    return int(qtype)


def gguf_dequantize(raw: np.ndarray, qtype, shape=None) -> np.ndarray:
    """Decode a flat run of GGUF blocks to float32 (gguf-py 0.19.0 operation order)."""
    tid = gguf_type_id(qtype)
    _, qk, ts = GGUF_TYPES[GGUF_BY_ID[tid]]
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    assert raw.size % ts == 0, "byte count is not a whole number of blocks"
    nb = raw.size // ts
    out = np.empty(nb * qk, dtype=np.float32)
    rc = lib().qlo_gguf_dequantize(tid, _p(raw), nb, _p(out))
    assert rc == 0, f"unsupported ggml type {tid}"
    if shape is not None:
        n, k = shape
        if n * k != out.size:
            out = out[: n * k]
        out = out.reshape(n, k)
    return out


# --- INT8 ------------------------------------------------------------------------------------

def dequantize_int8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    n, k = q.shape
    s = np.ascontiguousarray(np.asarray(scale, dtype=np.float32).reshape(-1))
    if s.size == 1:
        s = np.full(n, s[0], dtype=np.float32)
    out = np.empty((n, k), dtype=np.float32)
    lib().qlo_dequantize_int8(_p(q), _p(s), n, k, _p(out))
    return out


def quantize_int8_rowwise(x: np.ndarray, bf16: bool = False):
    """quantize_int8_rowwise for fp32, fp16 or bf16 rows (bf16 given as uint16 bit patterns with
    bf16=True); returns (int8 q, fp32 scale [m, 1])."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    q = np.empty((m, k), dtype=np.int8)
    s = np.empty(m, dtype=np.float32)
    if bf16:
        lib().qlo_quantize_int8_rowwise_bf16(_p(x.view(np.uint16)), m, k, _p(q), _p(s))
    elif x.dtype == np.float16:
        lib().qlo_quantize_int8_rowwise_f16(_p(x.view(np.uint16)), m, k, _p(q), _p(s))
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        lib().qlo_quantize_int8_rowwise_f32(_p(x), m, k, _p(q), _p(s))
    return q, s.reshape(m, 1)


def hadamard(g: int) -> np.ndarray:
    """Normalized Hadamard matrix of size g (power of 4, or 2 * power of 4)."""
    assert lib().qlo_hadamard_valid(g), f"unsupported Hadamard size {g}"
    L = lib()
    sgn = np.array([[L.qlo_hadamard_sign(g, i, j) for j in range(g)] for i in range(g)], dtype=np.float64)
    return sgn / np.sqrt(g)


def rotate(x: np.ndarray, g: int) -> np.ndarray:
    """Per-group rotation x[:, grp] @ H^T, computed exactly and rounded once (fp32 in -> fp32,
    fp16 in -> fp16)."""
    x = np.ascontiguousarray(x)
    lead = x.shape[:-1]
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    out = np.empty_like(x2)
    if x.dtype == np.float16:
        rc = lib().qlo_rotate_f16(_p(x2.view(np.uint16)), x2.shape[0], k, g, _p(out.view(np.uint16)))
    else:
        x2 = np.ascontiguousarray(x2, dtype=np.float32)
        out = np.empty_like(x2)
        rc = lib().qlo_rotate_f32(_p(x2), x2.shape[0], k, g, _p(out))
    assert rc == 0, "rotation needs K % G == 0 and G a power of 4 or 2*4^p"
    return out.reshape(*lead, k)


def dequantize_int8_convrot(q, scale, g=256) -> np.ndarray:
    """Original-basis weight rotate(q * s) (weight_error_app.py:126-127)."""
    return rotate(dequantize_int8(q, scale), g)


# --- W4A8 / W6A8 -----------------------------------------------------------------------------

def srel_to_f32(s_rel: np.ndarray, dtype: str) -> np.ndarray:
    """Widen stored group scales (e4m3 bits as uint8, fp16, or fp32) to float32."""
    if dtype == "e4m3":
        return e4m3_to_f32(np.asarray(s_rel, dtype=np.uint8))
    return np.asarray(s_rel).astype(np.float32)


def unpack_codes(q: np.ndarray, k: int, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(q).view(np.uint8)
    n = q.shape[0]
    codes = np.empty((n, k), dtype=np.int32)
    lib().qlo_unpack_codes(_p(q), n, k, bits, _p(codes))
    return codes


def w4a8_int8_grid(q, s_rel_f32, codebook, k, bits, group_size) -> np.ndarray:
    """Packed codes -> int8 grid w8 (weight_error_app.py:326-337)."""
    q = np.ascontiguousarray(q).view(np.uint8)
    n = q.shape[0]
    sr = np.ascontiguousarray(s_rel_f32, dtype=np.float32)
    assert sr.shape == (n, k // group_size)
    cb = None if codebook is None else np.ascontiguousarray(codebook, dtype=np.float32)
    w8 = np.empty((n, k), dtype=np.int8)
    lib().qlo_w4a8_int8_grid(_p(q), _p(sr), None if cb is None else _p(cb), n, k, bits, group_size, _p(w8))
    return w8


def dequantize_w4a8(q, s_rel_f32, s_channel, codebook, group_size=16, convrot_groupsize=256,
                    bits=None, rotated_basis=False) -> np.ndarray:
    """Packed storage -> fp32 weight (original basis unless rotated_basis)."""
    q = np.ascontiguousarray(q).view(np.uint8)
    n, cols = q.shape
    k = s_rel_f32.shape[1] * group_size
    bits = bits or (cols * 8) // k
    w8 = w4a8_int8_grid(q, s_rel_f32, codebook, k, bits, group_size)
    w = w8.astype(np.float32) * np.asarray(s_channel, dtype=np.float32).reshape(n, 1)
    if rotated_basis or not convrot_groupsize:
        return w
    return rotate(w, convrot_groupsize)


# --- dense reference ------------------------------------------------------------------------

def linear_f64(x: np.ndarray, w: np.ndarray, bias=None) -> np.ndarray:
    """y = x @ w^T (+ bias) over float32 operands, accumulated in float64 (BLAS-free)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().qlo_linear_f64(_p(x), _p(w), None if b is None else _p(b), m, n, k, _p(y))
    return y


def linear_ref(x: np.ndarray, w: np.ndarray, bias=None) -> np.ndarray:
    """Fast float64 reference for large shapes (numpy BLAS in float64)."""
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def int8_gemm_i64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), dtype=np.int64)
    lib().qlo_int8_gemm_i64(_p(a), _p(b), m, n, k, _p(c))
    return c


def rel_fro(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))
