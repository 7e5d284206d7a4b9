"""The C ABI library without a GPU: it loads, exports every symbol include/qlin.h declares, and
rejects malformed or unsupported calls before launching anything."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "qlin.h")).read()
    return sorted(set(re.findall(r"\b(qlin_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from qlin import _lib
    L = _lib.load()
    syms = header_symbols()
    assert len(syms) >= 12
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(_lib.EXPORTS)
    assert L.qlin_version() == 1
    assert L.qlin_status_string(1) == b"unsupported"


def test_query_and_workspace():
    from qlin import _lib
    L = _lib.load()
    assert L.qlin_query(_lib.OP_GGUF_LINEAR, 1, 4096, 4096, 12, _lib.DT_F16, _lib.DT_F16) == 0
    assert L.qlin_query(_lib.OP_GGUF_LINEAR, 1, 4096, 4096, 99, _lib.DT_F16, _lib.DT_F16) == 1
    assert L.qlin_query(_lib.OP_GGUF_LINEAR, 1, 4096, 4000, 12, _lib.DT_F16, _lib.DT_F16) == 1
    assert L.qlin_query(_lib.OP_INT8_LINEAR, 8, 64, 768, 256, _lib.DT_F16, _lib.DT_F16) == 0
    assert L.qlin_query(_lib.OP_INT8_LINEAR, 8, 64, 768, 100, _lib.DT_F16, _lib.DT_F16) == 1
    assert L.qlin_query(_lib.OP_W4A8_LINEAR, 8, 64, 3072, 4, _lib.DT_F16, _lib.DT_BF16) == 0
    assert L.qlin_query(_lib.OP_W4A8_LINEAR, 8, 64, 3072, 5, _lib.DT_F16, _lib.DT_F16) == 1
    assert b"bits" in L.qlin_last_error()
    # contractions: A8 up to 131072 (its int32 sums stay exact), the weight-only linears up to 2^20
    # (chunked prologue past 32768, fp32 accumulation); longer ones decline
    for op, p, kmax in ((_lib.OP_INT8_LINEAR, 128, 1 << 20), (_lib.OP_W4A8_LINEAR, 6, 131072),
                        (_lib.OP_GGUF_LINEAR, 12, 1 << 20)):
        assert L.qlin_query(op, 8, 64, kmax, p, _lib.DT_F16, _lib.DT_F16) == 0
        assert L.qlin_query(op, 8, 64, kmax + 256, p, _lib.DT_F16, _lib.DT_F16) == 1
    ws = L.qlin_workspace_size(_lib.OP_INT8_LINEAR, 256, 3072, 3072, 128, _lib.DT_F16)
    assert ws >= 256 * 3072 * 2 + 256 * 4


def test_workspace_sizes_follow_the_paths():
    """The sizes the C ABI asks for: the A8 int8 grid (N*K bytes) only where the call decodes the
    weight once (from 512 rows, with a group size that is a multiple of 64; counted when the group
    size is not given), and the GGUF decoded fp16 copy above the split kernel's 512 rows, capped at
    256 MiB; the split kernel's fp32 partials where it splits K."""
    from qlin import _lib
    L = _lib.load()
    a = lambda v: (v + 255) // 256 * 256
    m, n, k = 1024, 4096, 4096
    act = a(m * k) + a(m * 4)
    size = lambda p: L.qlin_workspace_size(_lib.OP_W4A8_LINEAR, m, n, k, p, _lib.DT_F16)
    assert size(4 | 16 << 8) == act                  # group 16: decoded per tile, no grid
    assert size(4 | 64 << 8) == act + a(n * k)       # group 64: the grid
    assert size(6 | 128 << 8) == act + a(n * k)
    assert size(4) == act + a(n * k)                 # group size not given: counted
    assert L.qlin_workspace_size(_lib.OP_W4A8_LINEAR, 16, n, k, 4 | 64 << 8, _lib.DT_F16) == a(16 * k) + a(16 * 4)
    lora = lambda p: L.qlin_workspace_size(_lib.OP_W4A8_LINEAR_LORA, m, n, k, p, _lib.DT_F16)
    assert lora(64 | 64 << 16) - lora(64 | 16 << 16) == a(n * k)
    # GGUF above 512 rows (Q4_K, type 12): the decoded copy, at most 256 MiB (32768 rows of K = 4096)
    g = lambda m, n, t=12: L.qlin_workspace_size(_lib.OP_GGUF_LINEAR, m, n, 4096, t, _lib.DT_F16)
    base = lambda m, n: a(m * 4096 * 2) + a(m * 4) + a(n * 4)
    assert g(600, 4096) == base(600, 4096) + a(4096 * 4096 * 2)
    assert g(600, 128256) == base(600, 128256) + (256 << 20)
    assert g(64, 128256) < (64 << 20)                # K split or small-M kernels: no copy
    # the split kernel's m-tiles up to 512 rows: 32 row blocks x 2 m-tiles = 64 tiles -> 4 splits
    # of fp32 partials at M = 100; 32 x 8 tiles fill the GPU at M = 512 -> one split, no partials
    assert g(100, 4096) == base(100, 4096) + a(4 * 100 * 4096 * 4)
    assert g(512, 4096) == base(512, 4096)
    assert g(384, 4096) == base(384, 4096)           # 192 tiles, 3/4 of the GPU: one split
    assert g(256, 4096) == base(256, 4096) + a(2 * 256 * 4096 * 4)  # 128 tiles: two splits
    assert g(512, 4096, 14) == base(512, 4096)       # Q6_K: the split kernel to 512 rows as well
    assert g(520, 4096, 14) == base(520, 4096) + a(4096 * 4096 * 2)


def _d(t, dt=None):
    from qlin import _lib
    return _lib.desc(t, dt)


def test_malformed_calls_are_rejected_before_launch():
    from qlin import _lib
    L = _lib.load()
    x = torch.zeros(4, 256, dtype=torch.float16)
    y = torch.zeros(4, 32, dtype=torch.float16)
    # unknown ggml type -> unsupported
    assert L.qlin_gguf_linear(_d(x), 1, 99, 32, 256, None, _d(y), None, 0, None) == _lib.QLIN_EUNSUPPORTED
    # K not a whole number of blocks -> unsupported (rows would straddle blocks)
    assert L.qlin_gguf_linear(_d(x), 1, 12, 32, 250, None, _d(y), None, 0, None) == _lib.QLIN_EUNSUPPORTED
    # y with the wrong shape -> invalid
    yb = torch.zeros(4, 31, dtype=torch.float16)
    assert L.qlin_gguf_linear(_d(x), 1, 8, 32, 256, None, _d(yb), None, 0, None) == _lib.QLIN_EINVAL
    # workspace too small
    assert L.qlin_gguf_linear(_d(x), 1, 8, 32, 256, None, _d(y), None, 0, None) == _lib.QLIN_EWORKSPACE
    # INT8: bad ConvRot group, non-int8 weight, missing x
    q = torch.zeros(32, 256, dtype=torch.int8)
    s = torch.ones(32)
    assert L.qlin_int8_linear(_d(x), _d(q), _d(s), None, _d(y), 100, None, 0, None) == _lib.QLIN_EUNSUPPORTED
    assert L.qlin_int8_linear(_d(x), _d(q.float()), _d(s), None, _d(y), 0, None, 0, None) == _lib.QLIN_EUNSUPPORTED
    assert L.qlin_int8_linear(None, _d(q), _d(s), None, _d(y), 0, None, 0, None) == _lib.QLIN_EINVAL
    # scale with the wrong length
    assert L.qlin_int8_linear(_d(x), _d(q), _d(torch.ones(7)), None, _d(y), 0, None, 0, None) == _lib.QLIN_EINVAL
    # W4A8: 5 bits, codebook with 6 bits
    qq = torch.zeros(32, 128, dtype=torch.int8)
    sr = torch.ones(32, 16)
    assert L.qlin_w4a8_linear(_d(x), _d(qq), _d(sr), _d(s), None, None, _d(y), 5, 16, 256, None, 0, None) == 1
    q6 = torch.zeros(32, 192, dtype=torch.int8)
    cb = torch.zeros(16)
    assert L.qlin_w4a8_linear(_d(x), _d(q6), _d(sr), _d(s), _d(cb), None, _d(y), 6, 16, 256, None, 0, None) == 1
    assert b"codebook" in L.qlin_last_error()


def test_gradient_and_lora_calls_are_rejected_before_launch():
    from qlin import _lib
    L = _lib.load()
    dy = torch.zeros(4, 32, dtype=torch.float16)
    dx = torch.zeros(4, 256, dtype=torch.float16)
    q = torch.zeros(32, 256, dtype=torch.int8)
    s = torch.ones(32)
    big = 1 << 30
    # dx of the wrong shape, an unsupported group, K not a multiple of 16, a short workspace
    assert L.qlin_int8_linear_grad_input(_d(dy), _d(q), _d(s), 0, _d(dx[:, :255]), None, big, None) == _lib.QLIN_EINVAL
    assert L.qlin_int8_linear_grad_input(_d(dy), _d(q), _d(s), 100, _d(dx), None, big, None) == _lib.QLIN_EUNSUPPORTED
    q8 = torch.zeros(32, 248, dtype=torch.int8)
    dx8 = torch.zeros(4, 248, dtype=torch.float16)
    assert L.qlin_int8_linear_grad_input(_d(dy), _d(q8), _d(s), 0, _d(dx8), None, big, None) == _lib.QLIN_EUNSUPPORTED
    assert L.qlin_int8_linear_grad_input(_d(dy), _d(q), _d(s), 0, _d(dx), None, 0, None) == _lib.QLIN_EWORKSPACE
    need = L.qlin_workspace_size(_lib.OP_INT8_GRAD_INPUT, 4, 32, 256, 0, _lib.DT_F16)
    assert need >= 4 * 128 * 2 + 4 * 4  # dy rows padded to 128 values, plus exponents
    assert L.qlin_workspace_size(_lib.OP_W4A8_GRAD_INPUT, 4, 32, 256, 4, _lib.DT_F16) >= need + 32 * 256
    # W4A8 gradient: 5 bits, s_rel of the wrong shape
    qq = torch.zeros(32, 128, dtype=torch.int8)
    sr = torch.ones(32, 16)
    assert L.qlin_w4a8_linear_grad_input(_d(dy), _d(qq), _d(sr), _d(s), None, _d(dx), 5, 16, 256, None, big, None) == 1
    assert L.qlin_w4a8_linear_grad_input(_d(dy), _d(qq), _d(sr[:, :8]), _d(s), None, _d(dx), 4, 16, 256, None, big,
                                         None) == _lib.QLIN_EINVAL
    # LoRA: factors that do not fit x and y, a short workspace
    x = torch.zeros(4, 256, dtype=torch.float16)
    y = torch.zeros(4, 32, dtype=torch.float16)
    down, up = torch.zeros(8, 256, dtype=torch.float16), torch.zeros(32, 8, dtype=torch.float16)
    assert L.qlin_lora_apply(_d(x), _d(down[:, :128]), _d(up), 1.0, _d(y), None, big, None) == _lib.QLIN_EINVAL
    assert L.qlin_lora_apply(_d(x), _d(down), _d(up[:, :4]), 1.0, _d(y), None, big, None) == _lib.QLIN_EINVAL
    assert L.qlin_lora_apply(_d(x), _d(down), _d(up), 1.0, _d(y), None, 0, None) == _lib.QLIN_EWORKSPACE


def test_decode_calls_are_rejected_before_launch():
    """The standalone decodes check their operands like the linears do."""
    from qlin import _lib
    L = _lib.load()
    n, k = 32, 256
    s = torch.ones(n)
    q4 = torch.zeros(n, k // 2, dtype=torch.int8)
    q6 = torch.zeros(n, k * 3 // 4, dtype=torch.int8)
    sr = torch.ones(n, k // 16)
    out = torch.zeros(n, k)
    cb = torch.zeros(16)
    # a codebook with 6-bit codes (codes reach 63, the table has 16 entries)
    assert L.qlin_dequantize_w4a8(_d(q6), _d(sr), _d(s), _d(cb), _d(out), 6, 16, 0, None) == _lib.QLIN_EUNSUPPORTED
    assert b"codebook" in L.qlin_last_error()
    # a codebook that is not float32
    assert L.qlin_dequantize_w4a8(_d(q4), _d(sr), _d(s), _d(cb.half()), _d(out), 4, 16, 0, None) == \
        _lib.QLIN_EUNSUPPORTED
    # qdata of the wrong dtype, columns that do not hold whole 6-bit codes, s_channel not float32
    assert L.qlin_dequantize_w4a8(_d(q4.float()), _d(sr), _d(s), None, _d(out), 4, 16, 0, None) == \
        _lib.QLIN_EUNSUPPORTED
    q6bad = torch.zeros(n, 191, dtype=torch.int8)
    assert L.qlin_dequantize_w4a8(_d(q6bad), _d(sr), _d(s), None, _d(out), 6, 16, 0, None) == _lib.QLIN_EINVAL
    assert L.qlin_dequantize_w4a8(_d(q4), _d(sr), _d(s.half()), None, _d(out), 4, 16, 0, None) == \
        _lib.QLIN_EUNSUPPORTED


def test_dequantize_gguf_checks_the_buffer_on_the_host():
    """A short, strided or mistyped weight buffer raises before anything is launched."""
    import qlin
    raw = torch.zeros(8 * 144, dtype=torch.uint8)          # 8 Q4_K blocks: 8 rows of 256 values
    with pytest.raises(ValueError):
        qlin.dequantize_gguf(raw[:-1], "Q4_K", (8, 256))     # one byte short
    with pytest.raises(ValueError):
        qlin.dequantize_gguf(raw, "Q4_K", (8, 512))          # shape needs twice the bytes
    with pytest.raises(ValueError):
        qlin.dequantize_gguf(raw, "Q4_K", (3, 100))          # not a whole number of blocks
    with pytest.raises(qlin.NoCapableBackendError):
        qlin.dequantize_gguf(raw.view(torch.int8), "Q4_K", (8, 256))
    with pytest.raises(qlin.NoCapableBackendError):
        qlin.dequantize_gguf(torch.zeros(8, 288, dtype=torch.uint8)[:, ::2], "Q4_K", (8, 256))
    with pytest.raises(qlin.NoCapableBackendError):         # well-formed, but on the host
        qlin.dequantize_gguf(raw, "Q4_K", (8, 256))


def test_gradient_ops_decline_on_the_host():
    import qlin
    dy = torch.zeros(2, 8, dtype=torch.float16)
    with pytest.raises(qlin.NoCapableBackendError):
        qlin.int8_linear_grad_input(dy, torch.zeros(8, 256, dtype=torch.int8), torch.ones(8), True, 256)
    with pytest.raises(qlin.NoCapableBackendError):  # the asymmetric variant, before any device check
        qlin.w4a8_linear_trainable(torch.zeros(2, 256), torch.zeros(8, 128, dtype=torch.int8), torch.ones(8, 16),
                                   torch.ones(8), None, torch.zeros(16, 8), None, 16, 256)


def test_ops_decline_cpu_tensors():
    import qlin
    x = torch.zeros(2, 256, dtype=torch.float16)
    with pytest.raises(qlin.NoCapableBackendError):
        qlin.int8_linear(x, torch.zeros(8, 256, dtype=torch.int8), torch.ones(8))


def test_registry():
    import qlin
    from qlin.exceptions import NoCapableBackendError
    fn = qlin.registry.get_implementation("int8_linear")
    assert fn is qlin.int8_linear
    # the lora_* keywords are declared by the three linears; other opt-in keywords still decline
    assert qlin.registry.get_implementation("gguf_linear", kwargs={"lora_down": object()}) is qlin.gguf_linear
    with pytest.raises(NoCapableBackendError) as e:
        qlin.registry.get_implementation("int8_linear", kwargs={"correction": object()})
    assert "hip" in e.value.reasons
    with pytest.raises(NoCapableBackendError):
        qlin.registry.get_implementation("scaled_mm_nvfp4")
    os.environ["QLIN_DISABLE"] = "1"
    try:
        with pytest.raises(NoCapableBackendError):
            qlin.registry.get_implementation("gguf_linear")
        assert "gguf_linear" in qlin.registry.capabilities()
    finally:
        del os.environ["QLIN_DISABLE"]


@pytest.mark.parametrize("g", [4, 8, 16, 32, 64, 128, 256])
def test_hadamard_invariants(g):
    import oracle as O
    from qlin.quantize import hadamard_signs
    h = O.hadamard(g)
    assert np.allclose(h, h.T)
    assert np.allclose(h @ h, np.eye(g), atol=1e-12)
    assert np.allclose(np.abs(h), 1 / np.sqrt(g))
    assert np.array_equal(hadamard_signs(g), np.sign(h))
    if g in (4, 16, 64, 256):  # the reference's construction: kron powers of H4, normalized
        h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
        r = h4
        while r.shape[0] < g:
            r = np.kron(r, h4)
        assert np.array_equal(np.sign(h), r)
    x = np.random.default_rng(0).standard_normal((3, 4 * g)).astype(np.float32)
    rx = O.rotate(x, g)
    assert np.allclose(rx, (x.astype(np.float64).reshape(3, 4, g) @ h.T).reshape(3, 4 * g), atol=1e-6)
    assert np.allclose(O.rotate(rx, g), x, atol=1e-5)


@pytest.mark.parametrize("name", ["Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K",
                                  "IQ4_NL", "IQ4_XS"])
def test_gguf_quantizer_round_trip(name):
    """The packer and the oracle's decoder agree on every field's position: the decode of the
    packed gaussian reproduces it to the format's precision (a swapped nibble, a misplaced scale
    or a wrong high-bit index blows the error up to O(1))."""
    import oracle as O
    from qlin.quantize import quantize_gguf
    bound = {"Q4_0": .1, "Q4_1": .1, "Q5_0": .05, "Q5_1": .05, "Q8_0": .007, "Q2_K": .4, "Q3_K": .2, "Q4_K": .1,
             "Q5_K": .05, "Q6_K": .025, "IQ4_NL": .1, "IQ4_XS": .1}[name]
    w = (np.random.default_rng(1).standard_normal((32, 512)) * 0.02).astype(np.float32)
    raw = quantize_gguf(w, name)
    assert raw.shape == (32, 512 // O.GGUF_TYPES[name][1] * O.GGUF_TYPES[name][2])
    assert O.rel_fro(O.gguf_dequantize(raw, name, w.shape), w) < bound


def test_int8_convrot_quantizer_matches_oracle():
    import oracle as O
    from qlin.quantize import quantize_int8_convrot_weight
    w = (np.random.default_rng(2).standard_normal((64, 512)) * 0.02).astype(np.float32)
    q, s = quantize_int8_convrot_weight(w, 256)
    oq, os_ = O.quantize_int8_rowwise(O.rotate(w, 256))
    assert np.array_equal(q, oq) and np.array_equal(s, os_.reshape(-1))
