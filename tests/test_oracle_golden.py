"""The CPU oracle and the offline quantizers against the reference's own golden vectors.

Fixtures: tests/golden/selftest_raw.npz + selftest_sha256.json, extracted by
tests/golden/make_fixtures.py from roblennon/mac-kernels-public
modal/results/2026-11-09-weight-error-selftest-container.json.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
from inputs import selftest_inputs

HERE = os.path.dirname(os.path.abspath(__file__))
RAW = np.load(os.path.join(HERE, "golden", "selftest_raw.npz"))
META = json.load(open(os.path.join(HERE, "golden", "selftest_sha256.json")))
SMALL = ("gauss_96x1024", "heavy_96x1024")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def inputs():
    return selftest_inputs()


def fmt(case, name):
    return META["cases"][case]["formats"][name]


def err(w, deq):
    d = deq.astype(np.float64) - w.astype(np.float64)
    return float(np.sqrt((d ** 2).sum() / (w.astype(np.float64) ** 2).sum())), float(np.abs(d).max())


def test_inputs_are_the_reference_inputs(inputs):
    for case, w in inputs.items():
        assert sha(w) == META["cases"][case]["input_sha256"], case


@pytest.mark.parametrize("case", SMALL)
@pytest.mark.parametrize("name,qtype", [("gguf_q8_0", "Q8_0"), ("gguf_q4_k", "Q4_K")])
def test_gguf_decode_bit_exact(case, name, qtype):
    raw = RAW[f"{case}/{name}/q"]
    deq = O.gguf_dequantize(raw, qtype, (96, 1024))
    assert sha(deq) == fmt(case, name)["deq"]


@pytest.mark.parametrize("case", SMALL + ("chunked_4200x1024",))
def test_int8_rowwise_quantize_and_decode_bit_exact(case, inputs):
    w = inputs[case]
    q, s = O.quantize_int8_rowwise(w)
    f = fmt(case, "int8_rowwise")
    assert sha(q) == f["q"] and sha(s) == f["scale"]
    assert sha(O.dequantize_int8(q, s)) == f["deq"]


@pytest.mark.parametrize("case", SMALL + ("chunked_4200x1024",))
def test_int8_convrot_codes(case, inputs):
    """ConvRot codes match the reference bit for bit with the exactly rounded rotation; the
    reference rotates through BLAS, so a row scale may differ by one ulp (heavy case)."""
    w = inputs[case]
    q, s = O.quantize_int8_rowwise(O.rotate(w, 256))
    f = fmt(case, "int8_convrot")
    assert sha(q) == f["q"]
    if case != "heavy_96x1024":
        assert sha(s) == f["scale"]
    rel, mx = err(w, O.dequantize_int8_convrot(q, s, 256))
    assert rel == pytest.approx(f["rel_fro"], rel=1e-6)
    assert mx == pytest.approx(f["max_abs"], rel=1e-5)


@pytest.mark.parametrize("case", SMALL)
@pytest.mark.parametrize("name,bits", [("w4a8", 4), ("w6a8", 6)])
def test_w4a8_int8_grid_decode(case, name, bits, inputs):
    """Decoding the reference's stored q/s_rel/s_channel/codebook reproduces its error figures to
    1e-6 relative (a single wrong int8 code moves rel_fro by ~4e-6)."""
    w = inputs[case]
    q = RAW[f"{case}/{name}/q"].reshape(96, -1)
    sr = O.e4m3_to_f32(RAW[f"{case}/{name}/s_rel"].reshape(96, -1))
    sc = RAW[f"{case}/{name}/s_channel"].view(np.float32)
    key = f"{case}/{name}/codebook"
    cb = RAW[key].view(np.float32) if key in RAW.files else None
    deq = O.dequantize_w4a8(q, sr, sc, cb, 16, 256)
    rel, mx = err(w, deq)
    f = fmt(case, name)
    assert rel == pytest.approx(f["rel_fro"], rel=1e-6)
    assert mx == pytest.approx(f["max_abs"], rel=1e-5)
    assert sha(np.ascontiguousarray(RAW[f"{case}/{name}/q"])) == f["q"]


@pytest.mark.parametrize("case", SMALL)
@pytest.mark.parametrize("name,bits", [("w4a8", 4), ("w6a8", 6)])
def test_w4a8_quantizer_matches_reference(case, name, bits, inputs):
    import torch
    from qlin.quantize import quantize_w4a8_int8_weight
    w = inputs[case]
    q, sr, sch, cb = quantize_w4a8_int8_weight(w, bits=bits, group_size=16, convrot_groupsize=256, codebook="auto")
    f = fmt(case, name)
    assert sha(q.numpy()) == f["q"]
    assert sha(sr.view(torch.uint8).numpy()) == f["s_rel"]
    if cb is not None:
        assert sha(cb.numpy()) == f["codebook"]
    # s_channel is a float max over BLAS-rotated values: equal bits on the gauss case, <= 1 ulp apart otherwise
    ref_sc = RAW[f"{case}/{name}/s_channel"].view(np.float32)
    assert np.max(np.abs(sch.numpy().view(np.int32) - ref_sc.view(np.int32))) <= 1


def test_q4_0_closed_form():
    """modal/modal_app.py:42-50: value = d * (nib - 8), low nibbles first, then high nibbles."""
    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, size=(300, 18), dtype=np.uint8)
    blocks[:, :2] = (np.abs(rng.standard_normal(300)) * 1e-2).astype(np.float16).view(np.uint8).reshape(300, 2)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32)
    nib = np.concatenate([blocks[:, 2:] & 0x0F, blocks[:, 2:] >> 4], axis=1).astype(np.float32)
    want = (d * (nib - 8.0)).reshape(-1)
    assert np.array_equal(O.gguf_dequantize(blocks, "Q4_0"), want)


def test_q8_0_known_answer():
    """tests/test_gguf_audit.py:33-35: codes arange(32), d = fp16(0.02) -> w[j] = j * fp16(0.02)."""
    blk = np.zeros((1, 34), dtype=np.uint8)
    blk[0, :2] = np.array([0.02], dtype=np.float16).view(np.uint8)
    blk[0, 2:] = np.arange(32, dtype=np.int8).view(np.uint8)
    got = O.gguf_dequantize(blk, "Q8_0")
    want = np.arange(32, dtype=np.float32) * np.float32(np.float16(0.02))
    assert np.array_equal(got, want)


def test_f16_e4m3_conversions_are_exact():
    L = O.lib()
    for h in range(0, 0x10000, 7):
        v = np.array([h], dtype=np.uint16).view(np.float16)[0]
        got = L.qlo_f16_to_f32(h)
        if np.isnan(v):
            assert np.isnan(got)
        else:
            assert got == np.float32(v)
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
                        np.array([65504, 65519.99, 65520, 6e-8, 2 ** -25, 3 * 2 ** -26], np.float32)])
    for v in x:
        assert L.qlo_f32_to_f16(float(v)) == np.array([np.float16(v)]).view(np.uint16)[0]
    import torch
    vals = torch.tensor(rng.standard_normal(5000).astype(np.float32) * 10.0 ** rng.integers(-4, 3, 5000))
    vals = torch.cat([vals, torch.tensor([448.0, 464.0, 465.0, 479.0, 480.0, 2 ** -9, 2 ** -10, 0.0])])
    ref = vals.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.f32_to_e4m3(vals.numpy())
    assert np.array_equal(got, ref)
    assert np.array_equal(O.e4m3_to_f32(np.arange(256, dtype=np.uint8)[:127]),
                          torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy())
