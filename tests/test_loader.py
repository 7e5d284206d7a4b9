"""Readers of the on-disk formats (qlin.loader), on the host: safetensors files written by the
safetensors library itself, and GGUF files built byte by byte from the format layout
(tests/gguf_file.py).  Checked: every tensor's bytes, dtype and shape come back unchanged; config
tensors stay on the host; the file is not modified; layer records are built from `comfy_quant`;
malformed files are rejected.  Device copies are covered in test_gpu_loader.py."""
import hashlib
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import gguf_file as G
import oracle as O
import qlin
from qlin import quantize as QZ
from qlin.exceptions import NoCapableBackendError


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def conf_tensor(conf):
    return torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)


def test_safetensors_int8_roundtrip(tmp_path):
    # the reference's direct-load fixture (tests/test_mps_pread_load.py:24-30)
    state = {
        "layer.weight": torch.arange(1024, dtype=torch.int32).remainder(255).sub(127).to(torch.int8).reshape(4, 256),
        "layer.weight_scale": torch.tensor([.001, .002, .003, .004]),
        "layer.comfy_quant": conf_tensor({"format": "int8_tensorwise", "convrot": False}),
    }
    path = tmp_path / "quant.safetensors"
    save_file(state, str(path), metadata={"description": "direct-load contract"})
    before = sha(path)
    loaded, meta = qlin.load_safetensors(str(path), device="cpu", return_metadata=True)
    assert meta == {"description": "direct-load contract"}
    for k, v in state.items():
        assert loaded[k].dtype == v.dtype and torch.equal(loaded[k], v), k
    assert json.loads(loaded["layer.comfy_quant"].numpy().tobytes()) == {"format": "int8_tensorwise", "convrot": False}
    layers = qlin.quantized_linears(loaded)
    lin = layers["layer"]
    assert (lin.kind, lin.out_features, lin.in_features) == ("int8", 4, 256)
    assert lin.params == {"convrot": False, "convrot_groupsize": 256}
    assert lin.tensors["qdata"].data_ptr() == loaded["layer.weight"].data_ptr()  # no copy
    assert sha(path) == before


@pytest.mark.parametrize("fmt,bits,gs", [("asym_w4a8_int8", 4, 16), ("w6a8_int8", 6, 32)])
def test_safetensors_w4a8_layer(tmp_path, fmt, bits, gs):
    # tests/test_h3_scale_ownership.py:24-29: I8 codes, F8_E4M3 s_rel, F32 s_channel and codebook
    n, k = 64, 256
    source = {
        "blk.weight": torch.randint(-128, 128, (n, k * bits // 8), dtype=torch.int8, generator=torch.Generator().manual_seed(0)),
        "blk.weight_s_rel": torch.rand(n, k // gs, generator=torch.Generator().manual_seed(1)).to(torch.float8_e4m3fn),
        "blk.weight_s_channel": torch.rand(n),
        "blk.weight_codebook": torch.linspace(-1, 1, 16),
        "blk.bias": torch.randn(n).half(),
        "blk.comfy_quant": conf_tensor({"format": fmt, "group_size": gs, "convrot_groupsize": 256}),
    }
    path = tmp_path / "h3.safetensors"
    save_file(source, str(path))
    loaded = qlin.load_safetensors(str(path), device="cpu")
    for key, v in source.items():
        assert loaded[key].dtype == v.dtype
        assert torch.equal(loaded[key].view(torch.uint8), v.view(torch.uint8)), key
    lin = qlin.quantized_linears(loaded)["blk"]
    assert (lin.kind, lin.out_features, lin.in_features, lin.params["bits"]) == ("w4a8", n, k, bits)
    assert lin.params["group_size"] == gs and "codebook" in lin.tensors and lin.bias is not None


def test_safetensors_keys_and_errors(tmp_path):
    path = tmp_path / "a.safetensors"
    save_file({"a": torch.arange(6, dtype=torch.float32), "b": torch.ones(2, 2, dtype=torch.bfloat16)}, str(path))
    only = qlin.load_safetensors(str(path), device="cpu", keys=["b"])
    assert list(only) == ["b"] and torch.equal(only["b"], torch.ones(2, 2, dtype=torch.bfloat16))
    with pytest.raises(KeyError):
        qlin.load_safetensors(str(path), device="cpu", keys=["c"])
    raw = open(path, "rb").read()
    (hlen,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + hlen])

    def rewrite(h, tail=None):
        hb = json.dumps(h).encode()
        p = tmp_path / "bad.safetensors"
        p.write_bytes(struct.pack("<Q", len(hb)) + hb + (raw[8 + hlen:] if tail is None else tail))
        return str(p)

    bad = dict(header)
    bad["b"] = dict(header["b"], data_offsets=[0, 8])  # overlaps "a" and has the wrong size
    with pytest.raises(ValueError):
        qlin.load_safetensors(rewrite(bad), device="cpu")
    bad = dict(header)
    bad["a"] = dict(header["a"], dtype="Q4")
    with pytest.raises(ValueError):
        qlin.load_safetensors(rewrite(bad), device="cpu")
    with pytest.raises(ValueError):  # data cut short
        qlin.load_safetensors(rewrite(header, raw[8 + hlen:-4]), device="cpu")
    p = tmp_path / "short.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40))
    with pytest.raises(ValueError):
        qlin.safetensors_header(str(p))


def test_unsupported_formats_decline(tmp_path):
    state = {"l.weight": torch.zeros(4, 8, dtype=torch.int8), "l.comfy_quant": conf_tensor({"format": "mxfp4"})}
    with pytest.raises(NoCapableBackendError):
        qlin.quantized_linears(state)
    state = {"l.weight": torch.zeros(4, 64, dtype=torch.int8), "l.weight_s_rel": torch.ones(4, 8),
             "l.weight_s_channel": torch.ones(4), "l.weight_correction": torch.zeros(8, 4),
             "l.comfy_quant": conf_tensor({"format": "asym_w4a8_int8", "group_size": 16})}
    with pytest.raises(NoCapableBackendError):
        qlin.quantized_linears(state)
    state["l.weight"] = torch.zeros(4, 60, dtype=torch.int8)  # not 4-bit codes for K = 128
    del state["l.weight_correction"]
    with pytest.raises(ValueError):
        qlin.quantized_linears(state)


def gguf_fixture(tmp_path, alignment=32):
    w = (torch.randn(3, 512, generator=torch.Generator().manual_seed(3)) * 0.02).numpy()
    q4k = QZ.quantize_gguf(w, "Q4_K")
    # tests/test_gguf_node.py:144-174: Q8_0 [3, 32], zero codes, d = 0.02
    q8 = np.zeros((3, 34), np.uint8)
    q8[:, :2] = np.array([0.02], np.float16).view(np.uint8)
    straddle = QZ.quantize_gguf((np.arange(96, dtype=np.float32).reshape(3, 32) - 48) / 50, "Q4_0")
    f32 = np.arange(5, dtype=np.float32)
    f16 = (np.arange(6, dtype=np.float16) / 3).reshape(2, 3)
    kv = [("general.architecture", G.STRING, "test"), ("general.file_type", G.U32, 15),
          ("general.weight", G.F32, 0.5), ("tags", G.ARRAY, ["a", "b"], G.STRING),
          ("comfy.gguf.orig_shape.straddle", G.ARRAY, [2, 48], G.I32)]
    tensors = [("blk.q4k.weight", [512, 3], 12, q4k.tobytes()), ("blk.q8.weight", [32, 3], 8, q8.tobytes()),
               ("straddle", [32, 3], 2, straddle.tobytes()), ("norm", [5], 0, f32.tobytes()),
               ("emb", [3, 2], 1, f16.tobytes())]
    path = tmp_path / "t.gguf"
    offs = G.write_gguf(str(path), kv, tensors, alignment)
    return str(path), offs, dict(q4k=q4k, q8=q8, straddle=straddle, f32=f32, f16=f16)


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_header_and_load(tmp_path, alignment):
    path, offs, src = gguf_fixture(tmp_path, alignment)
    before = sha(path)
    version, kv, infos, start = qlin.gguf_header(path)
    assert version == 3 and start % alignment == 0
    assert kv["general.architecture"] == "test" and kv["general.file_type"] == 15 and kv["general.weight"] == 0.5
    assert kv["tags"] == ["a", "b"] and kv["comfy.gguf.orig_shape.straddle"] == [2, 48]
    by = {i.name: i for i in infos}
    assert by["blk.q4k.weight"].shape == (3, 512) and by["blk.q4k.weight"].nbytes == 3 * 2 * 144
    assert by["straddle"].shape == (2, 48)  # orig_shape replaces the ggml dims
    for name, off in offs.items():
        assert start + by[name].offset == off
    out, kv2 = qlin.load_gguf(path, device="cpu")
    assert kv2 == kv
    q4k = out["blk.q4k.weight"]
    assert (q4k.kind, q4k.out_features, q4k.in_features, q4k.params["qtype"]) == ("gguf", 3, 512, "Q4_K")
    assert tuple(q4k.tensors["data"].shape) == (3, 288)
    assert np.array_equal(q4k.tensors["data"].numpy(), src["q4k"].reshape(3, 288))
    assert np.array_equal(out["blk.q8.weight"].tensors["data"].numpy(), src["q8"])
    s = out["straddle"]
    assert (s.out_features, s.in_features) == (2, 48) and s.tensors["data"].dim() == 1
    assert np.array_equal(s.tensors["data"].numpy(), src["straddle"].reshape(-1))
    # flat-index decode of the straddling rows equals the decode of the three whole-block rows
    np.testing.assert_array_equal(O.gguf_dequantize(s.tensors["data"].numpy(), "Q4_0", (2, 48)).reshape(-1),
                                  O.gguf_dequantize(src["straddle"], "Q4_0", (3, 32)).reshape(-1))
    assert torch.equal(out["norm"], torch.from_numpy(src["f32"]))
    assert out["emb"].dtype == torch.float16 and torch.equal(out["emb"], torch.from_numpy(src["f16"]))
    with pytest.raises(NoCapableBackendError):  # rows straddle blocks: the linear declines
        s(torch.zeros(1, 48))
    assert sha(path) == before


def test_gguf_rejects_malformed(tmp_path):
    path, offs, _ = gguf_fixture(tmp_path)
    raw = open(path, "rb").read()
    p = tmp_path / "bad.gguf"
    for blob in (b"GGUX" + raw[4:], raw[:4] + struct.pack("<I", 1) + raw[8:], raw[:40],
                 raw[:offs["emb"] + 4]):
        p.write_bytes(blob)
        with pytest.raises(ValueError):
            qlin.load_gguf(str(p), device="cpu")
    # a tensor whose values are not a whole number of blocks, and an unknown ggml type
    for dims, qt in (([40], 8), ([32], 16)):
        G.write_gguf(str(p), [], [("t", dims, qt, bytes(64))])
        with pytest.raises((ValueError, NoCapableBackendError)):
            qlin.load_gguf(str(p), device="cpu")
    # orig_shape that does not hold the tensor's values
    G.write_gguf(str(p), [("comfy.gguf.orig_shape.t", G.ARRAY, [3, 32], G.I32)], [("t", [32], 8, bytes(34))])
    with pytest.raises(ValueError):
        qlin.gguf_header(str(p))
