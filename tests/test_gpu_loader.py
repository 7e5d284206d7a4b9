"""Files to HBM on the GPU (qlin.loader): staged copies arrive byte-identical (small staging
chunks make every tensor take many turns of both pinned buffers), and layers built from the files
compute exactly what the ops compute on the same operands."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import gguf_file as G
import oracle as O
import qlin
from qlin import quantize as QZ

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def conf_tensor(conf):
    import json
    return torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)


@pytest.mark.parametrize("chunk", [4096, 1 << 20, 32 << 20])
def test_safetensors_to_hbm(tmp_path, chunk):
    n, k, g = 384, 1024, 256
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(0)) * 0.02).numpy()
    qn, sn = QZ.quantize_int8_convrot_weight(w, g)
    q4, s_rel, s_ch, book = QZ.quantize_w4a8_int8_weight(w, bits=4, group_size=16, convrot_groupsize=g,
                                                         codebook=None, s_rel_dtype=torch.float8_e4m3fn)
    state = {
        "a.weight": torch.from_numpy(qn), "a.weight_scale": torch.from_numpy(sn).reshape(-1),
        "a.bias": torch.randn(n).half(),
        "a.comfy_quant": conf_tensor({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": g}),
        "b.weight": q4.view(torch.int8), "b.weight_s_rel": s_rel, "b.weight_s_channel": s_ch,
        "b.comfy_quant": conf_tensor({"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": g}),
        "odd": torch.arange(12345, dtype=torch.uint8),
    }
    if book is not None:
        state["b.weight_codebook"] = book
    path = tmp_path / "m.safetensors"
    save_file(state, str(path))
    loaded = qlin.load_safetensors(str(path), device=DEV, chunk=chunk)
    for key, v in state.items():
        want_dev = "cpu" if key.endswith("comfy_quant") else "cuda"
        assert loaded[key].device.type == want_dev, key
        assert torch.equal(loaded[key].cpu().view(torch.uint8), v.contiguous().view(torch.uint8)), key
    layers = qlin.quantized_linears(loaded)
    x = torch.randn(37, k, generator=torch.Generator().manual_seed(1)).half().to(DEV)
    ya = layers["a"](x)
    want = qlin.int8_linear(x, torch.from_numpy(qn).to(DEV), torch.from_numpy(sn).reshape(-1).to(DEV),
                            state["a.bias"].to(DEV), convrot=True, convrot_groupsize=g)
    torch.testing.assert_close(ya, want, rtol=0, atol=0)
    yb = layers["b"](x)
    want = qlin.w4a8_int8_linear(x, q4.to(DEV), s_rel.to(DEV), s_ch.to(DEV),
                                 None if book is None else book.to(DEV), None, None, 16, g)
    torch.testing.assert_close(yb, want, rtol=0, atol=0)


@pytest.mark.parametrize("chunk", [4096, 32 << 20])
def test_gguf_to_hbm(tmp_path, chunk):
    n, k = 256, 1024
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(2)) * 0.02).numpy()
    q4k, q6k = QZ.quantize_gguf(w, "Q4_K"), QZ.quantize_gguf(w, "Q6_K")
    # ComfyUI-GGUF's converter stores some tensors reshaped to rows of whole blocks and records
    # the torch shape: [3, 512] stored as [48, 32], and [4, 48] (rows straddle blocks) as [6, 32]
    reshaped = QZ.quantize_gguf(w[:3, :512].reshape(48, 32), "Q8_0")
    straddle = QZ.quantize_gguf(w[:4, :48].reshape(6, 32), "Q8_0")
    bias = np.linspace(-1, 1, n, dtype=np.float32)
    tensors = [("l.q4k", [k, n], 12, q4k.tobytes()), ("l.q6k", [k, n], 14, q6k.tobytes()),
               ("l.bias", [n], 0, bias.tobytes()), ("reshaped", [32, 48], 8, reshaped.tobytes()),
               ("straddle", [32, 6], 8, straddle.tobytes())]
    kv = [("comfy.gguf.orig_shape.reshaped", G.ARRAY, [3, 512], G.I32),
          ("comfy.gguf.orig_shape.straddle", G.ARRAY, [4, 48], G.I32)]
    path = tmp_path / "m.gguf"
    G.write_gguf(str(path), kv, tensors, alignment=64)
    out, _ = qlin.load_gguf(str(path), device=DEV, chunk=chunk)
    assert np.array_equal(out["l.q4k"].tensors["data"].cpu().numpy(), q4k.reshape(n, -1))
    assert np.array_equal(out["l.q6k"].tensors["data"].cpu().numpy(), q6k.reshape(n, -1))
    assert out["l.bias"].device.type == "cuda"
    assert np.array_equal(out["l.bias"].cpu().numpy(), bias)
    x = torch.randn(9, k, generator=torch.Generator().manual_seed(3)).half().to(DEV)
    for name, raw, qt in (("l.q4k", q4k, "Q4_K"), ("l.q6k", q6k, "Q6_K")):
        y = out[name](x)
        want = qlin.gguf_linear(x, torch.from_numpy(raw).to(DEV), qt, (n, k))
        torch.testing.assert_close(y, want, rtol=0, atol=0)
    # the decodes index the bytes by flat element, so both equal the oracle's decode of the stored rows
    for name, raw, shape in (("reshaped", reshaped, (3, 512)), ("straddle", straddle, (4, 48))):
        t = out[name]
        assert (t.out_features, t.in_features) == shape
        want = O.gguf_dequantize(raw, "Q8_0", (raw.size // 34, 32)).reshape(shape)
        np.testing.assert_array_equal(t.dequantize().cpu().numpy(), want)
    xs = torch.randn(5, 512, generator=torch.Generator().manual_seed(4)).half().to(DEV)
    torch.testing.assert_close(out["reshaped"](xs), qlin.gguf_linear(xs, torch.from_numpy(reshaped).to(DEV), "Q8_0",
                                                                    (3, 512)), rtol=0, atol=0)
