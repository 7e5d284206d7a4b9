"""The residual epilogue and the layout carriers on the GPU.

Residual semantics (roblennon/mac-kernels-public tests/test_lora_sidepath.py:363-386): the output
is residual + residual_scale * (linear + bias [+ LoRA]), the bias first, then the scaled
residual add (docs/upstream/comfy-kitchen-mps-backend.md:52), rounded once.  Checked against the
oracle's float64 linear at the 1e-3 relative Frobenius / 2e-2 max-abs bar, for the three linears,
with LoRA, in every output dtype; integer cases check the single rounding exactly.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks
from a8_check import check_a8_activation_rows

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
HERE = os.path.dirname(os.path.abspath(__file__))


def qlin():
    import qlin as Q
    return Q


def qz():
    from qlin import quantize as QZ
    return QZ


def check(got, want, what):
    got = got.double().cpu().numpy()
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max())
    assert rel < 1e-3 and mx < 2e-2, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


@pytest.mark.parametrize("m", [1, 5, 300])
@pytest.mark.parametrize("rdt", [torch.float16, torch.float32])
def test_int8_linear_residual(m, rdt):
    n, k, g = 96, 1024, 128
    rng = np.random.default_rng(m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = qz().quantize_int8_convrot_weight(w, g)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half()
    b = torch.randn(n, generator=torch.Generator().manual_seed(2)) * 0.1
    res = (torch.randn(m, n, generator=torch.Generator().manual_seed(3)) * 2).to(rdt)
    rs = torch.full((n,), 0.5).to(rdt)
    y = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), b.to(DEV),
                           convrot=True, convrot_groupsize=g, residual=res.to(DEV), residual_scale=rs.to(DEV))
    lin = O.linear_ref(O.rotate(x.float().numpy(), g), O.dequantize_int8(q, s), b.numpy())
    want = res.double().numpy() + rs.double().numpy()[None, :] * lin
    assert y.dtype == torch.float16
    check(y, want, f"M={m} residual {rdt}")
    # without a scale the residual is added as is
    y1 = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), b.to(DEV),
                            convrot=True, convrot_groupsize=g, residual=res.to(DEV))
    check(y1, res.double().numpy() + lin, f"M={m} residual, no scale")


@pytest.mark.parametrize("name,m", [("Q4_K", 1), ("Q8_0", 8), ("Q6_K", 64), ("IQ4_XS", 100)])
def test_gguf_linear_residual_with_lora(name, m):
    """Bias, LoRA and residual together: residual + rs * (x W^T + b + scale x down^T up^T)."""
    n, k, r = 256, 1024, 16
    raw = random_gguf_blocks(name, n, k, seed=4)
    wdec = O.gguf_dequantize(raw, name, (n, k))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half()
    b = torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.1
    down = (torch.randn(r, k, generator=torch.Generator().manual_seed(6)) * 0.05).to(torch.bfloat16)
    up = (torch.randn(n, r, generator=torch.Generator().manual_seed(7)) * 0.05).to(torch.bfloat16)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    rs = torch.linspace(-1, 1, n).to(torch.bfloat16)
    y = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), b.to(DEV), torch.bfloat16,
                           down.to(DEV), up.to(DEV), 0.7, residual=res.to(DEV), residual_scale=rs.to(DEV))
    side = 0.7 * (x.double().numpy() @ down.double().numpy().T) @ up.double().numpy().T
    want = res.double().numpy() + rs.double().numpy()[None, :] * (O.linear_ref(x.float().numpy(), wdec, b.numpy()) + side)
    assert y.dtype == torch.bfloat16
    rb = torch.from_numpy(want.astype(np.float32)).bfloat16().double().numpy()  # one bf16 rounding
    assert O.rel_fro(y.double().cpu().numpy(), rb) < 1e-3


def test_w4a8_linear_residual_single_rounding():
    """Integer operands: the linear and the residual term are exact in fp32, so the output must be
    the exactly rounded sum; with the linear rounded to fp16 first it would not be."""
    m, n, k = 16, 64, 1024
    g = torch.Generator().manual_seed(1)
    codes = torch.randint(1, 16, (n, k), generator=g, dtype=torch.int32)
    from qlin.quantize import pack_codes
    q = pack_codes(codes, 4)
    s_rel = torch.full((n, k // 128), 16.0).half()        # grid = 16 * (code - 8), exact
    s_ch = torch.ones(n)
    x = torch.randint(-100, 101, (m, k), generator=g).half()
    Q = qlin()
    xq, sx = check_a8_activation_rows(Q, x.to(DEV), 0, np.arange(m), "A8 residual case: activations")
    w8 = Q.w4a8_int8_grid(q.to(DEV), s_rel.to(DEV), None, 128)
    acc = (xq.double() @ w8.double().T).cpu()
    lin = ((acc.float() * sx.cpu().reshape(-1, 1)) * s_ch[None, :])  # the A8 epilogue in fp32
    res = torch.full((m, n), 0.25).half()
    y = Q.w4a8_int8_linear(x.to(DEV), q.to(DEV), s_rel.to(DEV), s_ch.to(DEV), None, None, None, 128, 0,
                           residual=res.to(DEV), residual_scale=torch.full((n,), 3.0).half().to(DEV))
    # fp32 fma (the exact value rounded once to fp32, computed in float64), then the fp16 rounding
    want = (3.0 * lin.double() + res.double()).float().half()
    assert torch.equal(y.cpu(), want)
    # the linear alone rounded to fp16 first, then the residual, differs somewhere (the case is sharp)
    twice = (3.0 * lin.half().double() + res.double()).float().half()
    assert not torch.equal(twice, want)


@pytest.mark.parametrize("case", ["gauss_96x1024", "heavy_96x1024"])
def test_carriers_dispatch_to_the_ops(case):
    """QuantizedTensor carriers built from the reference's stored tensors dequantize and run the
    linear exactly as the ops on the plain tensors do."""
    from qlin.layouts import AsymW4A8Int8Layout, QuantizedTensor, TensorWiseINT8Layout, linear
    raw = np.load(os.path.join(HERE, "golden", "selftest_raw.npz"))
    Q = qlin()
    x = torch.randn(7, 1024, generator=torch.Generator().manual_seed(0)).half().to(DEV)
    q = torch.from_numpy(raw[f"{case}/int8_convrot/q"].copy().view(np.int8)).reshape(96, 1024).to(DEV)
    s = torch.from_numpy(raw[f"{case}/int8_convrot/scale"].copy().view(np.float32)).to(DEV)
    w = QuantizedTensor(q, "TensorWiseINT8Layout",
                        TensorWiseINT8Layout.Params(scale=s, orig_dtype=torch.float32, convrot=True,
                                                    convrot_groupsize=256))
    assert torch.equal(w.dequantize(), Q.dequantize_int8_convrot_weight(q, s, 256))
    assert torch.equal(linear(x, w), Q.int8_linear(x, q, s, convrot=True, convrot_groupsize=256))
    for fmt in ("w4a8", "w6a8"):
        qa = torch.from_numpy(raw[f"{case}/{fmt}/q"].copy().view(np.int8)).reshape(96, -1).to(DEV)
        sr = torch.from_numpy(raw[f"{case}/{fmt}/s_rel"].copy()).reshape(96, -1).view(torch.float8_e4m3fn).to(DEV)
        sc = torch.from_numpy(raw[f"{case}/{fmt}/s_channel"].copy().view(np.float32)).to(DEV)
        key = f"{case}/{fmt}/codebook"
        cb = torch.from_numpy(raw[key].copy().view(np.float32)).to(DEV) if key in raw.files else None
        wa = QuantizedTensor(qa, "AsymW4A8Int8Layout",
                             AsymW4A8Int8Layout.Params(scale=sr, s_channel=sc, codebook=cb, group_size=16,
                                                       convrot_groupsize=256, orig_dtype=torch.float32))
        assert torch.equal(wa.dequantize(), Q.dequantize_w4a8_int8_weight(qa, sr, sc, cb, None, 16, 256))
        assert torch.equal(linear(x, wa), Q.w4a8_int8_linear(x, qa, sr, sc, cb, None, None, 16, 256))
