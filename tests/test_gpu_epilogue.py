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


def _separate(Q, linear, res, rs, odt):
    """The linear in fp32, then the residual epilogue kernel: the reference bits for the fused call."""
    from qlin import _lib
    base = linear(torch.float32)
    y = torch.empty(base.shape, dtype=odt, device=DEV)
    st = _lib.load().qlin_residual_epilogue(_lib.desc(base), _lib.desc(res), _lib.desc(rs), _lib.desc(y),
                                            _lib.stream_of(base.device))
    _lib.check(st, "qlin_residual_epilogue")
    return y


@pytest.mark.parametrize("m,n,k", [
    (2048, 5120, 1024),   # 160 tiles of 256 x 256: the LDS-DMA GEMM
    (2600, 6100, 512),    # 264 tiles: rows 0..2559 on 256 x 256 tiles, the last 40 on 128 x 256 tiles
    (1000, 2560, 1024),   # register-staged 128 x 128 tiles, a ragged M
    (100, 512, 1024),     # the DMA-ring kernel (a few hundred rows)
    (5, 512, 1024),       # small M: the linear in fp32, then the residual kernel
])
@pytest.mark.parametrize("odt,rdt", [(torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_int8_residual_fused_equals_separate(m, n, k, odt, rdt):
    """The residual applied in the GEMM epilogue gives the bits of the fp32 linear followed by the
    residual kernel (the same fma and rounding); small M takes that second route itself."""
    Q = qlin()
    g = torch.Generator().manual_seed(m + n)
    q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(DEV)
    s = (torch.rand(n, generator=g) * 1e-3).to(DEV)
    x = torch.randn(m, k, generator=g).half().to(DEV)
    b = torch.randn(n, generator=g).half().to(DEV)
    res = (torch.randn(m, n, generator=g) * 3).to(rdt).to(DEV)
    rs = torch.linspace(-2, 2, n).to(rdt).to(DEV)
    y = Q.int8_linear(x, q, s, b, odt, convrot=True, convrot_groupsize=128, residual=res, residual_scale=rs)
    want = _separate(Q, lambda dt: Q.int8_linear(x, q, s, b, dt, convrot=True, convrot_groupsize=128), res, rs, odt)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"M={m} N={n}: fused != separate"


@pytest.mark.parametrize("m,n,k,bits,gs", [
    (1024, 4096, 1024, 4, 64),   # grid decoded once, then the int8 DMA GEMM (128 x 256 tiles)
    (2600, 6100, 512, 6, 64),    # 264 tiles of 256 x 256: the last 40 rows on 128 x 256 tiles
    (1000, 5100, 1024, 6, 64),   # the same with 2 x 5 waves on 128 x 160 tiles (256 of them)
    (300, 24600, 1024, 6, 64),   # one 256-row tile over a wide grid: the fused-decode GEMM
    (100, 1000, 1024, 4, 16),    # group 16: the 128 x 128 decode-in-load kernel, residual kernel after
    (8, 512, 1024, 6, 64),       # small M
])
def test_w4a8_residual_fused_equals_separate(m, n, k, bits, gs):
    from qlin.quantize import pack_codes
    Q = qlin()
    g = torch.Generator().manual_seed(m + n + bits)
    hi = 15 if bits == 4 else 63
    q = pack_codes(torch.randint(1, hi + 1, (n, k), generator=g, dtype=torch.int32), bits).to(DEV)
    s_rel = (2 + 2 * torch.rand(n, k // gs, generator=g)).half().to(DEV)
    s_ch = (torch.rand(n, generator=g) * 2e-4 + 1e-4).to(DEV)
    x = torch.randn(m, k, generator=g).half().to(DEV)
    b = torch.randn(n, generator=g).half().to(DEV)
    res = (torch.randn(m, n, generator=g) * 3).half().to(DEV)
    rs = torch.linspace(-2, 2, n).half().to(DEV)
    args = (x, q, s_rel, s_ch, None, None, b, gs, 256)
    y = Q.w4a8_int8_linear(*args, residual=res, residual_scale=rs)
    want = _separate(Q, lambda dt: Q.w4a8_int8_linear(*args, out_dtype=dt), res, rs, torch.float16)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"w{bits}a8 M={m} N={n}: fused != separate"


@pytest.mark.parametrize("name,m,n,k", [
    ("Q4_K", 100, 1000, 2048),  # split kernel, m-tiles, 8 splits: the reduction applies it
    ("Q4_0", 64, 1000, 2048),   # split kernel, 8 splits
    ("Q8_0", 65, 1000, 2048),   # split kernel, two m-tiles (the second one row)
    ("Q5_K", 512, 4096, 1024),  # split kernel, 256 tiles, one split: the kernel's own epilogue
    ("Q6_K", 600, 1000, 2048),  # the GEMM over the decoded weight
    ("Q6_K", 300, 1000, 2048),  # split kernel, 5 m-tiles
    ("IQ4_XS", 8, 1000, 2048),  # small-M kernel, then the residual kernel
])
def test_gguf_residual_fused_equals_separate(name, m, n, k):
    """From 17 to 512 rows (Q6_K from 3) the split kernel, or its reduction, applies the residual;
    above, the GEMM over the decoded weight; fewer rows take the weight-streaming kernels and the
    residual kernel after them.  Every route gives the bits of the separate residual kernel."""
    Q = qlin()
    raw = torch.from_numpy(random_gguf_blocks(name, n, k, seed=m)).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half().to(DEV)
    b = torch.randn(n, generator=torch.Generator().manual_seed(1)).to(DEV)
    res = torch.randn(m, n, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    y = Q.gguf_linear(x, raw, name, (n, k), b, torch.bfloat16, residual=res)
    want = _separate(Q, lambda dt: Q.gguf_linear(x, raw, name, (n, k), b, dt), res, None, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16)), f"{name} M={m}: fused != separate"
