"""Unmerged LoRA (lora_down / lora_up / lora_scale) on the three quantized linears, on the GPU.

Reference semantics (roblennon/mac-kernels-public tests/test_lora_sidepath.py:80-91,
tests/test_gguf_node.py:110-174): the output equals the linear over the dequantized base weight
plus delta = scale * up @ down, applied to the caller's activation (before ConvRot).  Checked here:
  - the side term y(lora) - y(base) against the exact float64 product scale * (x down^T) up^T,
    within the reference's bar: 2 eps(out dtype) * max|y| + 2e-3 * max|side|;
  - the whole output against the oracle's float64 linear plus that product, within 1e-3 relative
    Frobenius and 2e-2 max-abs error;
  - the reference's overflow case (a merged delta of 2 from factors 4e4 and 2.5e-5) to the bit.
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def qlin():
    import qlin as Q
    return Q


def qz():
    from qlin import quantize as QZ
    return QZ


def factors(n, k, r, dt_down, dt_up, seed=5):
    g = torch.Generator().manual_seed(seed)
    up = (torch.randn(n, r, generator=g) * 0.05).to(dt_up)
    down = (torch.randn(r, k, generator=g) * 0.05).to(dt_down)
    return down, up


def side_ref(x, down, up, scale):
    x64 = x.double().cpu().numpy().reshape(-1, x.shape[-1])
    return scale * (x64 @ down.double().numpy().T) @ up.double().numpy().T


def check_side(y_lora, y_base, ref, what):
    eps = torch.finfo(y_lora.dtype).eps
    got = y_lora.float().cpu().numpy().reshape(ref.shape).astype(np.float64)
    base = y_base.float().cpu().numpy().reshape(ref.shape).astype(np.float64)
    assert np.isfinite(got).all(), what
    tol = 2 * eps * float(np.abs(got).max()) + 2e-3 * float(np.abs(ref).max())
    err = float(np.abs((got - base) - ref).max())
    assert err <= tol, f"{what}: side error {err:.3e} > {tol:.3e}"


def check_full(y, want, what):
    got = y.float().cpu().numpy().reshape(want.shape).astype(np.float64)
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max())
    assert rel < 1e-3 and mx < 2e-2, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


@pytest.mark.parametrize("m,r,xdt,fdt", [(64, 16, torch.bfloat16, torch.bfloat16), (37, 1, torch.float16, torch.float16),
                                         (300, 64, torch.bfloat16, torch.float32), (5, 200, torch.float16, torch.bfloat16)])
def test_int8_convrot_lora(m, r, xdt, fdt):
    Q = qlin()
    n, k, g = 384, 512, 256
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(0)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, g)
    q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(sn).reshape(-1).to(DEV)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(1)) * 0.5).to(xdt)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(2)) * 0.1).half().to(DEV)
    down, up = factors(n, k, r, fdt, fdt)
    base = Q.int8_linear(x.to(DEV), q, s, b, convrot=True, convrot_groupsize=g)
    y = Q.int8_linear(x.to(DEV), q, s, b, convrot=True, convrot_groupsize=g,
                      lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.8)
    assert y.dtype == xdt and y.shape == (m, n)
    ref = side_ref(x, down, up, 0.8)
    check_side(y, base, ref, f"int8 m={m} r={r}")
    if xdt == torch.float16:
        wdq = O.dequantize_int8_convrot(qn, sn, g)  # original basis, so x enters unrotated
        want = O.linear_ref(x.float().numpy(), wdq) + b.double().cpu().numpy()[None, :] + ref
        check_full(y, want, "int8 full")


@pytest.mark.parametrize("bits,m", [(4, 48), (6, 1100), (6, 3)])
def test_w4a8_lora(bits, m):
    Q = qlin()
    n, k, g, gs = 256, 1024, 256, 64
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(3)) * 0.02).numpy()
    q, s_rel, s_ch, book = qz().quantize_w4a8_int8_weight(w, bits=bits, group_size=gs, convrot_groupsize=g,
                                                          codebook=None, s_rel_dtype=torch.float16)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(4)).half()
    down, up = factors(n, k, 32, torch.bfloat16, torch.bfloat16)
    dev = lambda t: t.to(DEV)
    base = Q.w4a8_int8_linear(dev(x), dev(q), dev(s_rel), dev(s_ch), None, None, None, gs, g)
    y = Q.w4a8_int8_linear(dev(x), dev(q), dev(s_rel), dev(s_ch), None, None, None, gs, g,
                           lora_down=dev(down), lora_up=dev(up), lora_scale=1.5)
    check_side(y, base, side_ref(x, down, up, 1.5), f"w{bits}a8 m={m}")


@pytest.mark.parametrize("name,m", [("Q4_K", 1), ("Q4_K", 8), ("Q8_0", 64), ("Q6_K", 5), ("IQ4_XS", 130)])
def test_gguf_lora(name, m):
    Q = qlin()
    n, k = 192, 512
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(6)) * 0.02).numpy()
    raw = torch.from_numpy(qz().quantize_gguf(w, name)).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(7)).half()
    down, up = factors(n, k, 16, torch.float16, torch.bfloat16)
    base = Q.gguf_linear(x.to(DEV), raw, name, (n, k))
    y = Q.gguf_linear(x.to(DEV), raw, name, (n, k), lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.5)
    ref = side_ref(x, down, up, 0.5)
    check_side(y, base, ref, f"{name} m={m}")
    wdq = O.gguf_dequantize(raw.cpu().numpy(), name, (n, k))
    check_full(y, O.linear_ref(x.float().numpy(), wdq) + ref, f"{name} full")


@pytest.mark.parametrize("odt", [torch.float32, torch.float16])
def test_lora_fp32_activations(odt):
    """fp32 x and the fp32 output path of the up kernel (no y prefetch), odd N and M."""
    Q = qlin()
    n, k, g, m = 200, 512, 256, 45
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(8)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, g)
    q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(sn).reshape(-1).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(9))
    down, up = factors(n, k, 24, torch.float32, torch.float32, seed=10)
    base = Q.int8_linear(x.to(DEV), q, s, None, odt, convrot=True, convrot_groupsize=g)
    y = Q.int8_linear(x.to(DEV), q, s, None, odt, convrot=True, convrot_groupsize=g,
                      lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.7)
    assert y.dtype == odt
    ref = side_ref(x, down, up, 0.7)
    check_side(y, base, ref, f"fp32 x, {odt} out")
    wdq = O.dequantize_int8_convrot(qn, sn, g)
    check_full(y, O.linear_ref(x.numpy(), wdq) + ref, "fp32 full")


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("large_down", [False, True])
def test_lora_large_factors_exact(xdt, large_down):
    """tests/test_gguf_node.py:139-165: Q8_0 [3, 32] with zero codes, x = 1, up and down of 4e4 and
    2.5e-5 (either way round), strength 2: every output is exactly 64 (fp16 factors or an fp16
    intermediate would overflow or round away from it)."""
    Q = qlin()
    packed = torch.zeros(3, 34, dtype=torch.uint8)
    packed[:, :2] = torch.tensor([0.02], dtype=torch.float16).view(torch.uint8)
    up_value, down_value = (0.000025, 40000.) if large_down else (40000., 0.000025)
    up = torch.full((3, 1), up_value)
    down = torch.full((1, 32), down_value)
    x = torch.ones(2, 32, dtype=xdt, device=DEV)
    y = Q.gguf_linear(x, packed.to(DEV), "Q8_0", (3, 32), lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=2.0)
    assert y.dtype == xdt and torch.isfinite(y).all()
    torch.testing.assert_close(y.cpu(), torch.full((2, 3), 64.0, dtype=xdt), rtol=0, atol=0)


def test_lora_arguments():
    Q = qlin()
    n, k = 64, 256
    q = torch.zeros(n, k, dtype=torch.int8, device=DEV)
    s = torch.ones(n, device=DEV)
    x = torch.randn(3, k, device=DEV).half()
    down = torch.randn(8, k, device=DEV).half() * 0.1
    up = torch.randn(n, 8, device=DEV).half() * 0.1
    base = Q.int8_linear(x, q, s)
    # lora_scale None means 1.0; non-contiguous factors are accepted
    y1 = Q.int8_linear(x, q, s, lora_down=down, lora_up=up)
    yt = Q.int8_linear(x, q, s, lora_down=down.t().contiguous().t(), lora_up=up.t().contiguous().t(), lora_scale=1.0)
    torch.testing.assert_close(y1, yt, rtol=0, atol=0)
    check_side(y1, base, side_ref(x.cpu(), down.cpu().float(), up.cpu().float(), 1.0), "scale None")
    with pytest.raises(ValueError):
        Q.int8_linear(x, q, s, lora_down=down)
    with pytest.raises(ValueError):
        Q.int8_linear(x, q, s, lora_down=down, lora_up=up[:, :4])
    with pytest.raises(ValueError):
        Q.int8_linear(x, q, s, lora_scale=0.5)
    # empty activations
    e = Q.int8_linear(torch.empty(0, k, device=DEV).half(), q, s, lora_down=down, lora_up=up)
    assert e.shape == (0, n)


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 4, 200])
def test_lora_cancelling_the_weight_is_exactly_zero(odt, m):
    """The base and LoRA terms are summed in fp32 and rounded once into a 16-bit y
    (docs/upstream/comfy-kitchen-mps-backend.md:54-56): a LoRA equal to minus the weight gives
    exactly 0 even where the base output itself is not representable in the output dtype, and a
    base beyond the 16-bit range that the LoRA brings back stays finite.  All operands are small
    integers, so both terms are exact in fp32 and only the order of rounding can matter."""
    k, n = 64, 48
    g = torch.Generator().manual_seed(m)
    x = torch.randint(-7, 8, (m, k), generator=g).half()
    q = torch.randint(-100, 101, (n, k), generator=g).to(torch.int8)
    s = torch.ones(n)
    down = torch.eye(k).to(torch.bfloat16)            # t = x exactly
    Q = qlin()
    base = x.double() @ q.double().T
    assert (base.abs() > 2048).any(), "the case must hold outputs that round in 16 bits"
    y = Q.int8_linear(x.to(DEV), q.to(DEV), s.to(DEV), None, odt, lora_down=down.to(DEV),
                      lora_up=(-q.float()).to(torch.bfloat16).to(DEV), lora_scale=1.0)
    assert y.dtype == odt and torch.count_nonzero(y).item() == 0
    # a base of about 1.9e5 (beyond fp16) brought back to x @ d^T by the LoRA term
    xb = torch.full((m, k), 30.0).half()
    d = torch.randint(-1, 2, (n, k), generator=g)
    qb = torch.full((n, k), 100, dtype=torch.int8)
    yb = Q.int8_linear(xb.to(DEV), qb.to(DEV), s.to(DEV), None, odt, lora_down=down.to(DEV),
                       lora_up=(d.float() - 100.0).to(torch.bfloat16).to(DEV), lora_scale=1.0)
    want = (xb.double() @ d.double().T).to(odt)
    assert torch.isfinite(yb.float()).all()
    assert torch.equal(yb.cpu(), want)


# ------------------------------------------------------------------------------------------------
# LoRA fused into the large-M GEMMs (qlin_int8_linear_lora / qlin_w4a8_linear_lora): the GEMM adds
# scale * t up^T to its own output tile after the bias and rounds once.  A zero residual keeps the
# same single rounding through the separate kernels (fp32 base, LoRA, residual epilogue), so the
# two paths are compared output for output, besides the reference's bars.
# ------------------------------------------------------------------------------------------------

@pytest.fixture
def fused_calls(monkeypatch):
    """The outcomes of the wrapper's fused attempts for calls with a LoRA, in order: True where the
    GEMM carried the LoRA term, False where the call took the separate kernels."""
    from qlin import ops
    seen = []
    real = ops._fused_lora

    def spy(op, lora, *a):
        ran = real(op, lora, *a)
        if lora is not None:
            seen.append(ran)
        return ran

    monkeypatch.setattr(ops, "_fused_lora", spy)
    return seen


def _close_or_equal(fused, plain, what):
    """The fused GEMM adds (scale t) up^T into the base inside its MFMAs, the separate kernels form
    base + scale (t up^T): the same terms with fp32 roundings in another order (a few fp32 ulps
    apart), rounded once to the output dtype.  So the outputs agree to the rounding step of the
    output dtype (two steps at a power of two) plus 1e-5 of the output's scale for results that
    cancel towards 0."""
    f, p = fused.float(), plain.float()
    eps = torch.finfo(fused.dtype).eps
    diff = (f - p).abs()
    lim = 2 * eps * torch.maximum(f.abs(), p.abs()) + 1e-5 * p.abs().max()
    worst = (diff - lim).max().item()
    assert worst <= 0, f"{what}: fused and separate LoRA differ beyond the output rounding (excess {worst:.3e})"


@pytest.mark.parametrize("r,fdt,xdt", [(64, torch.bfloat16, torch.bfloat16), (16, torch.float16, torch.float16),
                                       (48, torch.float32, torch.bfloat16), (8, torch.bfloat16, torch.float32),
                                       (128, torch.bfloat16, torch.bfloat16), (72, torch.float16, torch.float16),
                                       (120, torch.float32, torch.bfloat16)])
def test_int8_lora_fused_into_gemm(r, fdt, xdt, fused_calls):
    """M2048 N5120: 160 tiles of 256 x 256, the GEMM that carries the LoRA term; ranks above 64
    in two passes over the tile."""
    Q = qlin()
    m, n, k, g = 2048, 5120, 1024, 128
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(20)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, g)
    q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(sn).reshape(-1).to(DEV)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(21)) * 0.5).to(xdt).to(DEV)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(22)) * 0.1).half().to(DEV)
    down, up = factors(n, k, r, fdt, fdt, seed=23)
    kw = dict(convrot=True, convrot_groupsize=g, lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.8)
    base = Q.int8_linear(x, q, s, b, convrot=True, convrot_groupsize=g)
    y = Q.int8_linear(x, q, s, b, **kw)
    plain = Q.int8_linear(x, q, s, b, residual=torch.zeros(m, n, dtype=y.dtype, device=DEV), **kw)
    torch.cuda.synchronize()
    assert fused_calls == [True, False]
    _close_or_equal(y, plain, f"int8 r={r} {fdt}")
    ref = side_ref(x.cpu(), down, up, 0.8)
    check_side(y, base, ref, f"int8 fused r={r} {fdt}")
    rows = torch.tensor([0, 1000, m - 1])
    wdq = O.dequantize_int8_convrot(qn, sn, g)
    want = O.linear_ref(x.cpu()[rows].float().numpy(), wdq) + b.double().cpu().numpy()[None, :] + ref[rows.numpy()]
    if xdt != torch.bfloat16:
        check_full(y[rows.to(DEV)], want, f"int8 fused full r={r}")


@pytest.mark.parametrize("bits,m,n,r,fdt", [
    (4, 2048, 6144, 64, torch.bfloat16),   # 8 x 24 = 192 tiles of 256 x 256
    (6, 2304, 6144, 32, torch.float32),    # 9 x 24 = 216 tiles of 256 x 256, fp32 up factors
    (6, 2048, 4096, 32, torch.float16),    # 128 x 256 tiles (128 of 256 x 256 would not fill the GPU)
    (4, 1024, 2048, 64, torch.bfloat16),   # 128 x 128 tiles
    (6, 1100, 1024, 32, torch.float32),    # 128 x 64 tiles (fewer than 128 tiles of 128 x 128)
    (4, 200, 2048, 16, torch.bfloat16),    # 128 x 64 tiles, a few hundred rows
    (4, 2048, 6144, 128, torch.bfloat16),  # 256 x 256 tiles, rank 128 in two passes of 64
    (6, 2048, 4096, 96, torch.float16),    # 128 x 256 tiles, passes of 64 and 32
    (6, 1024, 2048, 64, torch.float32),    # 128 x 128 tiles, fp32 up factors in passes of 32
])
def test_w4a8_lora_fused_into_gemm(bits, m, n, r, fdt, fused_calls):
    """A8 calls whose weight grid is decoded once (from 512 rows, and above 32 rows on grids of fewer
    than 192 tiles of 256 x 256), then the DMA GEMM that carries the LoRA term, at each of its tile
    shapes: 256 x 256 from 192 such tiles, else 128 x 256, 128 x 128 or 128 x 64."""
    Q = qlin()
    k, g, gs = 1024, 256, 64
    gen = torch.Generator().manual_seed(30 + bits)
    hi = 15 if bits == 4 else 63
    codes = torch.randint(1, hi + 1, (n, k), generator=gen, dtype=torch.int32)
    q = qz().pack_codes(codes, bits).to(DEV)
    lo, top = (8.0, 18.0) if bits == 4 else (2.0, 4.1)
    s_rel = (lo + (top - lo) * torch.rand(n, k // gs, generator=gen)).half().to(DEV)
    s_ch = (torch.rand(n, generator=gen) * 2e-4 + 1e-4).float().to(DEV)
    x = torch.randn(m, k, generator=gen).half().to(DEV)
    down, up = factors(n, k, r, fdt, fdt, seed=31)
    args = (x, q, s_rel, s_ch, None, None, None, gs, g)
    kw = dict(lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=1.5)
    base = Q.w4a8_int8_linear(*args)
    y = Q.w4a8_int8_linear(*args, **kw)
    plain = Q.w4a8_int8_linear(*args, residual=torch.zeros(m, n, dtype=torch.float16, device=DEV), **kw)
    torch.cuda.synchronize()
    assert fused_calls == [True, False]
    _close_or_equal(y, plain, f"w{bits}a8 m={m} r={r}")
    check_side(y, base, side_ref(x.cpu(), down, up, 1.5), f"w{bits}a8 fused m={m} r={r}")


@pytest.mark.parametrize("name,m,n,k,r,fdt", [
    ("Q4_K", 64, 4096, 4096, 64, torch.bfloat16),  # the decode shape: 32 row blocks x 8 splits
    ("Q6_K", 40, 1000, 2048, 128, torch.float16),  # ragged N, rank 128 in two passes
    ("Q8_0", 200, 4096, 1024, 32, torch.float32),  # four m-tiles (the last 8 rows), 2 splits, fp32 up
    ("Q4_0", 512, 4096, 1024, 16, torch.bfloat16), # 256 tiles: one split without the LoRA, two with it
    ("IQ4_XS", 17, 520, 512, 8, torch.bfloat16),   # one m-tile of 17 rows, a ragged column block
    ("Q2_K", 100, 136, 1024, 24, torch.bfloat16),  # 16-value units, 2 m-tiles
    ("Q6_K", 48, 4096, 2048, 64, torch.float16),   # t by the split kernel: 2 ranks per column, 4 splits
    ("Q5_K", 40, 4096, 4096, 32, torch.float32),   # t by the split kernel, fp32 down, 1 rank per column
    ("Q4_1", 24, 1024, 2048, 8, torch.bfloat16),   # t by the split kernel: 32-row m-tile
    ("Q4_K", 100, 4096, 2048, 64, torch.float16),  # t by the split kernel over 2 m-tiles
    ("Q8_0", 48, 4096, 4096, 128, torch.bfloat16), # 4 ranks per column: the separate down kernel
])
def test_gguf_lora_fused_into_split(name, m, n, k, r, fdt, fused_calls):
    """GGUF calls from 17 rows to the split kernel's limit: the K-split reduction adds the LoRA term
    to each 64 x 128 output tile before its one rounding (the reference's GGUF LoRA in the epilogue,
    to rank 128).  With 4 or more splits and at most 2 ranks per column of the grid, the split kernel also
    forms t = x down^T from the activation slices it stages (its K-split partials summed in the
    reduction); otherwise the separate down kernel does.  Against the separate kernels, the exact
    side term and the oracle's linear."""
    Q = qlin()
    from gguf_blocks import random_gguf_blocks
    raw = random_gguf_blocks(name, n, k, seed=m + r)
    rd = torch.from_numpy(raw).to(DEV)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(m)) * 0.5).half()
    b = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).half().to(DEV)
    down, up = factors(n, k, r, fdt, fdt, seed=r)
    kw = dict(lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.7)
    base = Q.gguf_linear(x.to(DEV), rd, name, (n, k), b)
    y = Q.gguf_linear(x.to(DEV), rd, name, (n, k), b, **kw)
    plain = Q.gguf_linear(x.to(DEV), rd, name, (n, k), b, residual=torch.zeros(m, n, dtype=y.dtype, device=DEV), **kw)
    torch.cuda.synchronize()
    assert fused_calls == [True, False]
    _close_or_equal(y, plain, f"{name} m={m} r={r}")
    ref = side_ref(x, down, up, 0.7)
    check_side(y, base, ref, f"{name} fused m={m} r={r}")
    want = O.linear_ref(x.float().numpy(), O.gguf_dequantize(raw, name, (n, k)), b.double().cpu().numpy()) + ref
    check_full(y, want, f"{name} fused full m={m} r={r}")


@pytest.mark.parametrize("m,r", [(64, 64), (24, 16), (200, 32)])
def test_gguf_lora_fused_graph_replays(m, r, fused_calls):
    """A fused GGUF LoRA call captured in a HIP graph and replayed with new activations, eager calls
    (their own workspace) between the replays: every replay equals the eager call bit for bit (the
    split kernel's t partials at 64 and 24 rows, the separate down kernel at 200; sums in a fixed
    order either way)."""
    Q = qlin()
    from gguf_blocks import random_gguf_blocks
    name, n, k = "Q4_K", 4096, 2048
    rd = torch.from_numpy(random_gguf_blocks(name, n, k, seed=71)).to(DEV)
    down, up = factors(n, k, r, torch.bfloat16, torch.bfloat16, seed=72)
    down, up = down.to(DEV), up.to(DEV)
    xs = [(torch.randn(m, k, generator=torch.Generator().manual_seed(73 + i)) * 0.5).half().to(DEV) for i in range(3)]
    xin = xs[0].clone()
    kw = dict(lora_down=down, lora_up=up, lora_scale=0.6)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        Q.gguf_linear(xin, rd, name, (n, k), **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg = Q.gguf_linear(xin, rd, name, (n, k), **kw)
    torch.cuda.synchronize()
    for i in range(6):
        xin.copy_(xs[i % 3])
        g.replay()
        torch.cuda.synchronize()
        got = yg.clone()
        want = Q.gguf_linear(xs[i % 3], rd, name, (n, k), **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager call"
    assert all(fused_calls)


@pytest.mark.parametrize("name,m,r", [("Q4_K", 16, 16), ("Q4_K", 600, 16), ("Q4_K", 64, 136), ("Q6_K", 520, 16),
                                      ("Q4_K", 64, 12)])
def test_gguf_lora_declines_to_the_separate_kernels(name, m, r, fused_calls):
    """16 rows or fewer (the GEMV and small-M kernels), past the split kernel's 512 rows (the GEMM
    over the decoded weight), rank above 128 or not a multiple of 8: the fused entry
    point declines before launching and the separate kernels give the result."""
    Q = qlin()
    from gguf_blocks import random_gguf_blocks
    n, k = 256, 1024
    rd = torch.from_numpy(random_gguf_blocks(name, n, k, seed=9)).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(10)).half()
    down, up = factors(n, k, r, torch.bfloat16, torch.bfloat16, seed=11)
    base = Q.gguf_linear(x.to(DEV), rd, name, (n, k))
    y = Q.gguf_linear(x.to(DEV), rd, name, (n, k), lora_down=down.to(DEV), lora_up=up.to(DEV), lora_scale=0.5)
    torch.cuda.synchronize()
    assert fused_calls == ([] if m <= 16 else [False])
    check_side(y, base, side_ref(x, down, up, 0.5), f"{name} m={m} r={r}")


@pytest.mark.parametrize("r,fdt", [(12, torch.bfloat16), (136, torch.bfloat16), (72, torch.float32)])
def test_lora_fused_declines_to_the_separate_kernels(r, fdt, fused_calls):
    """Ranks the GEMM epilogue does not take at a fused shape (not a multiple of 8; above 128; fp32 up
    factors above 64 in the A8 GEMM): the fused entry point declines before launching and the
    separate LoRA kernels give the result."""
    Q = qlin()
    m, n, k = 2048, 5120, 512
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(41)).half()
    down, up = factors(n, k, r, fdt, fdt, seed=42)
    dd, ud = down.to(DEV), up.to(DEV)
    from qlin import _lib
    L = _lib.load()
    if fdt == torch.float32:
        # the INT8 GEMM takes fp32 up factors to rank 128; the A8 GEMM's LDS holds 32 at a time
        codes = torch.randint(1, 16, (n, k), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
        qp = qz().pack_codes(codes, 4).to(DEV)
        s_rel = torch.full((n, k // 64), 10.0, dtype=torch.float16, device=DEV)
        s_ch = torch.full((n,), 1e-4, device=DEV)
        args = (x.to(DEV), qp, s_rel, s_ch, None, None, None, 64, 0)
        base = Q.w4a8_int8_linear(*args)
        y = Q.w4a8_int8_linear(*args, lora_down=dd, lora_up=ud, lora_scale=0.5)
        nb = L.qlin_workspace_size(_lib.OP_W4A8_LINEAR_LORA, m, n, k, r, _lib.DT_F16)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        st = L.qlin_w4a8_linear_lora(_lib.desc(x.to(DEV)), _lib.desc(qp), _lib.desc(s_rel), _lib.desc(s_ch), None,
                                     None, _lib.desc(torch.empty_like(y)), 4, 64, 0, _lib.desc(dd), _lib.desc(ud),
                                     0.5, ws.data_ptr(), ws.numel(), _lib.stream_of(ws.device))
    else:
        q = torch.randint(-100, 101, (n, k), generator=torch.Generator().manual_seed(40)).to(torch.int8).to(DEV)
        s = torch.full((n,), 1e-3, device=DEV)
        base = Q.int8_linear(x.to(DEV), q, s)
        y = Q.int8_linear(x.to(DEV), q, s, lora_down=dd, lora_up=ud, lora_scale=0.5)
        nb = L.qlin_workspace_size(_lib.OP_INT8_LINEAR_LORA, m, n, k, r, _lib.DT_F16)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        st = L.qlin_int8_linear_lora(_lib.desc(x.to(DEV)), _lib.desc(q), _lib.desc(s), None,
                                     _lib.desc(torch.empty_like(y)), 0, _lib.desc(dd), _lib.desc(ud),
                                     0.5, ws.data_ptr(), ws.numel(), _lib.stream_of(ws.device))
    assert fused_calls == [False]
    check_side(y, base, side_ref(x, down, up, 0.5), f"r={r} {fdt} at a fused shape")
    assert st == _lib.QLIN_EUNSUPPORTED


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16])
def test_lora_fused_cancelling_the_weight_is_exactly_zero(odt, fused_calls):
    """The cancellation case at a shape the fused GEMM takes (M2048 N5120): base and LoRA terms meet
    in fp32 in the GEMM epilogue and round once, so a LoRA equal to minus the weight gives 0."""
    m, n, k = 2048, 5120, 64
    g = torch.Generator().manual_seed(50)
    x = torch.randint(-7, 8, (m, k), generator=g).half()
    q = torch.randint(-100, 101, (n, k), generator=g).to(torch.int8)
    Q = qlin()
    y = Q.int8_linear(x.to(DEV), q.to(DEV), torch.ones(n, device=DEV), None, odt,
                      lora_down=torch.eye(k).to(torch.bfloat16).to(DEV),
                      lora_up=(-q.float()).to(torch.bfloat16).to(DEV), lora_scale=1.0)
    assert fused_calls == [True]
    assert y.dtype == odt and torch.count_nonzero(y).item() == 0
