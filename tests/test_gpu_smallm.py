"""GPU parity of the weight-streaming paths for few activation rows against the oracle: INT8
weight-only (the VALU GEMV for one or two rows, the small-M MFMA kernel up to 16 rows) and
W4A8 / W6A8 (the small-M int8 MFMA kernel with the decode in the load stage, up to 32 rows; its
int32 GEMM and epilogue replayed exactly).

Bar: relative Frobenius error < 1e-3 and max-abs error < 2e-2 of a float64 linear over the same
dequantized operands (the rotated activation and q * scale).  Shapes cover the reference's
small-M probe (bench/probe_small_m.py:31-47: one token against K = N = 3072, and the range
edge cases of :84-101) and long rows (K up to 13824), ragged N and every output dtype.
"""
import numpy as np
import pytest
import torch

import oracle as O
from a8_check import check_a8_activation_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REL_TOL, ABS_TOL = 1e-3, 2e-2


def qlin():
    import qlin as Q
    return Q


def check(got, want, what):
    got = got.double().cpu().numpy()
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max())
    assert np.isfinite(got).all(), what
    assert rel < REL_TOL and mx < ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


def int8_weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.clamp(torch.round(torch.randn(n, k, generator=g) * 40), -127, 127).to(torch.int8)
    s = (torch.rand(n, generator=g) * 2e-4 + 2e-4)
    return q, s


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize("k,n,g", [(1024, 200, 0), (3072, 3072, 128), (5120, 1000, 256), (13824, 77, 128)])
def test_int8_linear_small_m(m, k, n, g):
    q, s = int8_weight(n, k, seed=m + k)
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(m)) * 2).half()
    b = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).float()
    Q = qlin()
    y = Q.int8_linear(x.to(DEV), q.to(DEV), s.to(DEV), b.to(DEV), convrot=bool(g), convrot_groupsize=g or 256)
    assert y.shape == (m, n) and y.dtype == torch.float16
    xr = O.rotate(x.float().numpy(), g) if g else x.float().numpy()
    want = O.linear_ref(xr, O.dequantize_int8(q.numpy(), s.numpy()), b.numpy())
    check(y, want, f"M={m} K={k} N={n} G={g}")


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("g", [64, 128, 256])
@pytest.mark.parametrize("m,k", [(1, 1024), (1, 3072), (1, 5120), (1, 8192), (2, 3072), (2, 4096)])
def test_int8_gemv_fused_prologue_matches_prologue_kernel(m, k, g, xdt):
    """One or two fp16 / bf16 rows with a rotation: the GEMV rotates and normalizes them itself.
    The same rows in a view whose row stride is not a multiple of 8 take the prologue kernel and
    the plain GEMV instead; both paths must give the same output bit for bit (the normalized
    operand and the exponent come from the same arithmetic), and both meet the oracle's bar."""
    n = 520
    q, s = int8_weight(n, k, seed=k + g)
    gen = torch.Generator().manual_seed(k + m)
    x = (torch.randn(m, k, generator=gen) * 3)
    x[:, 5] = 900.0  # a large value: the row exponent differs from 0
    x = x.to(xdt)
    b = (torch.randn(n, generator=gen) * 0.1).half()
    Q = qlin()
    xd = x.to(DEV)
    padded = torch.zeros(m, k + 4, dtype=xdt, device=DEV)
    padded[:, :k] = xd
    xs = padded[:, :k]
    assert xs.stride(0) % 8 != 0
    args = (q.to(DEV), s.to(DEV), b.to(DEV))
    y_fused = Q.int8_linear(xd, *args, convrot=True, convrot_groupsize=g)
    y_plain = Q.int8_linear(xs, *args, convrot=True, convrot_groupsize=g)
    torch.cuda.synchronize()
    assert torch.equal(y_fused, y_plain), f"M={m} K={k} G={g} {xdt}: fused and prologue paths differ"
    y32 = Q.int8_linear(xd, *args, torch.float32, convrot=True, convrot_groupsize=g)
    want = O.linear_ref(O.rotate(x.float().numpy(), g), O.dequantize_int8(q.numpy(), s.numpy()), b.float().numpy())
    check(y32, want, f"fused M={m} K={k} G={g} {xdt}")
    # the default output dtype is the input's: the same fp32 value, rounded once (RNE)
    assert torch.equal(y_fused, y32.to(xdt)), f"M={m} K={k} G={g} {xdt}: output rounding differs"


@pytest.mark.parametrize("xdt,odt,sdt", [(torch.bfloat16, torch.bfloat16, torch.float16),
                                         (torch.float32, torch.float32, torch.float32),
                                         (torch.float16, torch.float32, torch.float16)])
@pytest.mark.parametrize("m", [1, 3, 12])
def test_int8_linear_small_m_dtypes(xdt, odt, sdt, m):
    n, k = 300, 2048
    q, s = int8_weight(n, k, seed=7)
    s = s.to(sdt)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(11)).to(xdt)
    Q = qlin()
    y = Q.int8_linear(x.to(DEV), q.to(DEV), s.to(DEV), None, odt, convrot=True, convrot_groupsize=256)
    assert y.dtype == odt
    want = O.linear_ref(O.rotate(x.float().numpy(), 256), O.dequantize_int8(q.numpy(), s.float().numpy()))
    if odt == torch.bfloat16:  # one bf16 rounding of the output
        rb = torch.from_numpy(want.astype(np.float32)).bfloat16().double().numpy()
        assert O.rel_fro(y.double().cpu().numpy(), rb) < 1e-3
    else:
        check(y, want, f"M={m} {xdt} -> {odt}, scale {sdt}")


def test_int8_linear_small_m_strided_and_scalar_scale():
    """A row-strided activation view, a scalar scale and batched leading dimensions."""
    n, k = 130, 3072
    q, s = int8_weight(n, k, seed=9)
    Q = qlin()
    xs = torch.randn(3, k + 64, generator=torch.Generator().manual_seed(1)).half()[:, 64:]
    s1 = torch.tensor([3e-4])
    y = Q.int8_linear(xs.to(DEV), q.to(DEV), s1.to(DEV), convrot=True, convrot_groupsize=128)
    want = O.linear_ref(O.rotate(xs.float().numpy(), 128), O.dequantize_int8(q.numpy(), np.full(n, 3e-4, np.float32)))
    check(y, want, "strided x, scalar scale")
    x3 = torch.randn(2, 2, k, generator=torch.Generator().manual_seed(2)).half()
    y3 = Q.int8_linear(x3.to(DEV), q.to(DEV), s.to(DEV))
    y2 = Q.int8_linear(x3.reshape(4, k).to(DEV), q.to(DEV), s.to(DEV))
    assert y3.shape == (2, 2, n)
    torch.testing.assert_close(y3.reshape(4, n), y2, rtol=0, atol=0)


def test_int8_linear_small_m_extremes():
    """The reference's small-M range cases (bench/probe_small_m.py:84-101) at one token, K = 3072:
    a large dot product bound, huge / tiny / zero scales, 2^-26 inputs, the rotation growth of
    10000 * sign(H[:, 0]) and activations near the fp16 maximum."""
    Q = qlin()
    k, n = 3072, 64
    h = O.hadamard(128)
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    growth = np.tile(10000 * np.sign(h[:, 0]), k // 128).reshape(1, k).astype(np.float32)
    cases = [
        ("dot_bound", np.full((1, k), 100.0, np.float32), np.full((n, k), 127, np.int8), np.full(n, 1e-2, np.float32), 0),
        ("large_scale", rng.standard_normal((1, k)).astype(np.float32), q,
         np.tile(np.array([1e5, 3e7, 1e-30, 1e-3], np.float32), n // 4), 0),
        ("tiny_input", np.full((1, k), 2.0 ** -26, np.float32), q, np.full(n, 1e-3, np.float32), 128),
        ("zero_scale", rng.standard_normal((1, k)).astype(np.float32), q, np.zeros(n, np.float32), 128),
        ("rotation_growth", growth, q, np.full(n, 1e-3, np.float32), 128),
        ("near_max", np.full((1, k), 60000.0, np.float32), q, np.full(n, 1e-6, np.float32), 0),
    ]
    for name, x, qq, s, g in cases:
        got = Q.int8_linear(torch.from_numpy(x).to(DEV), torch.from_numpy(qq).to(DEV), torch.from_numpy(s).to(DEV),
                            None, torch.float32, convrot=bool(g), convrot_groupsize=g or 256).cpu().numpy()
        xr = O.rotate(x, g) if g else x
        want = O.linear_ref(xr, O.dequantize_int8(qq, s))
        den = max(float(np.abs(want).max()), 1e-30)
        assert np.isfinite(got).all(), name
        assert float(np.abs(got - want).max()) / den < 2e-3, f"{name}: max rel {float(np.abs(got - want).max()) / den}"


# ------------------------------------------------------------------------------------------------
# W4A8 / W6A8 for few rows: decode in the load stage, int8 MFMA, exact int32 sums
# ------------------------------------------------------------------------------------------------

def packed_weight(n, k, bits, gs, seed, srel_dtype, codebook):
    """Random legal codes packed in the storage format, group scales inside the int8 grid."""
    from qlin.quantize import FIXED_CODEBOOK, pack_codes
    g = torch.Generator().manual_seed(seed)
    lo_code = 0 if codebook else 1
    codes = torch.randint(lo_code, (15 if bits == 4 else 63) + 1, (n, k), generator=g, dtype=torch.int32)
    if codebook:
        lo, hi = 60.0, 127.0     # codebook levels lie in [-1, 1]
    else:
        lo, hi = (8.0, 18.0) if bits == 4 else (2.0, 4.1)
    s_rel = (lo + (hi - lo) * torch.rand(n, k // gs, generator=g)).to(srel_dtype)
    s_ch = (torch.rand(n, generator=g) * 2e-4 + 1e-4).float()
    cb = torch.from_numpy(FIXED_CODEBOOK.copy()) if codebook else None
    return pack_codes(codes, bits), s_rel, s_ch, cb


A8_SMALL = [
    (4, 128, torch.float16, False, 1024),
    (4, 16, torch.float8_e4m3fn, True, 3072),
    (6, 64, torch.float16, False, 5120),
    (6, 32, torch.bfloat16, False, 13824),
    (4, 64, torch.float32, True, 13824),
]


@pytest.mark.parametrize("bits,gs,srdt,cb,k", A8_SMALL)
@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 32])
def test_w4a8_linear_small_m(bits, gs, srdt, cb, k, m):
    n, g = 200, 128
    q, s_rel, s_ch, book = packed_weight(n, k, bits, gs, seed=m + k + bits, srel_dtype=srdt, codebook=cb)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m))
    x = torch.where(torch.rand(m, k, generator=torch.Generator().manual_seed(m + 1)) < 0.01, 20.0 * torch.sign(x), x)
    x = x.half()
    b = (torch.randn(n, generator=torch.Generator().manual_seed(4)) * 0.1).float()
    dev = lambda t: None if t is None else t.to(DEV)
    Q = qlin()
    y = Q.w4a8_int8_linear(x.to(DEV), dev(q), dev(s_rel), dev(s_ch), dev(book), None, dev(b), gs, g)
    assert y.shape == (m, n)
    if srdt == torch.float8_e4m3fn:
        sr32 = O.srel_to_f32(s_rel.view(torch.uint8).numpy(), "e4m3")
    else:
        sr32 = s_rel.float().numpy()
    w8 = O.w4a8_int8_grid(q.numpy(), sr32, None if book is None else book.numpy(), k, bits, gs)
    xq, sx = check_a8_activation_rows(Q, x.to(DEV), g, np.arange(m), f"w{bits}a8 M={m} K={k}: activations")
    xq, sx = xq.cpu().numpy(), sx.cpu().numpy().reshape(-1)
    # exact replay of the int32 GEMM and the epilogue ((f32(acc) * sx) * s_channel) + bias
    acc = O.int8_gemm_i64(xq, w8)
    replay = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * s_ch.numpy()[None, :]).astype(np.float32)
    replay = (replay + b.numpy()[None, :]).astype(np.float32)
    got = y.cpu().numpy()
    bad = got.view(np.uint16) != replay.astype(np.float16).view(np.uint16)
    assert not bad.any(), f"{int(bad.sum())} outputs differ from the exact replay, first at {np.argwhere(bad)[:3].tolist()}"
    want = O.linear_ref(xq.astype(np.float32) * sx[:, None], w8.astype(np.float32) * s_ch.numpy()[:, None],
                        b.numpy())
    check(y, want, f"w{bits}a8 gs={gs} M={m} K={k}")
