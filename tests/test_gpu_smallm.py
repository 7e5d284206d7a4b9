"""GPU parity of the weight-streaming paths for few activation rows (INT8 weight-only: the VALU
GEMV for 1..4 rows, the small-M MFMA kernel up to 16 rows), against the oracle.

Bar: relative Frobenius error < 1e-3 and max-abs error < 2e-2 of a float64 linear over the same
dequantized operands (the rotated activation and q * scale).  Shapes cover the reference's
small-M probe (bench/probe_small_m.py:31-47: one token against K = N = 3072, and the range
edge cases of :84-101) and long rows (K up to 13824), ragged N and every output dtype.
"""
import numpy as np
import pytest
import torch

import oracle as O

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
