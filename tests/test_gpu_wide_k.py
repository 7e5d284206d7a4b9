"""GPU parity of the three linears at contractions longer than one workgroup's rows (K > 32768).

The reference computes layers with K > 65504 (docs/upstream/comfy-kitchen-mps-backend.md:50, 112)
and tests them (:97).  Here the prologue takes such rows in 32768-value chunks, twice (the row's
max first, then the outputs), and the GEMMs accumulate in fp32 over normalized operands, so the
fp16 range is never the limit; the A8 int32 sums stay exact for K < 132104.

Each case runs at K = 65536 or 73728 through the kernel its row count selects (the small-M
kernels, the K-split and tiled GEMMs) and is held to the parity bar against the oracle's float64
linear over the same dequantized operands: relative Frobenius error < 1e-3, max-abs < 2e-2.  The
A8 activation quantization is bit-exact against the oracle, and the A8 linear equals an exact
replay of its int8 GEMM and epilogue.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks
from a8_check import check_a8_activation_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REL_TOL, ABS_TOL = 1e-3, 2e-2


def qlin():
    import qlin as Q
    return Q


def qz():
    from qlin import quantize as QZ
    return QZ


def check(got, want, what):
    got = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else got
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max())
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert rel < REL_TOL and mx < ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


def rows_of(m):
    return np.unique(np.array([0, m // 3, m // 2, m - 1], dtype=np.int64))


@pytest.mark.parametrize("m", [1, 4, 40, 300])
@pytest.mark.parametrize("k,g,xdt", [(65536, 128, torch.float16), (73728, 256, torch.bfloat16),
                                     (65536, 0, torch.float32)])
def test_int8_linear_wide_k(m, k, g, xdt):
    n = 96
    gen = torch.Generator().manual_seed(k + m + g)
    w = (torch.randn(n, k, generator=gen) * 0.005).numpy()  # outputs of order 1 over 65536 terms
    q, s = qz().quantize_int8_convrot_weight(w, g) if g else qz().quantize_int8_rowwise(w)
    s = s.astype(np.float32).reshape(-1)
    x = (torch.randn(m, k, generator=gen) * 2).to(xdt)
    b = (torch.randn(n, generator=gen) * 0.1).float()
    y = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), b.to(DEV),
                           torch.float32, convrot=bool(g), convrot_groupsize=g or 256)
    rows = rows_of(m)
    xr = x[torch.from_numpy(rows)].float().numpy()
    if g:
        xr = O.rotate(xr, g)
    want = O.linear_ref(xr, O.dequantize_int8(q, s), b.numpy())
    check(y[torch.from_numpy(rows).to(DEV)], want, f"int8 M={m} K={k} G={g} {xdt}")


@pytest.mark.parametrize("name", ["Q4_K", "Q8_0", "Q6_K", "IQ4_XS"])
@pytest.mark.parametrize("m", [1, 8, 40, 100])
def test_gguf_linear_wide_k(name, m):
    n, k = 64, 65536
    raw = random_gguf_blocks(name, n, k, seed=m + 7)
    wdq = O.gguf_dequantize(raw, name, (n, k))
    # |w| ~ 0.02-0.05: activations of 0.5 keep outputs of order 10 over 65536 terms
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(m)) * 0.5).half()
    y = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), out_dtype=torch.float32)
    rows = rows_of(m)
    want = O.linear_ref(x[torch.from_numpy(rows)].float().numpy(), wdq)
    check(y[torch.from_numpy(rows).to(DEV)], want, f"{name} M={m} K={k}")


@pytest.mark.parametrize("m", [4, 40, 1100])
@pytest.mark.parametrize("bits,gs", [(4, 128), (6, 64)])
def test_w4a8_linear_wide_k(m, bits, gs):
    """Up to 32 rows: the small-M int8 kernel; 40: the 128 x 128 decode-in-load kernel; 1100: the
    grid decoded once, then the int8 DMA GEMM."""
    n, k, g = 64, 65536, 128
    gen = torch.Generator().manual_seed(m + bits)
    hi = 15 if bits == 4 else 63
    codes = torch.randint(1, hi + 1, (n, k), generator=gen, dtype=torch.int32)
    q = qz().pack_codes(codes, bits)
    lo, top = (8.0, 18.0) if bits == 4 else (2.0, 4.1)
    s_rel = (lo + (top - lo) * torch.rand(n, k // gs, generator=gen)).half()
    s_ch = (torch.rand(n, generator=gen) * 2e-4 + 1e-4).float()
    x = torch.randn(m, k, generator=gen).half()
    Q = qlin()
    xd, qd, srd, scd = x.to(DEV), q.to(DEV), s_rel.to(DEV), s_ch.to(DEV)
    y = Q.w4a8_int8_linear(xd, qd, srd, scd, None, None, None, gs, g)
    what = f"w{bits}a8 M={m} K={k}"
    w8 = O.w4a8_int8_grid(q.numpy(), s_rel.float().numpy(), None, k, bits, gs)
    rows = rows_of(m)
    rd = torch.from_numpy(rows).to(DEV)
    xq, sx = check_a8_activation_rows(Q, xd, g, rows, what + ": activation quantization")
    acc = xq.double() @ torch.from_numpy(w8).to(DEV).double().T  # exact: |acc| < 2^53
    replay = ((acc.float() * sx[:, None]) * scd[None, :]).half()
    nbad = int((y.view(torch.int16) != replay.view(torch.int16)).sum().item())
    assert nbad == 0, f"{what}: {nbad} outputs differ from the exact replay"
    acc_o = O.int8_gemm_i64(xq[rd].cpu().numpy(), w8)
    assert np.array_equal(acc[rd].cpu().numpy().astype(np.int64), acc_o), what + ": replay != int64 oracle"
    sxn = sx[rd].cpu().numpy()
    want = O.linear_ref(xq[rd].cpu().numpy().astype(np.float32) * sxn[:, None],
                        w8.astype(np.float32) * s_ch.numpy()[:, None])
    check(y[rd], want, what)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_act_int8_wide_k_bit_exact(dt):
    """quantize_int8_rowwise over 73728-value rows (three 32768-value chunks), with a zero row and a
    tiny row: the two-pass prologue gives the oracle's codes and scales bit for bit."""
    m, k = 6, 73728
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(3)) * 3
    x[2] = 0.0
    x[3] = x[3] * 1e-6
    x[4, k - 1] = 900.0  # the row max in the last chunk
    x = x.to(dt)
    q, s = qlin().quantize_int8_rowwise(x.to(DEV))
    if dt == torch.bfloat16:
        wq, ws = O.quantize_int8_rowwise(x.view(torch.int16).numpy().view(np.uint16), bf16=True)
    else:
        wq, ws = O.quantize_int8_rowwise(x.numpy())
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), ws.reshape(-1).view(np.uint32))


# Past the A8 linear's exact int32 range (K < 132104) the weight-only linears go on: their fp16
# MFMAs accumulate in fp32 over normalized operands, and the prologue takes any number of chunks.

@pytest.mark.parametrize("m,k,g,xdt", [(1, 196608, 256, torch.float16), (4, 196608, 128, torch.bfloat16),
                                       (40, 196608, 256, torch.float16), (300, 196608, 0, torch.float32),
                                       (40, 1 << 20, 256, torch.float16)])
def test_int8_linear_wider_than_a8(m, k, g, xdt):
    n = 64
    gen = torch.Generator().manual_seed(k + m + g)
    w = (torch.randn(n, k, generator=gen) * 0.002).numpy()  # outputs of order 1 over the long rows
    q, s = qz().quantize_int8_convrot_weight(w, g) if g else qz().quantize_int8_rowwise(w)
    s = s.astype(np.float32).reshape(-1)
    x = (torch.randn(m, k, generator=gen) * 2).to(xdt)
    y = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), None,
                           torch.float32, convrot=bool(g), convrot_groupsize=g or 256)
    rows = rows_of(m)
    xr = x[torch.from_numpy(rows)].float().numpy()
    if g:
        xr = O.rotate(xr, g)
    check(y[torch.from_numpy(rows).to(DEV)], O.linear_ref(xr, O.dequantize_int8(q, s)), f"int8 M={m} K={k} G={g}")


@pytest.mark.parametrize("name,m,k", [("Q4_K", 1, 196608), ("Q4_K", 8, 196608), ("Q8_0", 40, 196608),
                                      ("Q6_K", 100, 196608), ("IQ4_XS", 600, 196608), ("Q4_K", 8, 1 << 20)])
def test_gguf_linear_wider_than_a8(name, m, k):
    """One row and 8 rows (the small-M kernel: the GEMV stops at K = 8192), the K split, the
    m-tiles, and above 512 rows the weight decoded once to fp16 (25 MB here)."""
    n = 64
    raw = random_gguf_blocks(name, n, k, seed=m + 11)
    wdq = O.gguf_dequantize(raw, name, (n, k))
    x = (torch.randn(m, k, generator=torch.Generator().manual_seed(m)) * 0.25).half()
    y = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), out_dtype=torch.float32)
    rows = rows_of(m)
    want = O.linear_ref(x[torch.from_numpy(rows)].float().numpy(), wdq)
    check(y[torch.from_numpy(rows).to(DEV)], want, f"{name} M={m} K={k}")


def test_a8_declines_past_its_exact_range():
    """W4A8 at K = 132096 (its int32 sums could overflow): declined before launching, as a backend
    that cannot take the call."""
    n, k, gs = 8, 132096, 64
    q = torch.zeros(n, k // 2, dtype=torch.uint8, device=DEV)
    s_rel = torch.ones(n, k // gs, dtype=torch.float16, device=DEV)
    s_ch = torch.ones(n, device=DEV)
    x = torch.zeros(2, k, dtype=torch.float16, device=DEV)
    with pytest.raises(qlin().NoCapableBackendError):
        qlin().w4a8_int8_linear(x, q, s_rel, s_ch, None, None, None, gs, 256)


@pytest.mark.parametrize("k,g", [(65536, 256), (196608, 128)])
def test_dequantize_int8_convrot_wide(k, g):
    """The original-basis dequantization of rows longer than 32768 values (the rotation in chunks)."""
    n = 4
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(k)) * 0.02).numpy()
    q, s = qz().quantize_int8_convrot_weight(w, g)
    got = qlin().dequantize_int8_convrot_weight(torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                                                g).cpu().numpy()
    want = O.dequantize_int8_convrot(q, s.reshape(-1), g)
    assert np.abs(got.astype(np.float64) - want).max() <= 1e-6 * np.abs(want).max() + 1e-12
