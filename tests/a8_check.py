"""Checks of the A8 activation leg against the oracle, shared by the GPU tests.

The reference quantizes A8 activations as quantize_int8_rowwise(rot(x)) (modal/weight_error_app.py:109-115;
the rotation x[:, group] @ H^T of :101-106 applied to activations as in bench/probe_small_m.py:51-56).
The GPU rotates in fp32 and rounds once to x's dtype; the oracle rotates exactly and rounds once,
so the two rotated rows may differ by one unit in the last place, rarely, or by the fp32 rounding
error of the butterflies where a value is far smaller than its group.  The quantization of the
GPU's rotated row must then equal the oracle's quantization of that same row bit for bit.
"""
import numpy as np
import torch

import oracle as O


def _ordered(bits16):
    """Sign-magnitude 16-bit float patterns as integers that step by one per ulp (+0 and -0 equal)."""
    b = bits16.astype(np.int32)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def exact_rotation_bits(x, g):
    """The exactly rotated rows of x (fp16 or bf16, CPU), rounded once to x's dtype, as uint16 bits.
    bf16 rows are rotated exactly by the oracle into fp32 and then rounded to bf16 (RNE): the fp32
    intermediate has 16 more bits than bf16, so this double rounding moves a value by at most the
    one-ulp slack the comparison allows."""
    if x.dtype == torch.float16:
        return O.rotate(x.numpy(), g).view(np.uint16)
    assert x.dtype == torch.bfloat16, x.dtype
    r32 = torch.from_numpy(O.rotate(x.float().numpy(), g))
    return r32.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _values(bits16, bf16):
    """float64 values of fp16 or bf16 bit patterns."""
    if bf16:
        return (bits16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits16.view(np.float16).astype(np.float64)


def _ulp(v, bf16):
    """Spacing of the fp16 / bf16 numbers at |v| (the subnormal spacing below the normal range)."""
    p, emin = (7, -126) if bf16 else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** emin)))
    return np.exp2(e - p)


def assert_rotation_close(x, xr, g, what, rare=1e-2):
    """xr (the GPU's rotated rows, CPU tensor of x's dtype) against the exact rotation of x rounded
    once (want).  The GPU's rotation is an fp32 FWHT: log2(G) butterfly stages whose partial sums
    are bounded by the group's L1 norm, then 1/sqrt(G) (one more rounding unless G is a power of 4).
    So before its final rounding it is within (log2 G + 1) 2^-24 |x_group|_1 / sqrt(G) of the exact
    value, and got and want may differ by one unit in the last place plus that bound; a value much
    smaller than its group (cancellation) can therefore be two or more ulps off.  Every value must
    be within one ulp or within that bound, and at most a fraction `rare` may differ at all."""
    bf16 = x.dtype == torch.bfloat16
    gb = xr.contiguous().view(torch.int16).numpy().view(np.uint16)
    wb = exact_rotation_bits(x.contiguous(), g)
    ulps = np.abs(_ordered(gb) - _ordered(wb))
    got, want = _values(gb, bf16), _values(wb, bf16)
    m, k = x.shape
    l1 = np.abs(x.float().numpy().astype(np.float64)).reshape(m, k // g, g).sum(-1)
    bound32 = np.repeat((np.log2(g) + 1) * 2.0 ** -24 * l1 / np.sqrt(g), g, axis=1)
    lim = bound32 + np.maximum(_ulp(got, bf16), _ulp(want, bf16))
    bad = (ulps > 1) & (np.abs(got - want) > lim)
    off = float((ulps > 0).mean())
    assert not bad.any() and off < rare, (
        f"{what}: {int(bad.sum())} rotated values beyond one ulp and the fp32 bound "
        f"(first at {np.argwhere(bad)[:3].tolist()}), fraction off by any ulp {off:.2e}")


def oracle_quantize(xr):
    """The oracle's quantize_int8_rowwise of rows xr (CPU tensor, fp16 / bf16 / fp32)."""
    xr = xr.contiguous()
    if xr.dtype == torch.bfloat16:
        return O.quantize_int8_rowwise(xr.view(torch.int16).numpy().view(np.uint16), bf16=True)
    return O.quantize_int8_rowwise(xr.numpy())


def assert_quantized_like_oracle(xr, q, s, what):
    """q int8 and s fp32 (CPU) equal the oracle's quantization of the rotated rows xr, bit for bit."""
    wq, ws = oracle_quantize(xr)
    qn = q.contiguous().numpy()
    sn = s.contiguous().numpy().reshape(-1)
    nq = int((qn != wq).sum())
    assert nq == 0, f"{what}: {nq} int8 codes differ from the oracle's, first at {np.argwhere(qn != wq)[:3].tolist()}"
    assert np.array_equal(sn.view(np.uint32), ws.reshape(-1).view(np.uint32)), f"{what}: row scales differ"


def check_a8_activation_rows(Q, xd, g, rows, what):
    """Runs quantize_int8_rowwise(xd, g, return_rotated=True) on the GPU and holds the rows `rows`
    to the oracle: the rotation within one ulp, codes and scales bit-exact.  Returns (q, s) of all
    rows, on the GPU, for the GEMM replay."""
    q, s, xr = Q.quantize_int8_rowwise(xd, g, return_rotated=True)
    rd = torch.as_tensor(rows, device=xd.device)
    x_rows = xd[rd].cpu()
    xr_rows = xr[rd].cpu()
    if g:
        assert_rotation_close(x_rows, xr_rows, g, what)
    else:
        assert torch.equal(x_rows, xr_rows), f"{what}: unrotated rows were changed"
    assert_quantized_like_oracle(xr_rows, q[rd].cpu(), s[rd].cpu(), what)
    return q, s.reshape(-1)
