"""Seeded sweep of shapes around the dispatch boundaries of the three linears (GGUF, INT8-ConvRot,
W4A8 / W6A8): each case against the oracle's dequantized weight and a float64 matmul.

The shapes come from one fixed seed: activation rows on both sides of every switch point (1, 2,
16/17, 32/33, 64/65, 512/513, 2047/2049 and a few thousand, where the A8 pre-pass and the tail
split of 256 x 256 grids apply), weight rows ragged or whole 256-row tiles, and K over the formats'
block sizes.  The bar is the relative Frobenius error of the fp16 output (its own rounding is
about 3e-4 of it).
"""
import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TYPES = ["Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS"]
ROWS = [1, 2, 5, 16, 17, 32, 33, 64, 65, 129, 300, 512, 513, 1000, 2047, 2049, 2600, 4100]
REL_TOL = 2e-3


def _cases(seed=20261202, count=60, max_macs=4e9):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        kind = ("gguf", "int8", "a8")[len(out) % 3]
        m = int(rng.choice(ROWS))
        big = m >= 2047  # grids of 256 x 256 tiles past one round, some with a partial last round
        if big:
            n = 256 * int(rng.integers(8, 26)) + int(rng.choice([0, 8, 100]))
        else:
            n = int(rng.integers(1, 48)) * int(rng.choice([8, 16, 64, 128])) + int(rng.choice([0, 0, 4]))
        if kind == "gguf":
            t = TYPES[int(rng.integers(len(TYPES)))]
            qk = O.GGUF_TYPES[t][1]
            k = qk * int(rng.integers(1, max(2, (768 if big else 3072) // qk)))
            case = (kind, t, m, n, k)
        else:
            g = int(rng.choice([0, 128, 256]) if kind == "int8" else rng.choice([128, 256]))
            k = max(g, 128) * int(rng.integers(1 if g == 256 else 2, 4 if big else 12))
            case = (kind, g, m, n, k)
        if m * n * k <= max_macs:
            out.append(case)
    return out


def _rel(got, want):
    got, want = got.astype(np.float64), want.astype(np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "-".join(str(v) for v in c))
def test_shape_sweep(case):
    import qlin
    from qlin import quantize as QZ
    kind, var, m, n, k = case
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m * 31 + n)).half()
    rng = np.random.default_rng(n * 7 + k)
    if kind == "gguf":
        raw = random_gguf_blocks(var, n, k, seed=m + n)
        want = O.linear_ref(x.float().numpy(), O.gguf_dequantize(raw, var, (n, k)))
        got = qlin.gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), var, (n, k))
    elif kind == "int8":
        g = var
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        q, s = QZ.quantize_int8_convrot_weight(w, g) if g else QZ.quantize_int8_rowwise(w)
        xr = O.rotate(x.float().numpy(), g) if g else x.float().numpy()
        want = O.linear_ref(xr, O.dequantize_int8(q, s.astype(np.float32)))
        got = qlin.int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                               convrot=bool(g), convrot_groupsize=g or 256)
    else:
        g, bits, gs = var, 4 + 2 * (m % 2), 64 if k % 128 else 128
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        q, sr, sc, book = QZ.quantize_w4a8_int8_weight(w, bits=bits, group_size=gs, convrot_groupsize=g,
                                                        s_rel_dtype=torch.float16)
        got = qlin.w4a8_int8_linear(x.to(DEV), q.to(DEV), sr.to(DEV), sc.to(DEV),
                                    None if book is None else book.to(DEV), None, None, gs, g)
        # the oracle's product over the int8 operands the call multiplies: the activations as the
        # oracle quantizes the rotated rows, the weight grid as the oracle decodes it
        xq, sx = O.quantize_int8_rowwise(O.rotate(x.numpy(), g))
        w8 = O.w4a8_int8_grid(q.numpy(), sr.float().numpy(), None if book is None else book.numpy(), k, bits, gs)
        want = O.linear_ref(xq.astype(np.float32) * np.asarray(sx, np.float32).reshape(-1, 1),
                            w8.astype(np.float32) * sc.numpy()[:, None])
    got = got.float().cpu().numpy()
    assert got.shape == (m, n) and np.isfinite(got).all()
    r = _rel(got, want)
    assert r < REL_TOL, f"{case}: rel_fro {r:.3e}"
