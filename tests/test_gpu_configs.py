"""GPU parity at the benchmark shapes, over the full contraction length.

The quantized-linear workloads this engine is measured on are, besides the GGUF decode-linear
(tests/test_gpu_parity.py::test_gguf_linear_decode_workload):
  - INT8-ConvRot weight-only, M256 K=N=3072, G=128, fp16 scales;
  - W4A8, M4096 K3072 N12288, group 128, fp16 group scales, 1% activation outliers at 20 sigma;
  - W6A8, M in {1024, 9504}, K5120 -> N13824 and K13824 -> N5120, group 64;
  - the INT8-ConvRot DiT block linears at 4608 tokens (QKV 3072->9216, O 3072->3072,
    MLP up 3072->12288, MLP down 12288->3072), G=128.
Each is run at its real shape, so every kernel's steady-state k-loop (stage reuse, alternating
register sets) runs 24..216 times.  Checks, per call:
  1. sampled output rows (every 256-row tile visited, first and last row included) against the
     oracle's float64 linear over the same dequantized operands (bench/probe_small_m.py:49 checks
     selected channels of large shapes the same way);
  2. the whole output against a float64 GEMM on the GPU over the oracle's operands (the weights
     dequantized by the oracle, the activations rotated by the oracle's Hadamard matrix);
  3. for A8, the activation leg against the oracle on the sampled rows (the rotated row within one
     ulp of the oracle's exact rotation, its int8 codes and fp32 scale bit-exact against the
     oracle's quantize_int8_rowwise), then an exact replay of the int8 GEMM and epilogue over the
     whole output: int8 x int8 products summed in float64 are exact (|acc| < 2^53), then
     (f32(acc) * sx) * s_channel in fp32 and one rounding, compared bit for bit; the float64
     accumulators of the sampled rows are checked against the oracle's int64 GEMM first.
Bar: relative Frobenius error < 1e-3 and max-abs error < 2e-2 against float64.

Mid-size cases run each large-tile kernel variant with at least 8 k-tiles per pipeline stage.
Random legal codes and scales stand in for the offline quantizer where it would take minutes
(the quantizer is pinned separately in tests/test_oracle_golden.py).
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


def qz():
    from qlin import quantize as QZ
    return QZ


def sample_rows(m, seed=0):
    """First and last row, and two rows of every 256-row tile (one random, one at the tile's end)."""
    rng = np.random.default_rng(seed)
    rows = {0, m - 1}
    for t0 in range(0, m, 256):
        t1 = min(m, t0 + 256)
        rows.add(int(rng.integers(t0, t1)))
        rows.add(t1 - 1)
    return np.array(sorted(rows), dtype=np.int64)


def randn(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def activations(m, k, seed, outliers=False):
    x = randn((m, k), seed)
    if outliers:
        g = torch.Generator().manual_seed(seed + 1000)
        mask = torch.rand(m, k, generator=g) < 0.01
        x = torch.where(mask, 20.0 * torch.sign(x), x)
    return x.half()


def bar(got64, want64, what):
    rel = O.rel_fro(got64, want64)
    mx = float(np.abs(got64 - want64).max())
    assert np.isfinite(got64).all(), f"{what}: non-finite output"
    assert rel < REL_TOL and mx < ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


def bar_gpu(got, want, what):
    """The same bar over whole outputs, computed on the GPU in float64."""
    got = got.double()
    assert torch.isfinite(got).all().item(), f"{what}: non-finite output"
    d = got - want
    den = torch.linalg.norm(want).item()
    rel = torch.linalg.norm(d).item() / (den if den > 0 else 1.0)
    mx = d.abs().max().item()
    assert rel < REL_TOL and mx < ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"


def rotate_gpu64(x16, g):
    """rot(x) in float64 on the GPU with the oracle's normalized Hadamard matrix."""
    m, k = x16.shape
    h = torch.from_numpy(O.hadamard(g)).to(DEV)
    return (x16.to(DEV).double().reshape(m, k // g, g) @ h.T.contiguous()).reshape(m, k)


# ------------------------------------------------------------------------------------------------
# INT8-ConvRot weight-only (fp16 MFMA)
# ------------------------------------------------------------------------------------------------

def int8_case(m, n, k, g, seed, scale_dtype=np.float16, bias=False):
    w = randn((n, k), seed, 0.02).numpy()
    q, s = qz().quantize_int8_convrot_weight(w, g)
    s = s.astype(scale_dtype)
    x = activations(m, k, seed + 1)
    b = randn((n,), seed + 2, 0.1).half() if bias else None
    Q = qlin()
    qd, sd = torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV)
    y = Q.int8_linear(x.to(DEV), qd, sd, None if b is None else b.to(DEV), convrot=True, convrot_groupsize=g)
    assert y.shape == (m, n) and y.dtype == torch.float16
    what = f"int8 G={g} M={m} N={n} K={k}"
    deq = O.dequantize_int8(q, s.astype(np.float32))
    bnp = None if b is None else b.float().numpy()
    rows = sample_rows(m, seed)
    xr = O.rotate(x[torch.from_numpy(rows)].float().numpy(), g)
    bar(y[torch.from_numpy(rows).to(DEV)].double().cpu().numpy(), O.linear_ref(xr, deq, bnp), what + " (oracle rows)")
    want = rotate_gpu64(x, g) @ torch.from_numpy(deq).to(DEV).double().T
    if b is not None:
        want = want + b.to(DEV).double()
    bar_gpu(y, want, what + " (whole output)")


def test_int8_convrot_m256_k3072():
    """INT8-ConvRot M256 K=N=3072, G=128, fp16 scales."""
    int8_case(256, 3072, 3072, 128, seed=100)


@pytest.mark.parametrize("name,n,k", [("qkv", 9216, 3072), ("o", 3072, 3072), ("mlp_up", 12288, 3072),
                                      ("mlp_down", 3072, 12288)])
def test_int8_convrot_dit_layer(name, n, k):
    """The DiT block's four INT8-ConvRot linears at 4608 tokens (4096 image + 512 text), G=128."""
    int8_case(4608, n, k, 128, seed=110 + k // 1024 + n // 1024)


@pytest.mark.parametrize("m,n,k", [
    (2048, 5120, 12288),   # 8 x 20 tiles of 256 x 256: the LDS-DMA kernel, 192 k-tiles over 3 stages
    (1024, 5120, 3072),    # 128 x 256 tiles, two-deep register prefetch (48 k-tiles)
    (640, 4000, 3136),     # 128 x 128 tiles, an odd k-tile count (49): one register set
    (256, 5120, 12288),    # 64 x 128 tiles
    (96, 3072, 13824),     # 64 x 64 tiles, 216 k-tiles
])
def test_int8_linear_long_k(m, n, k):
    int8_case(m, n, k, 128 if k % 128 == 0 else 64, seed=m + k, bias=True)


# ------------------------------------------------------------------------------------------------
# W4A8 / W6A8 (int8 MFMA)
# ------------------------------------------------------------------------------------------------

def random_packed(n, k, bits, gs, seed, srel_dtype):
    """Random legal symmetric codes (4-bit: 1..15 -> -7..7; 6-bit: 1..63 -> -31..31), packed as
    the storage format, with group scales that keep level * s_rel inside the int8 grid."""
    g = torch.Generator().manual_seed(seed)
    hi = 15 if bits == 4 else 63
    codes = torch.randint(1, hi + 1, (n, k), generator=g, dtype=torch.int32)
    q = qz().pack_codes(codes, bits)
    lo, top = (8.0, 18.0) if bits == 4 else (2.0, 4.1)
    s_rel = (lo + (top - lo) * torch.rand(n, k // gs, generator=g)).to(srel_dtype)
    s_ch = (torch.rand(n, generator=g) * 2e-4 + 1e-4).float()
    return q, s_rel, s_ch


def a8_case(m, n, k, bits, gs, g, seed, srel_dtype=torch.float16, outliers=True):
    q, s_rel, s_ch = random_packed(n, k, bits, gs, seed, srel_dtype)
    x = activations(m, k, seed + 1, outliers)
    Q = qlin()
    qd, srd, scd = q.to(DEV), s_rel.to(DEV), s_ch.to(DEV)
    xd = x.to(DEV)
    y = Q.w4a8_int8_linear(xd, qd, srd, scd, None, None, None, gs, g)
    assert y.shape == (m, n) and y.dtype == torch.float16
    what = f"w{bits}a8 gs={gs} M={m} N={n} K={k}"
    if srel_dtype == torch.float8_e4m3fn:
        sr32 = O.srel_to_f32(s_rel.view(torch.uint8).numpy(), "e4m3")
    else:  # fp16 / bf16 / fp32 widen to fp32 exactly
        sr32 = s_rel.float().numpy()
    w8 = O.w4a8_int8_grid(q.numpy(), sr32, None, k, bits, gs)
    assert torch.equal(Q.w4a8_int8_grid(qd, srd, None, gs).cpu(), torch.from_numpy(w8)), what + ": weight grid"
    rows = sample_rows(m, seed)
    rows_d = torch.from_numpy(rows).to(DEV)
    # the activation leg: rotation within one ulp of the oracle's, codes and scales bit-exact
    xq, sx = check_a8_activation_rows(Q, xd, g, rows, what + ": activation quantization")
    w8d = torch.from_numpy(w8).to(DEV)
    acc = xq.double() @ w8d.double().T                      # exact integer sums
    acc_o = O.int8_gemm_i64(xq[rows_d].cpu().numpy(), w8)
    assert np.array_equal(acc[rows_d].cpu().numpy().astype(np.int64), acc_o), what + ": float64 replay != int64 oracle"
    replay = ((acc.float() * sx[:, None]) * scd[None, :]).half()
    bad = (y.view(torch.int16) != replay.view(torch.int16))
    nbad = int(bad.sum().item())
    assert nbad == 0, f"{what}: {nbad} outputs differ from the exact replay, first at {bad.nonzero()[:3].tolist()}"
    sxn = sx[rows_d].cpu().numpy()
    want_rows = O.linear_ref(xq[rows_d].cpu().numpy().astype(np.float32) * sxn[:, None],
                             w8.astype(np.float32) * s_ch.numpy()[:, None])
    bar(y[rows_d].double().cpu().numpy(), want_rows, what + " (oracle rows)")
    want = (xq.double() * sx.double()[:, None]) @ (w8d.double() * scd.double()[:, None]).T
    bar_gpu(y, want, what + " (whole output)")


def test_w4a8_dit_mlp_up():
    """W4A8 M4096 K3072 N12288, group 128, fp16 s_rel, activation outliers."""
    a8_case(4096, 12288, 3072, 4, 128, 128, seed=200)


@pytest.mark.parametrize("m", [1024, 9504])
@pytest.mark.parametrize("n,k", [(13824, 5120), (5120, 13824)])
def test_w6a8_video_dit_ffn(m, n, k):
    """W6A8 14B video-DiT FFN, group 64, fp16 s_rel: up 5120->13824 and down 13824->5120."""
    a8_case(m, n, k, 6, 64, 256, seed=300 + m // 512 + k // 1024, outliers=False)


@pytest.mark.parametrize("m,n,k,bits,gs,srdt", [
    (2048, 6144, 13824, 4, 128, torch.float8_e4m3fn),  # grid once + DMA GEMM 256 x 256, 108 k-tiles
    (1024, 6144, 5120, 6, 64, torch.float16),          # ... 128 x 256 tiles
    (1100, 2000, 3072, 4, 64, torch.bfloat16),         # ... 128 x 128 tiles
    (1000, 12300, 13824, 4, 128, torch.float16),       # fused decode, scale table per thread pair
    (777, 12500, 5120, 6, 64, torch.float8_e4m3fn),    # fused decode, scale table per thread
    (1000, 12300, 3072, 6, 128, torch.float32),
    (130, 1000, 13824, 6, 64, torch.float16),          # 128 x 128 tiles with the decode in the load stage
])
def test_w4a8_linear_long_k(m, n, k, bits, gs, srdt):
    a8_case(m, n, k, bits, gs, 128, seed=m + n + k, srel_dtype=srdt)
