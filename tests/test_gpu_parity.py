"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the same seeded inputs.

Bars: decoded weights and int8 activation quantization bit-exact; linear outputs within 1e-3
relative Frobenius error and 2e-2 max-abs error of a float64 matmul over the same dequantized
operands (the A8 path also bit-exact against an exact replay of its integer GEMM + epilogue).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks
from a8_check import assert_quantized_like_oracle, assert_rotation_close, check_a8_activation_rows

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
REL_TOL, ABS_TOL = 1e-3, 2e-2
GGUF = ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS")
DEV = "cuda:0"


def qlin():
    import qlin as Q
    return Q


def qz():
    from qlin import quantize as QZ
    return QZ


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def check_linear(got, want, what=""):
    got = got.float().cpu().numpy().astype(np.float64)
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max()) if want.size else 0.0
    assert np.isfinite(got).all(), what
    assert rel < REL_TOL and mx < ABS_TOL, f"{what}: rel_fro={rel:.3e} max_abs={mx:.3e}"
    return rel, mx


def x_fp16(m, k, seed=1, outliers=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if outliers:
        mask = torch.rand(m, k, generator=g) < 0.01
        x = torch.where(mask, 20.0 * torch.sign(x), x)
    return x.half()


# ------------------------------------------------------------------------------------------------
# GGUF decode
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name", GGUF)
def test_dequantize_gguf_bit_exact(name):
    n, k = 40, 1024
    for seed, raw in ((0, random_gguf_blocks(name, n, k, seed=3)),
                      (1, qz().quantize_gguf(np.random.default_rng(4).standard_normal((n, k)).astype(np.float32) * 0.02, name))):
        want = O.gguf_dequantize(raw, name, (n, k))
        w = torch.from_numpy(np.ascontiguousarray(raw)).to(DEV)
        got = qlin().dequantize_gguf(w, name, (n, k)).cpu().numpy()
        assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), f"{name} seed {seed}"
        got16 = qlin().dequantize_gguf(w, name, (n, k), out_dtype=torch.float16).cpu().numpy().view(np.uint16)
        want16 = want.astype(np.float16).view(np.uint16)
        bad = np.flatnonzero(got16 != want16)
        assert bad.size == 0, (f"{name}: {bad.size} fp16 mismatches; first: f32 {want.reshape(-1)[bad[:4]]!r} "
                               f"got {got16.reshape(-1)[bad[:4]]} want {want16.reshape(-1)[bad[:4]]}")


@pytest.mark.parametrize("case", ["gauss_96x1024", "heavy_96x1024"])
@pytest.mark.parametrize("fmt,name", [("gguf_q8_0", "Q8_0"), ("gguf_q4_k", "Q4_K")])
def test_dequantize_gguf_golden(case, fmt, name):
    raw = np.load(os.path.join(HERE, "golden", "selftest_raw.npz"))[f"{case}/{fmt}/q"]
    meta = json.load(open(os.path.join(HERE, "golden", "selftest_sha256.json")))
    got = qlin().dequantize_gguf(torch.from_numpy(raw.copy()).to(DEV), name, (96, 1024)).cpu().numpy()
    assert sha(got) == meta["cases"][case]["formats"][fmt]["deq"]


@pytest.mark.parametrize("name", ["Q8_0", "Q4_K", "Q6_K", "Q4_0", "IQ4_XS"])
def test_dequantize_gguf_special_scales(name):
    """fp16 scale fields of 0, +-65504 and subnormals decode exactly."""
    _, qk, ts = O.GGUF_TYPES[name]
    raw = random_gguf_blocks(name, 8, 512, seed=9).reshape(-1, ts)
    specials = np.array([0.0, 65504.0, -65504.0, 6e-8, -3e-6, 2 ** -24, 1.0, -0.0], dtype=np.float16).view(np.uint8)
    offs = {"Q8_0": [0], "Q4_K": [0, 2], "Q6_K": [208], "Q4_0": [0], "IQ4_XS": [0]}[name]
    for i in range(raw.shape[0]):
        for off in offs:
            raw[i, off:off + 2] = specials[2 * (i % 8): 2 * (i % 8) + 2]
    want = O.gguf_dequantize(raw, name)
    got = qlin().dequantize_gguf(torch.from_numpy(raw.reshape(8, -1).copy()).to(DEV), name, (8, 512)).cpu().numpy()
    assert got.reshape(-1).view(np.uint32).tobytes() == want.view(np.uint32).tobytes()


@pytest.mark.parametrize("name", ["Q4_K", "Q8_0", "Q6_K"])
def test_dequantize_gguf_straddling_rows(name):
    """Rows that start mid-block (flat indexing, gguf-on-metal.md:38): N*K is a whole number of
    blocks but K is not."""
    _, qk, ts = O.GGUF_TYPES[name]
    n, k = 32, qk * 3 // 2 if qk == 256 else 48
    raw = random_gguf_blocks(name, 1, n * k, seed=2).reshape(-1)
    want = O.gguf_dequantize(raw, name).reshape(n, k)
    got = qlin().dequantize_gguf(torch.from_numpy(raw.copy()).to(DEV), name, (n, k)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------------------------
# GGUF linear
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name", GGUF)
@pytest.mark.parametrize("m", [1, 4, 5, 8, 16, 17, 64, 100, 128, 129])  # every kernel and each switch point
def test_gguf_linear(name, m):
    n, k = 80, 1024
    raw = random_gguf_blocks(name, n, k, seed=11)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=m)
    want = O.linear_ref(x.float().numpy(), w)
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k))
    assert got.dtype == torch.float16 and got.shape == (m, n)
    check_linear(got, want, f"{name} M={m}")


@pytest.mark.parametrize("name,m,n,k", [
    ("Q4_K", 33, 131, 256),     # one K stage: single split, epilogue in the kernel, ragged N
    ("Q4_0", 64, 131, 1280),    # five splits, N % 4 != 0 in the reduction
    ("Q8_0", 20, 12800, 1280),  # 100 row tiles: three splits over five stages (uneven)
    ("Q3_K", 64, 200, 2048),    # two-block stages, signed sub-scales
    ("Q2_K", 40, 136, 1024),    # four splits, 16-value units with minimums
    ("IQ4_XS", 47, 256, 4096),  # eight splits
    # N a multiple of 1024: each row block's partials are added by workgroups of the XCD that wrote them
    ("Q4_K", 64, 1024, 2048),   # 8 row blocks, 8 splits
    ("Q6_K", 24, 2048, 1024),   # 16 row blocks, 2 splits
    ("Q8_0", 40, 3072, 512),    # 24 row blocks, 2 splits
    ("Q5_K", 64, 16384, 1024),  # 128 row blocks, 2 splits
])
def test_gguf_linear_split_k(name, m, n, k):
    """The K-split kernel (M = 17..64): ragged N, uneven and single splits, bias."""
    raw = random_gguf_blocks(name, n, k, seed=21)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=m + 3)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.1).half()
    want = O.linear_ref(x.float().numpy(), w, b.float().numpy())
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), bias=b.to(DEV))
    check_linear(got, want, f"{name} M={m} N={n} K={k}")


@pytest.mark.parametrize("name,m,n,k", [
    ("Q4_K", 65, 131, 512),     # two m-tiles, the second one row; ragged N; 2 splits
    ("Q4_0", 100, 1000, 2048),  # 8 row blocks x 2 m-tiles, 8 splits
    ("Q8_0", 200, 4096, 1024),  # 32 x 4 tiles, 2 splits (XCD-local reduction)
    ("Q6_K", 256, 256, 2048),   # 2 x 4 tiles, 4 splits (two-block stages)
    ("IQ4_XS", 300, 4096, 512), # 32 x 5 tiles, 2 splits
    ("Q4_0", 384, 4096, 1024),  # 32 x 6 tiles, 3/4 of the GPU: one split
    ("Q5_K", 512, 4096, 1024),  # 32 x 8 tiles: one split, the epilogue in the kernel
    ("Q3_K", 130, 200, 1024),   # signed sub-scales across three m-tiles
    ("Q2_K", 193, 136, 512),    # 16-value units, four m-tiles, the last one row
    ("Q6_K", 450, 1024, 1024),  # 8 x 8 tiles, 2 splits
    ("Q3_K", 512, 2048, 1024),  # 16 x 8 tiles, 2 splits
    ("Q2_K", 400, 300, 512),    # 3 x 7 tiles, the last m-tile 16 rows
])
def test_gguf_linear_split_m_tiles(name, m, n, k):
    """From 65 to 512 rows the split kernel runs 64-row m-tiles along the
    grid's z, each decoding the weight in its load stage: ragged M and N, single and multiple splits,
    bias; no decoded copy is asked for."""
    from qlin import _lib
    raw = random_gguf_blocks(name, n, k, seed=23)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=m + 5)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(7)) * 0.1).half()
    want = O.linear_ref(x.float().numpy(), w, b.float().numpy())
    tid = qlin().GGUF_TYPES[name][0]
    size = _lib.load().qlin_workspace_size(_lib.OP_GGUF_LINEAR, m, n, k, tid, _lib._TORCH_DT[torch.float16])
    # fp16 activations, row and column exponents, fp32 partials of S splits; no decoded copy
    a = lambda v: (v + 255) // 256 * 256
    stages = k // (512 if name in ("Q6_K", "Q3_K") else 256)
    tiles = -(-n // 128) * -(-m // 64)
    splits = 1 if 4 * tiles >= 3 * 256 else max(1, min(-(-256 // tiles), stages, 8))
    assert size == a(m * k * 2) + a(m * 4) + a(n * 4) + (a(splits * m * n * 4) if splits > 1 else 0)
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), bias=b.to(DEV))
    check_linear(got, want, f"{name} M={m} N={n} K={k}")


def _split_call(raw, name, n, k, x, ws=None):
    """qlin_gguf_linear through the C ABI with a caller-owned workspace (None: the cached one)."""
    Q = qlin()
    if ws is None:
        return Q.gguf_linear(x, raw, name, (n, k))
    from qlin import _lib
    L = _lib.load()
    tid = Q.GGUF_TYPES[name][0]
    y = torch.empty(x.shape[0], n, dtype=torch.float16, device=DEV)
    st = L.qlin_gguf_linear(_lib.desc(x), raw.data_ptr(), tid, n, k, _lib.desc(None), _lib.desc(y),
                            ws.data_ptr(), ws.numel(), _lib.stream_of(x.device))
    _lib.check(st, "gguf_linear")
    return y


@pytest.mark.parametrize("fill", ["ff", "random", "repeat"])
def test_gguf_linear_split_k_workspace_contents(fill):
    """The K split keeps its partials in the caller's workspace without clearing it first: whatever
    the workspace holds (all ones, random bytes, a previous call's leftovers), every call is right
    and bit-identical to the others (the partials are added in split order)."""
    Q = qlin()
    name, m, n, k = "Q4_K", 64, 4096, 4096  # 32 row blocks x 8 splits
    raw = random_gguf_blocks(name, n, k, seed=51)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=52)
    want = O.linear_ref(x.float().numpy(), w)
    rawd, xd = torch.from_numpy(raw).to(DEV), x.to(DEV)
    tid = Q.GGUF_TYPES[name][0]
    from qlin import _lib
    nbytes = _lib.load().qlin_workspace_size(_lib.OP_GGUF_LINEAR, m, n, k, tid, _lib._TORCH_DT[torch.float16])
    g = torch.Generator().manual_seed(53)
    if fill == "ff":
        ws = torch.full((nbytes,), 255, dtype=torch.uint8)
    else:
        ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    ws = ws.to(DEV)
    outs = []
    for rep in range(3):
        if fill == "random" and rep:
            ws.copy_(torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g).to(DEV))
        outs.append(_split_call(rawd, name, n, k, xd, ws))
    torch.cuda.synchronize()
    check_linear(outs[0], want, f"{name} M={m} workspace {fill}")
    for o in outs[1:]:
        assert torch.equal(o, outs[0]), f"workspace {fill}: calls differ"


def test_gguf_linear_split_k_graph_replays():
    """A captured K-split call replayed several times, with eager calls (their own workspace) and new
    activations between the replays: every replay equals the eager call on the same input."""
    Q = qlin()
    name, m, n, k = "Q6_K", 48, 4096, 2048
    raw = torch.from_numpy(random_gguf_blocks(name, n, k, seed=61)).to(DEV)
    xs = [x_fp16(m, k, seed=62 + i).to(DEV) for i in range(4)]
    xin = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        Q.gguf_linear(xin, raw, name, (n, k))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg = Q.gguf_linear(xin, raw, name, (n, k))
    torch.cuda.synchronize()
    for i in range(8):
        xin.copy_(xs[i % 4])
        g.replay()
        torch.cuda.synchronize()
        got = yg.clone()
        want = Q.gguf_linear(xs[i % 4], raw, name, (n, k))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager call"


@pytest.mark.parametrize("name,m,n,k", [
    # from 17 to 512 rows the split kernel takes K a whole number of its 256-value stages (Q6_K 512):
    # these shapes have other K or more rows
    ("Q4_0", 65, 131, 1056),    # K % 64 == 32: the last k-tile's upper half is past K; ragged N
    ("Q8_0", 200, 300, 96),     # two k-tiles, the second half empty
    ("IQ4_NL", 129, 257, 2080),
    ("Q4_K", 600, 520, 2048),
    ("Q6_K", 96, 1000, 768),
    ("Q2_K", 577, 64, 512),     # one column tile, half of it past N
    ("Q5_K", 530, 256, 6144),   # the decode keeps 3 chunks of 8 per thread (4 slots)
    ("Q8_0", 520, 96, 8448),    # K > 8192: the decode reads each row twice
    ("Q4_K", 1024, 512, 1024),  # 128 x 128 tiles
])
def test_gguf_linear_decode_once(name, m, n, k):
    """Above the split kernel's rows, with the workspace qlin_workspace_size reports, the weight is decoded once into
    it as fp16 and a DMA-ring GEMM loads that copy (K % 64 == 32: the tiled GEMM loads it); with the
    minimum workspace (no room for the copy) the tiled GEMM decodes every tile it loads.  Both meet
    the oracle's bar.  The workspaces start as all-ones bytes (fp16 NaN), so any element of the
    copy left unwritten shows."""
    from qlin import _lib
    L = _lib.load()
    raw = random_gguf_blocks(name, n, k, seed=71)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=m + 7)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.1).half()
    want = O.linear_ref(x.float().numpy(), w, b.float().numpy())
    rawd, xd, bd = torch.from_numpy(raw).to(DEV), x.to(DEV), b.to(DEV)
    tid = qlin().GGUF_TYPES[name][0]
    full = L.qlin_workspace_size(_lib.OP_GGUF_LINEAR, m, n, k, tid, _lib._TORCH_DT[torch.float16])
    copy = (n * k * 2 + 255) // 256 * 256
    outs = []
    for nbytes in (full, full - copy):
        ws = torch.full((nbytes,), 255, dtype=torch.uint8, device=DEV)
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        st = L.qlin_gguf_linear(_lib.desc(xd), rawd.data_ptr(), tid, n, k, _lib.desc(bd), _lib.desc(y),
                                ws.data_ptr(), nbytes, _lib.stream_of(xd.device))
        _lib.check(st, "gguf_linear")
        outs.append(y)
    torch.cuda.synchronize()
    check_linear(outs[0], want, f"{name} M={m} N={n} K={k} decoded once")
    check_linear(outs[1], want, f"{name} M={m} N={n} K={k} decoded per tile")
    if k % 64:  # the same tiled GEMM over the same fp16 values: the same bits
        assert torch.equal(outs[0], outs[1]), "decoded copy and per-tile decode differ"
    # a weight at an odd address (the C ABI takes any byte pointer): the decode copies its rows
    # bytewise, and up to 64 rows the tiled GEMM decodes each tile
    if name in ("Q4_0", "Q4_K", "Q6_K"):
        buf = torch.empty(rawd.numel() + 1, dtype=torch.uint8, device=DEV)
        buf[1:].copy_(rawd.reshape(-1))
        for mm in (m, 8):
            ws = torch.full((L.qlin_workspace_size(_lib.OP_GGUF_LINEAR, mm, n, k, tid, _lib._TORCH_DT[torch.float16]),),
                            255, dtype=torch.uint8, device=DEV)
            yo = torch.empty(mm, n, dtype=torch.float16, device=DEV)
            st = L.qlin_gguf_linear(_lib.desc(xd[:mm]), buf.data_ptr() + 1, tid, n, k, _lib.desc(bd), _lib.desc(yo),
                                    ws.data_ptr(), ws.numel(), _lib.stream_of(xd.device))
            _lib.check(st, "gguf_linear (odd weight address)")
            torch.cuda.synchronize()
            check_linear(yo, want[:mm], f"{name} M={mm} N={n} K={k} weight at an odd address")
    # below the minimum: refused before anything runs (the pointer is never dereferenced)
    ws = torch.empty(full - copy - 256, dtype=torch.uint8, device=DEV)
    st = L.qlin_gguf_linear(_lib.desc(xd), rawd.data_ptr(), tid, n, k, _lib.desc(bd), _lib.desc(y),
                            ws.data_ptr(), ws.numel(), _lib.stream_of(xd.device))
    assert st == _lib.QLIN_EWORKSPACE


# Long rows.  One activation row with K / (values per lane chunk) in {16, 32, 64} takes the GEMV
# kernel for every format it covers (at K = 1024 most formats take the small-M kernel instead);
# K = 4096 is the decode shape.  M = 8 and 16 take the small-M kernel (Q6_K: the K split).
@pytest.mark.parametrize("name", GGUF)
@pytest.mark.parametrize("m,k", [(1, 2048), (1, 4096), (1, 8192), (8, 4096), (16, 8192)])
def test_gguf_linear_long_k(name, m, k):
    n = 72
    raw = random_gguf_blocks(name, n, k, seed=31)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = x_fp16(m, k, seed=k + m)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(6)) * 0.1).half()
    want = O.linear_ref(x.float().numpy(), w, b.float().numpy())
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), bias=b.to(DEV))
    assert got.shape == (m, n)
    check_linear(got, want, f"{name} M={m} K={k}")


@pytest.mark.parametrize("name", ["Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS"])
def test_gguf_linear_decode_workload(name):
    """The benchmarked calls themselves: K = N = 4096 at M = 1, 8 and 64 (GEMV, small-M or K split,
    and the K split with its XCD-local reduction, S = 8)."""
    n = k = 4096
    raw = random_gguf_blocks(name, n, k, seed=41)
    w = O.gguf_dequantize(raw, name, (n, k))
    wd = torch.from_numpy(raw).to(DEV)
    for m in (1, 8, 64):
        x = x_fp16(m, k, seed=m + 40)
        got = qlin().gguf_linear(x.to(DEV), wd, name, (n, k))
        check_linear(got, O.linear_ref(x.float().numpy(), w), f"{name} M={m} K=N=4096")


@pytest.mark.parametrize("name,odt", [("Q4_K", torch.float16), ("Q6_K", torch.bfloat16), ("Q8_0", torch.float32)])
def test_gguf_linear_decode_in_chunks(name, odt):
    """Above 512 rows the weight is decoded once into the workspace in chunks of weight rows (at most
    256 MiB each, multiples of 128 rows): with the workspace the size query asks for (one chunk
    here), with room for 256 rows (four chunks, the last ragged) or 130 rows (128-row chunks), the
    output equals the oracle's linear to the bar; with no room for 128 rows each GEMM tile decodes
    its own weights."""
    from qlin import _lib as L
    m, n, k = 520, 1000, 2048  # above the split kernel's rows
    raw = random_gguf_blocks(name, n, k, seed=77)
    w = O.gguf_dequantize(raw, name, (n, k))
    # activations of 0.25: outputs below 4, where one bf16 rounding step stays under the 2e-2 bar
    x = (x_fp16(m, k, seed=78).float() * 0.25).half()
    b = (torch.randn(n, generator=torch.Generator().manual_seed(79)) * 0.1).half()
    want = O.linear_ref(x.float().numpy(), w, b.float().numpy())
    if odt == torch.bfloat16:
        want = torch.from_numpy(want.astype(np.float32)).bfloat16().double().numpy()
    tid = O.gguf_type_id(name)
    full = L.load().qlin_workspace_size(L.OP_GGUF_LINEAR, m, n, k, tid, L.DT_F16)
    align = lambda v: (v + 255) // 256 * 256
    base = full - align(n * k * 2)   # everything but the decoded copy
    xd, rd, bd = x.to(DEV), torch.from_numpy(raw).to(DEV), b.to(DEV)
    for rows in (n, 256, 130, 100):
        nbytes = base + align(rows * k * 2)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        y = torch.full((m, n), float("nan"), dtype=odt, device=DEV)
        st = L.load().qlin_gguf_linear(L.desc(xd), rd.data_ptr(), tid, n, k, L.desc(bd), L.desc(y), ws.data_ptr(),
                                       ws.numel(), L.stream_of(xd.device))
        L.check(st, "qlin_gguf_linear")
        check_linear(y, want, f"{name} M={m} N={n} K={k}, workspace for {rows} decoded rows")


@pytest.mark.parametrize("xdt,odt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.float32), (torch.float16, torch.float32)])
@pytest.mark.parametrize("m", [3, 40, 200])
def test_gguf_linear_dtypes_and_bias(xdt, odt, m):
    name, n, k = "Q4_K", 96, 512
    raw = random_gguf_blocks(name, n, k, seed=5)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(3)).to(xdt)
    b = torch.randn(n, generator=torch.Generator().manual_seed(4)) * 0.1
    want = O.linear_ref(x.float().numpy(), w, b.numpy())
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), 12, (n, k), bias=b.to(DEV), out_dtype=odt)
    assert got.dtype == odt
    if odt == torch.bfloat16:
        # bf16 output rounding alone is ~1.1e-3 rel RMS: compare with the reference rounded to bf16
        want_b = torch.from_numpy(want).to(torch.bfloat16).double().numpy()
        assert O.rel_fro(got.double().cpu().numpy(), want_b) < 1e-3
        assert O.rel_fro(got.double().cpu().numpy(), want) < 4e-3
    else:
        check_linear(got, want, f"x {xdt} out {odt}")


def test_gguf_linear_large_activations_near_max_scales():
    """|x| ~ 3e4 against near-max fp16 block scales: fp32 accumulation, no overflow."""
    name, n, k = "Q8_0", 32, 256
    raw = random_gguf_blocks(name, n, k, seed=6).reshape(-1, 34)
    raw[:, :2] = np.array([60000.0], dtype=np.float16).view(np.uint8)
    raw = raw.reshape(n, -1)
    w = O.gguf_dequantize(raw, name, (n, k))
    x = (torch.randn(2, k, generator=torch.Generator().manual_seed(1)) * 1e4).clamp(-6e4, 6e4).half()
    x[:, :4] = 3e4
    want = O.linear_ref(x.float().numpy(), w)
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k), out_dtype=torch.float32)
    rel = O.rel_fro(got.cpu().numpy(), want)
    assert np.isfinite(got.cpu().numpy()).all() and rel < REL_TOL


SCALE_FIELDS = {"Q8_0": [0], "Q4_0": [0], "Q4_1": [0, 2], "Q5_1": [0, 2], "IQ4_NL": [0], "IQ4_XS": [0],
                "Q4_K": [0, 2], "Q5_K": [0, 2], "Q6_K": [208], "Q2_K": [80, 82], "Q3_K": [108]}


@pytest.mark.parametrize("m", [1, 4, 8, 40, 100])
@pytest.mark.parametrize("name", list(SCALE_FIELDS))
def test_gguf_linear_folded_scale_ranges(name, m):
    """The split kernel (Q6_K from 3 rows, every format from 17) folds block scales into fp16
    operands with a power of two per weight row and K half; the one-row kernel (M = 1) and the
    small-M kernel (M = 4) apply them in fp32 after exact fp16 code products.  Weight rows whose fp16 block scales are all subnormal, mix 6e4 with
    1e-3 and subnormals in one half, are all zero, or are ordinary: every output column within the
    bar of its own fp64 product (a missing or misplaced exponent loses the small rows' precision
    or overflows the large ones), zero rows exactly zero."""
    n, k = 128, 2048
    _, qk, ts = O.GGUF_TYPES[name]
    raw = random_gguf_blocks(name, n, k, seed=17).reshape(n, -1, ts)
    rng = np.random.default_rng(5)
    for r in range(n):
        kind = r % 4
        for b in range(raw.shape[1]):
            if kind == 0:    # all subnormal: |w| far below fp16's normal range
                v = float(rng.choice([6e-8, -3e-7, 2e-6, 1.5e-5]))
            elif kind == 1:  # a huge, a small and a subnormal scale in the same K half
                v = float([60000.0, 1e-3, -4e-7, 250.0][b % 4])
            elif kind == 2:
                continue
            else:
                v = 0.0
            for off in SCALE_FIELDS[name]:
                raw[r, b, off:off + 2] = np.array([v], np.float16).view(np.uint8)
    raw = raw.reshape(n, -1)
    w = O.gguf_dequantize(raw, name, (n, k)).astype(np.float64)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half()
    want = x.double().numpy() @ w.T
    got = qlin().gguf_linear(x.to(DEV), torch.from_numpy(raw).to(DEV), name, (n, k),
                             out_dtype=torch.float32).double().cpu().numpy()
    assert np.isfinite(got).all()
    zero = np.abs(w).max(axis=1) == 0
    assert zero[3::4].all() and not got[:, zero].any()
    xn = np.linalg.norm(x.double().numpy(), axis=1)
    for c in np.flatnonzero(~zero):
        err = np.linalg.norm(got[:, c] - want[:, c])
        if m >= 8:
            rel = err / np.linalg.norm(want[:, c])
        else:
            # a column of one to four dot products can cancel far below its terms by chance: the
            # bar is against the typical magnitude of x.w for this weight row, ||x|| ||w_c|| / sqrt(K)
            # (a lost or misplaced exponent still misses it by orders of magnitude)
            rel = err / (np.linalg.norm(xn) * np.linalg.norm(w[c]) / np.sqrt(k))
        assert rel < REL_TOL, (f"{name} M={m} row {c} (kind {c % 4}): rel {rel:.3e}, "
                               f"|want| {np.linalg.norm(want[:, c]):.3e}, err {err:.3e}")


def test_gguf_linear_shapes_and_empty():
    Q = qlin()
    name, n, k = "Q4_0", 48, 256
    raw = torch.from_numpy(random_gguf_blocks(name, n, k, seed=1)).to(DEV)
    x = torch.randn(2, 3, k, device=DEV).half()
    y = Q.gguf_linear(x, raw, name, (n, k))
    assert y.shape == (2, 3, n)
    y1 = Q.gguf_linear(x[0, 0], raw, name, (n, k))
    assert y1.shape == (n,)
    torch.testing.assert_close(y1, y[0, 0], rtol=0, atol=0)
    e = Q.gguf_linear(torch.empty(0, k, device=DEV).half(), raw, name, (n, k))
    assert e.shape == (0, n)
    xs = torch.randn(5, k + 8, device=DEV).half()[:, 8:]  # strided rows with a storage offset
    torch.testing.assert_close(Q.gguf_linear(xs, raw, name, (n, k)), Q.gguf_linear(xs.contiguous(), raw, name, (n, k)),
                               rtol=0, atol=0)
    with pytest.raises(ValueError):  # lora_down without lora_up
        Q.gguf_linear(x, raw, name, (n, k), lora_down=torch.zeros(1, k, device=DEV))


# ------------------------------------------------------------------------------------------------
# INT8 ConvRot weight-only
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("g", [0, 128, 256])
@pytest.mark.parametrize("m", [1, 33, 256])
def test_int8_linear(g, m):
    n, k = 192, 1024
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = qz().quantize_int8_convrot_weight(w, g) if g else qz().quantize_int8_rowwise(w)
    x = x_fp16(m, k, seed=m)
    xr = O.rotate(x.float().numpy(), g) if g else x.float().numpy()
    want = O.linear_ref(xr, O.dequantize_int8(q, s))
    got = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                             convrot=bool(g), convrot_groupsize=g or 256)
    check_linear(got, want, f"G={g} M={m}")
    # the original-basis weight gives the same product on the unrotated activation
    if g:
        want2 = O.linear_ref(x.float().numpy(), O.dequantize_int8_convrot(q, s, g))
        assert O.rel_fro(want2, want) < 1e-5


@pytest.mark.parametrize("g,m,n,xdt,odt", [(0, 2047, 6136, torch.float16, torch.float16),
                                           (128, 2303, 5880, torch.bfloat16, torch.bfloat16),
                                           (128, 640, 4000, torch.float16, torch.float32),
                                           (128, 2600, 6100, torch.float16, torch.float16),
                                           (0, 2600, 6100, torch.bfloat16, torch.float32),
                                           (128, 5000, 4000, torch.float16, torch.bfloat16)])
def test_int8_linear_large_tiles(g, m, n, xdt, odt):
    """Shapes that take the 256 x 256 tile (192 and 207 tiles, ragged M and N), the 128 x 128 tile
    (640 x 4000: 160 tiles), and 264 tiles of 256 x 256 whose last round would leave most CUs idle
    (rows 0..2559 on 256 x 256 tiles, then rows 2560..2599 on 128 x 256 tiles in a second launch),
    with fp16 scales and a bias."""
    k = 256
    rng = np.random.default_rng(17)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = qz().quantize_int8_convrot_weight(w, g) if g else qz().quantize_int8_rowwise(w)
    s16 = s.astype(np.float16)
    b = rng.standard_normal(n).astype(np.float32)
    x = x_fp16(m, k, seed=5).to(xdt)
    xr = O.rotate(x.float().numpy(), g) if g else x.float().numpy()
    want = O.linear_ref(xr, O.dequantize_int8(q, s16.astype(np.float32)), b)
    got = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s16).to(DEV),
                             torch.from_numpy(b).to(DEV), odt, convrot=bool(g), convrot_groupsize=g or 256)
    assert got.dtype == odt
    if odt == torch.bfloat16:  # one bf16 rounding of the output
        rb = torch.from_numpy(want.astype(np.float32)).bfloat16().double().numpy()
        assert O.rel_fro(got.double().cpu().numpy(), rb) < 1e-3
        assert O.rel_fro(got.double().cpu().numpy(), want) < 4e-3
    else:
        check_linear(got, want, f"G={g} large tiles")


def test_int8_linear_scales_bias_bf16():
    n, k, m = 64, 512, 70
    rng = np.random.default_rng(8)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal(n)) * 1e-3).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(2)).bfloat16()
    xr = O.rotate(x.float().numpy(), 256)
    want = O.linear_ref(xr, O.dequantize_int8(q, s), b)
    got = qlin().int8_linear(x.to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).half().to(DEV),
                             torch.from_numpy(b).to(DEV), torch.float32, convrot=True)
    want16 = O.linear_ref(xr, O.dequantize_int8(q, s.astype(np.float16).astype(np.float32)), b)
    check_linear(got, want16, "fp16 scale + bias")
    assert O.rel_fro(want16, want) < 1e-3


def test_int8_linear_extremes():
    """Edge cases of bench/probe_small_m.py:84-101: tiny inputs, huge/zero scales, rotation growth."""
    Q = qlin()
    h = O.hadamard(256)
    onehot = np.zeros((4, 256), np.int8)
    onehot[:, 0] = 1
    cases = [
        ("tiny_input", np.full((1, 256), 2.0 ** -26, np.float32), np.ones((4, 256), np.int8), np.ones(4, np.float32), 0),
        ("large_scale", np.full((1, 256), 0.001 / 256, np.float32), np.ones((4, 256), np.int8),
         np.array([1e5, 3e7, 1e-30, -1e5], np.float32), 0),
        ("zero_scale", np.ones((1, 256), np.float32), np.ones((4, 256), np.int8), np.zeros(4, np.float32), 256),
        ("rotation_growth", (10000 * np.sign(h[:, 0])).reshape(1, -1).astype(np.float32), onehot,
         np.full(4, 0.001, np.float32), 256),
    ]
    for name, x, q, s, g in cases:
        xt = torch.from_numpy(x).to(DEV)
        got = Q.int8_linear(xt, torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), None, torch.float32,
                            convrot=bool(g), convrot_groupsize=g or 256).cpu().numpy()
        xr = O.rotate(x, g) if g else x
        want = O.linear_ref(xr, O.dequantize_int8(q, s))
        den = max(np.abs(want).max(), 1e-30)
        assert np.isfinite(got).all(), name
        assert np.abs(got - want).max() / den < 2e-3, f"{name}: {got} vs {want}"


def test_dequantize_int8_bit_exact_and_rotation():
    n, k = 64, 512
    rng = np.random.default_rng(1)
    q = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    s = (np.abs(rng.standard_normal(n)) * 1e-3).astype(np.float32)
    qt, st = torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV)
    got = qlin().dequantize_int8(qt, st).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), O.dequantize_int8(q, s).view(np.uint32))
    rot = qlin().dequantize_int8_convrot_weight(qt, st, 256).cpu().numpy()
    assert O.rel_fro(rot, O.dequantize_int8_convrot(q, s, 256)) < 1e-6


# ------------------------------------------------------------------------------------------------
# A8 activation quantization and W4A8 / W6A8
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_act_int8_bit_exact(dt):
    m, k = 37, 768
    x = x_fp16(m, k, seed=5, outliers=True).float()
    x[3] = 0.0                       # zero row: scale clamps to 1e-30, dtype scale -> tiny
    x[4] = x[4] * 1e-6               # tiny row
    x = x.to(dt)
    q, s = qlin().quantize_int8_rowwise(x.to(DEV))
    if dt == torch.bfloat16:
        wq, ws = O.quantize_int8_rowwise(x.view(torch.int16).numpy().view(np.uint16), bf16=True)
    else:
        wq, ws = O.quantize_int8_rowwise(x.numpy())
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))


@pytest.mark.parametrize("g", [128, 256])
def test_quantize_act_rotated(g):
    """With ConvRot: the rotation is fp32 (within one fp16 ulp of the exact rotation, rarely off),
    and the int8 quantization of the rotated row is bit-exact."""
    m, k = 64, 1024
    x = x_fp16(m, k, seed=6, outliers=True)
    q, s, xr = qlin().quantize_int8_rowwise(x.to(DEV), g, return_rotated=True)
    xr = xr.cpu().numpy()
    exact = O.rotate(x.numpy(), g)
    diff = np.abs(xr.view(np.uint16).astype(np.int32) - exact.view(np.uint16).astype(np.int32))
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-2
    wq, ws = O.quantize_int8_rowwise(xr)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))



# Row widths of the A8 calls the benchmark runs and the prologue variant each takes: K = 3072 with
# G = 128 (W4A8 MLP-up; one slot of 16 values per thread), K = 5120 with G = 256 (W6A8 FFN up; one
# slot), K = 13824 with G = 256 (W6A8 FFN down; two slots), K = 24576 (two slots, 768 threads), and
# the two-pass wide kernel (four slots per chunk) at K = 65536 and 73728.
A8_WIDTHS = [(3072, 128, 40), (5120, 256, 40), (13824, 256, 24), (24576, 128, 12), (65536, 128, 6),
             (73728, 256, 5)]


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k,g,m", A8_WIDTHS)
def test_quantize_act_rotated_widths(k, g, m, dt):
    """quantize_int8_rowwise(rot(x)) at every A8 width, fp16 and bf16 rows with 1% outliers at 20
    sigma, a zero row and a tiny row: the rotated rows within one ulp of the oracle's exact rotation,
    the codes and scales of those rows bit-exact against the oracle's quantize_int8_rowwise."""
    x = x_fp16(m, k, seed=k + g, outliers=True).float()
    x[1] = 0.0
    x[2] = x[2] * 1e-6
    x = x.to(dt)
    q, s, xr = qlin().quantize_int8_rowwise(x.to(DEV), g, return_rotated=True)
    what = f"K={k} G={g} {dt}"
    assert_rotation_close(x, xr.cpu(), g, what)
    assert_quantized_like_oracle(xr.cpu(), q.cpu(), s.cpu(), what)


W4A8_CASES = [
    (4, 16, "auto", torch.float8_e4m3fn),
    (4, 128, None, torch.float16),
    (6, 16, None, torch.float8_e4m3fn),
    (6, 64, None, torch.float16),
]


@pytest.mark.parametrize("bits,gs,cb,srdt", W4A8_CASES)
@pytest.mark.parametrize("m", [1, 130])
def test_w4a8_linear(bits, gs, cb, srdt, m):
    n, k, g = 160, 1024, 256
    rng = np.random.default_rng(10 + bits)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s_rel, s_ch, book = qz().quantize_w4a8_int8_weight(w, bits=bits, group_size=gs, convrot_groupsize=g,
                                                          codebook=cb, s_rel_dtype=srdt)
    x = x_fp16(m, k, seed=m, outliers=True)
    b = torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.1
    dev = lambda t: None if t is None else t.to(DEV)
    Q = qlin()
    y = Q.w4a8_int8_linear(x.to(DEV), dev(q), dev(s_rel), dev(s_ch), dev(book), None, None, gs, g)
    # (1) the weight grid is bit-exact with the oracle's decode
    sr32 = s_rel.float().numpy()
    w8 = O.w4a8_int8_grid(q.numpy(), sr32, None if book is None else book.numpy(), k, bits, gs)
    assert np.array_equal(Q.w4a8_int8_grid(dev(q), dev(s_rel), dev(book), gs).cpu().numpy(), w8)
    # (2) exact replay of the int8 GEMM + epilogue on the activations the GPU quantized
    xq, sx = check_a8_activation_rows(Q, x.to(DEV), g, np.arange(m), f"bits={bits} gs={gs} M={m}: activations")
    xq, sx = xq.cpu().numpy(), sx.cpu().numpy().reshape(-1)
    acc = O.int8_gemm_i64(xq, w8)
    replay = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * s_ch.numpy()[None, :]).astype(np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), replay.astype(np.float16).view(np.uint16))
    # (3) tolerance against a float64 matmul over the dequantized operands
    want = O.linear_ref(xq.astype(np.float32) * sx[:, None], w8.astype(np.float32) * s_ch.numpy()[:, None])
    check_linear(y, want, f"bits={bits} gs={gs} M={m}")
    # bias joins after the rescale
    yb = Q.w4a8_int8_linear(x.to(DEV), dev(q), dev(s_rel), dev(s_ch), dev(book), None, dev(b), gs, g)
    check_linear(yb, want + b.numpy()[None, :].astype(np.float64), "bias")


A8_TILE_CASES = [
    # M >= 1024: int8 grid decoded once, then the LDS-DMA GEMM; 256 x 256 tiles (8 x 24 = 192, and
    # 9 x 23 = 207, not a multiple of the 8 XCDs)
    (4, None, torch.float16, 128, 256, 2047, 6136),
    (4, None, torch.float16, 64, 128, 2303, 5880),
    (4, "auto", torch.float8_e4m3fn, 64, 128, 2047, 6136),
    (6, None, torch.float8_e4m3fn, 64, 256, 2047, 6136),
    # the same GEMM with 128 x 256 tiles (6 x 20 tiles of 256 x 256 would not fill the GPU) and 128 x 128
    (6, "auto", torch.float16, 64, 128, 1300, 5000),
    (6, None, torch.float16, 64, 256, 1024, 4200),  # 216 tiles of 128 x 160 (2 x 5 waves, one round)
    (4, None, torch.float16, 64, 1024, 1000, 5100), # 256 tiles of 128 x 160, ragged M and N, 8 k-tiles
    (4, None, torch.float8_e4m3fn, 128, 256, 1024, 2000),
    # 264 tiles of 256 x 256: rows 0..2559 in whole rounds of them, the last 41 on 128 x 256 tiles
    (6, None, torch.float16, 64, 512, 2601, 6100),
    # 320 tiles of 256 x 256: rows 0..4095 in one round, the last 904 on 128 x 256 tiles
    (4, "auto", torch.float8_e4m3fn, 128, 256, 5000, 4000),
    # M < 512 with >= 192 tiles of 256 x 256: the fused-decode kernel, one scale table per thread
    # pair (group 128) and per thread (group 64)
    (4, None, torch.float16, 128, 128, 300, 24600),
    (6, "auto", torch.float8_e4m3fn, 64, 256, 257, 25000),
    # 512 <= M < 1024: the grid decoded once, then the int8 DMA GEMM
    (4, None, torch.float16, 128, 128, 1000, 12300),
    (6, "auto", torch.float8_e4m3fn, 64, 256, 777, 12500),
]


@pytest.mark.parametrize("bits,cb,srdt,gs,k,m,n", A8_TILE_CASES)
def test_w4a8_linear_large_tiles(bits, cb, srdt, gs, k, m, n):
    """Shapes that take the large-tile A8 kernels, ragged in M and N."""
    g = 128
    rng = np.random.default_rng(20 + bits)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if cb == "auto":  # heavy tails (the quantizer fits a codebook), rescaled to the same spread
        w = w * np.exp(rng.standard_normal((n, k)))
        w = (w * (0.02 / w.std())).astype(np.float32)
    q, s_rel, s_ch, book = qz().quantize_w4a8_int8_weight(w, bits=bits, group_size=gs, convrot_groupsize=g,
                                                          codebook=cb, s_rel_dtype=srdt)
    x = x_fp16(m, k, seed=3, outliers=True)
    dev = lambda t: None if t is None else t.to(DEV)
    Q = qlin()
    y = Q.w4a8_int8_linear(x.to(DEV), dev(q), dev(s_rel), dev(s_ch), dev(book), None, None, gs, g)
    w8 = O.w4a8_int8_grid(q.numpy(), s_rel.float().numpy(), None if book is None else book.numpy(), k, bits, gs)
    xq, sx = check_a8_activation_rows(Q, x.to(DEV), g, np.unique([0, m // 2, m - 1]), f"bits={bits} M={m}: activations")
    xq, sx = xq.cpu().numpy(), sx.cpu().numpy().reshape(-1)
    acc = O.int8_gemm_i64(xq, w8)
    replay = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * s_ch.numpy()[None, :]).astype(np.float32)
    got = y.cpu().numpy()
    bad = got.view(np.uint16) != replay.astype(np.float16).view(np.uint16)
    assert not bad.any(), f"{int(bad.sum())} mismatches, first at {np.argwhere(bad)[:3].tolist()}"
    want = O.linear_ref(xq.astype(np.float32) * sx[:, None], w8.astype(np.float32) * s_ch.numpy()[:, None])
    # against float64: the fp16 output's own rounding (half an ulp, |y| 2^-11) bounds the large
    # outputs of the outlier rows, above the absolute bar once |y| > 32
    got64 = y.float().cpu().numpy().astype(np.float64)
    assert O.rel_fro(got64, want) < REL_TOL
    err, lim = np.abs(got64 - want), np.maximum(ABS_TOL, np.abs(want) * 2.0 ** -10)
    assert (err <= lim).all(), f"bits={bits} large tiles: max error / bound {float((err / lim).max()):.3f}"


@pytest.mark.parametrize("xdt,g,k,bits,gs,srdt", [
    (torch.bfloat16, 256, 13824, 6, 64, torch.float16),       # two slots per prologue thread
    (torch.bfloat16, 128, 3072, 4, 128, torch.float8_e4m3fn),
    (torch.float16, 256, 5120, 4, 64, torch.bfloat16),
    (torch.float16, 128, 1024, 6, 64, torch.float32),         # fp16 scales widened to fp32
])
def test_w4a8_prepass_one_launch(xdt, g, k, bits, gs, srdt):
    """Decode-once shapes from 2048 rows with 16-bit activations and rotation group 128 or 256: the
    activation prologue (M = 2053 workgroups) and the weight-grid decode (ragged N = 137) share one
    launch.  The output replays exactly from the standalone quantizer's activations and the
    oracle's grid."""
    m, n = 2053, 137
    rng = np.random.default_rng(k + bits)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s_rel, s_ch, book = qz().quantize_w4a8_int8_weight(
        w, bits=bits, group_size=gs, convrot_groupsize=g,
        s_rel_dtype=torch.float16 if srdt == torch.float32 else srdt)
    s_rel = s_rel.to(srdt)
    x = x_fp16(m, k, seed=k, outliers=True).to(xdt)
    Q = qlin()
    y = Q.w4a8_int8_linear(x.to(DEV), q.to(DEV), s_rel.to(DEV), s_ch.to(DEV), None, None, None, gs, g)
    assert y.dtype == xdt
    w8 = O.w4a8_int8_grid(q.numpy(), s_rel.float().numpy(), None, k, bits, gs)
    xq, sx = check_a8_activation_rows(Q, x.to(DEV), g, np.array([0, 1, 1030, m - 1]), f"{xdt} K={k}: activations")
    xq, sx = xq.cpu().numpy(), sx.cpu().numpy().reshape(-1)
    acc = O.int8_gemm_i64(xq, w8)
    replay = torch.from_numpy(((acc.astype(np.float32) * sx[:, None]).astype(np.float32) *
                               s_ch.numpy()[None, :]).astype(np.float32)).to(xdt)
    bad = y.cpu().view(torch.int16) != replay.view(torch.int16)
    assert not bad.any(), f"{int(bad.sum())} mismatches, first at {bad.nonzero()[:3].tolist()}"


@pytest.mark.parametrize("kind", ["w6a8", "int8"])
def test_prepass_and_tail_split_graph_replays(kind):
    """Captured calls that take the one-launch A8 pre-pass (2601 rows) and the tail split (264 tiles
    of 256 x 256: 2560 rows, then 41 on 128 x 256 tiles), replayed with new activations and eager
    calls between the replays: every replay equals the eager call on the same input."""
    Q = qlin()
    m, n, k = 2601, 6100, 512
    g = torch.Generator().manual_seed(71)
    if kind == "w6a8":
        from qlin.quantize import pack_codes
        q = pack_codes(torch.randint(1, 64, (n, k), generator=g, dtype=torch.int32), 6).to(DEV)
        s_rel = (2 + 2 * torch.rand(n, k // 64, generator=g)).half().to(DEV)
        s_ch = (torch.rand(n, generator=g) * 2e-4 + 1e-4).to(DEV)
        call = lambda x: Q.w4a8_int8_linear(x, q, s_rel, s_ch, None, None, None, 64, 128)
    else:
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(DEV)
        s = (torch.rand(n, generator=g) * 1e-3).half().to(DEV)
        call = lambda x: Q.int8_linear(x, w, s, convrot=True, convrot_groupsize=128)
    xs = [x_fp16(m, k, seed=72 + i, outliers=True).to(DEV) for i in range(3)]
    xin = xs[0].clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        call(xin)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        yg = call(xin)
    torch.cuda.synchronize()
    for i in range(6):
        xin.copy_(xs[i % 3])
        graph.replay()
        torch.cuda.synchronize()
        got = yg.clone()
        want = call(xs[i % 3])
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{kind}: replay {i} differs from the eager call"


@pytest.mark.parametrize("case", ["gauss_96x1024", "heavy_96x1024"])
@pytest.mark.parametrize("fmt,bits", [("w4a8", 4), ("w6a8", 6)])
def test_dequantize_w4a8_golden(case, fmt, bits):
    """The reference's stored W4A8/W6A8 tensors decode on the GPU to its error figures."""
    from inputs import selftest_inputs
    raw = np.load(os.path.join(HERE, "golden", "selftest_raw.npz"))
    meta = json.load(open(os.path.join(HERE, "golden", "selftest_sha256.json")))["cases"][case]["formats"][fmt]
    w = selftest_inputs((case,))[case]
    q = torch.from_numpy(raw[f"{case}/{fmt}/q"].reshape(96, -1).copy()).to(DEV)
    sr = torch.from_numpy(raw[f"{case}/{fmt}/s_rel"].reshape(96, -1).copy()).view(torch.float8_e4m3fn).to(DEV)
    sc = torch.from_numpy(raw[f"{case}/{fmt}/s_channel"].copy().view(np.float32)).to(DEV)
    key = f"{case}/{fmt}/codebook"
    cb = torch.from_numpy(raw[key].copy().view(np.float32)).to(DEV) if key in raw.files else None
    deq = qlin().dequantize_w4a8_int8_weight(q, sr, sc, cb, None, 16, 256).cpu().numpy()
    d = deq.astype(np.float64) - w
    rel = float(np.sqrt((d ** 2).sum() / (w.astype(np.float64) ** 2).sum()))
    assert rel == pytest.approx(meta["rel_fro"], rel=1e-6)
    assert float(np.abs(d).max()) == pytest.approx(meta["max_abs"], rel=1e-5)


def test_w4a8_declines():
    Q = qlin()
    q = torch.zeros(16, 128, dtype=torch.int8, device=DEV)
    sr = torch.ones(16, 16, device=DEV)
    sc = torch.ones(16, device=DEV)
    x = torch.randn(2, 256, device=DEV).half()
    with pytest.raises(Q.NoCapableBackendError):
        Q.w4a8_int8_linear(x, q, sr, sc, None, torch.zeros(16, 16, device=DEV))
    with pytest.raises(ValueError):  # lora_up without lora_down
        Q.w4a8_int8_linear(x, q, sr, sc, lora_up=torch.zeros(16, 1, device=DEV))
