"""The C++ eager entry points (qlin/_qlin_torch.so) against the ctypes route of qlin/ops.py.

Plain linears (no LoRA, no residual) reach the C ABI through one C++ call; both routes run the same
kernels with the same operands, so their outputs must be identical bit for bit, their declines the
same exceptions, and a call captured in a HIP graph must replay to the eager result (the C++ route
takes a fresh workspace from the graph's pool during capture)."""
import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def qlin():
    import qlin as Q
    return Q


def both_routes(monkeypatch, fn):
    """(output of the C++ route, output of the ctypes route) of fn()."""
    from qlin import ops
    assert ops._FAST is not None, "the C++ module is not built"
    fast = fn()
    with monkeypatch.context() as mp:
        mp.setattr(ops, "_FAST", None)
        slow = fn()
    torch.cuda.synchronize()
    return fast, slow


def same(a, b, what):
    assert a.shape == b.shape and a.dtype == b.dtype, what
    assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"{what}: the two routes differ"


@pytest.mark.parametrize("m", [1, 8, 64, 100])
@pytest.mark.parametrize("name", ["Q4_K", "Q8_0", "Q6_K"])
def test_gguf_routes_agree(name, m, monkeypatch):
    n, k = 256, 1024
    raw = torch.from_numpy(random_gguf_blocks(name, n, k, seed=m)).to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half().to(DEV)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).to(DEV)
    Q = qlin()
    f, s = both_routes(monkeypatch, lambda: Q.gguf_linear(x, raw, name, (n, k), b))
    same(f, s, f"{name} M={m}")
    want = O.linear_ref(x.float().cpu().numpy(), O.gguf_dequantize(raw.cpu().numpy(), name, (n, k)), b.cpu().numpy())
    assert O.rel_fro(f.double().cpu().numpy(), want) < 1e-3
    # leading dims, a row-strided view and another output dtype
    x3 = torch.randn(2, 3, 2 * k, generator=torch.Generator().manual_seed(9)).half().to(DEV)[..., :k]
    f, s = both_routes(monkeypatch, lambda: Q.gguf_linear(x3, raw, name, (n, k), None, torch.float32))
    assert f.shape == (2, 3, n)
    same(f, s, f"{name} strided 3-D")


@pytest.mark.parametrize("m", [1, 5, 300])
def test_int8_routes_agree(m, monkeypatch):
    n, k, g = 384, 1024, 128
    q = torch.randint(-127, 128, (n, k), generator=torch.Generator().manual_seed(1), dtype=torch.int8).to(DEV)
    s = (torch.rand(n, generator=torch.Generator().manual_seed(2)) * 1e-3).half().to(DEV)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(DEV)
    Q = qlin()
    f, sl = both_routes(monkeypatch, lambda: Q.int8_linear(x, q, s, None, torch.float16, convrot=True,
                                                           convrot_groupsize=g))
    same(f, sl, f"int8 M={m}")
    f, sl = both_routes(monkeypatch, lambda: Q.int8_linear(x, q, s.reshape(n, 1)))
    same(f, sl, f"int8 M={m} no rotation, [N, 1] scale")


@pytest.mark.parametrize("m", [1, 40, 600])
@pytest.mark.parametrize("bits,gs", [(4, 128), (6, 64), (4, 16)])
def test_w4a8_routes_agree(m, bits, gs, monkeypatch):
    from qlin.quantize import pack_codes
    n, k = 320, 1024
    gen = torch.Generator().manual_seed(bits + m)
    hi = 15 if bits == 4 else 63
    q = pack_codes(torch.randint(1, hi + 1, (n, k), generator=gen, dtype=torch.int32), bits).to(DEV)
    s_rel = (2 + 2 * torch.rand(n, k // gs, generator=gen)).to(torch.float8_e4m3fn).to(DEV)
    s_ch = (torch.rand(n, generator=gen) * 2e-4 + 1e-4).to(DEV)
    x = torch.randn(m, k, generator=gen).half().to(DEV)
    b = torch.randn(n, generator=gen).half().to(DEV)
    Q = qlin()
    f, s = both_routes(monkeypatch, lambda: Q.w4a8_int8_linear(x, q, s_rel, s_ch, None, None, b, gs, 256))
    same(f, s, f"w{bits}a8 gs={gs} M={m}")


def test_routes_decline_alike(monkeypatch):
    Q = qlin()
    n, k = 64, 256
    raw = torch.from_numpy(random_gguf_blocks("Q4_0", n, k, seed=1)).to(DEV)
    x = torch.randn(4, k).half().to(DEV)
    cases = [
        (ValueError, lambda: Q.gguf_linear(x[:, :128], raw, "Q4_0", (n, k))),                # K mismatch
        (ValueError, lambda: Q.gguf_linear(x, raw[:-1], "Q4_0", (n, k))),                    # byte count
        (Q.NoCapableBackendError, lambda: Q.gguf_linear(x, raw.view(torch.int8), "Q4_0", (n, k))),
        (Q.NoCapableBackendError, lambda: Q.gguf_linear(x.cpu(), raw, "Q4_0", (n, k))),      # host tensor
        (Q.NoCapableBackendError, lambda: Q.gguf_linear(x.int(), raw, "Q4_0", (n, k))),
        (Q.NoCapableBackendError, lambda: Q.int8_linear(x, raw.view(n, -1), torch.ones(n, device=DEV))),
        (ValueError, lambda: Q.int8_linear(x, torch.zeros(n, k, dtype=torch.int8, device=DEV), torch.ones(n, device=DEV),
                                           torch.ones(n + 1, device=DEV))),
    ]
    from qlin import ops
    for exc, fn in cases:
        with pytest.raises(exc):
            fn()
        with monkeypatch.context() as mp:
            mp.setattr(ops, "_FAST", None)
            with pytest.raises(exc):
                fn()


def test_graph_capture_of_the_cpp_route():
    """Calls captured in a HIP graph take their workspace from the graph's pool; replays with eager
    calls of other shapes in between (which may grow the cached workspace) match the eager output."""
    Q = qlin()
    n, k = 512, 2048
    raw = torch.from_numpy(random_gguf_blocks("Q4_K", n, k, seed=5)).to(DEV)
    x = torch.randn(64, k, generator=torch.Generator().manual_seed(6)).half().to(DEV)
    want = Q.gguf_linear(x, raw, "Q4_K", (n, k))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        Q.gguf_linear(x, raw, "Q4_K", (n, k))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = Q.gguf_linear(x, raw, "Q4_K", (n, k))
    big = torch.randn(300, k).half().to(DEV)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {i}"
        Q.gguf_linear(big, raw, "Q4_K", (n, k))  # an eager call that needs a larger workspace
        torch.cuda.synchronize()
