"""qlin_gguf_linear_noalloc: the GGUF linear with its workspace in the library's fixed per-GPU
scratch instead of a caller buffer.  Every call goes through the C ABI and must equal
qlin_gguf_linear (same kernels, caller workspace) bit for bit, on consecutive calls of different
sizes (the scratch keeps the previous call's contents), and match the oracle's linear.  Above 64
rows both decode the weight once at these sizes (the scratch holds the fp16 copy)."""
import numpy as np
import pytest
import torch

import oracle as O
from gguf_blocks import random_gguf_blocks

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _lib():
    from qlin import _lib as L
    return L


def noalloc(x, raw, name, n, k, bias=None, out_dtype=torch.float16):
    L = _lib()
    tid = O.gguf_type_id(name)
    y = torch.full((x.shape[0], n), float("nan"), dtype=out_dtype, device=DEV)
    st = L.load().qlin_gguf_linear_noalloc(L.desc(x), raw.data_ptr(), tid, n, k, L.desc(bias), L.desc(y),
                                           L.stream_of(x.device))
    L.check(st, "qlin_gguf_linear_noalloc")
    return y


def with_workspace(x, raw, name, n, k, bias=None, out_dtype=torch.float16):
    L = _lib()
    tid = O.gguf_type_id(name)
    y = torch.empty((x.shape[0], n), dtype=out_dtype, device=DEV)
    nbytes = L.load().qlin_workspace_size(L.OP_GGUF_LINEAR, x.shape[0], n, k, tid, L._TORCH_DT[x.dtype])
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    st = L.load().qlin_gguf_linear(L.desc(x), raw.data_ptr(), tid, n, k, L.desc(bias), L.desc(y), ws.data_ptr(),
                                   ws.numel(), L.stream_of(x.device))
    L.check(st, "qlin_gguf_linear")
    return y


def case(name, m, n, k, seed, xdt=torch.float16, odt=torch.float16, bias=False):
    raw = random_gguf_blocks(name, n, k, seed=seed)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(seed + 1)).to(xdt)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(seed + 2)) * 0.1).half() if bias else None
    return raw, x, b


@pytest.mark.parametrize("first,second", [
    # K split with 8 splits (8 MiB of partials), then a smaller K-split call
    (("Q4_K", 64, 4096, 4096, torch.float16, torch.float16, False), ("Q8_0", 20, 1024, 2048, torch.float16,
                                                                     torch.float16, True)),
    # bf16 activations (normalized into the scratch by the prologue), then one fp16 row (GEMV)
    (("Q6_K", 40, 3072, 4096, torch.bfloat16, torch.float32, True), ("IQ4_XS", 1, 2048, 4096, torch.float16,
                                                                     torch.float16, False)),
    # the weight decoded once into the scratch and the fp16 GEMM (above the split kernel's 512 rows),
    # then small M
    (("Q5_K", 600, 1024, 2048, torch.float16, torch.bfloat16, False), ("Q4_0", 8, 512, 1024, torch.float16,
                                                                       torch.float16, True)),
    # the split kernel's m-tiles (8 splits of partials in the scratch), then a single-split call
    (("Q4_K", 200, 1024, 2048, torch.float16, torch.float16, True), ("Q8_0", 512, 4096, 1024, torch.float16,
                                                                     torch.float16, False)),
])
def test_noalloc_matches_the_workspace_entry_point(first, second):
    for i, (name, m, n, k, xdt, odt, bias) in enumerate((first, second)):
        raw, x, b = case(name, m, n, k, seed=10 * i + m)
        rd, xd = torch.from_numpy(raw).to(DEV), x.to(DEV)
        bd = None if b is None else b.to(DEV)
        got = noalloc(xd, rd, name, n, k, bd, odt)
        want = with_workspace(xd, rd, name, n, k, bd, odt)
        torch.cuda.synchronize()
        what = f"call {i + 1}: {name} M={m} N={n} K={k}"
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), what + ": differs from qlin_gguf_linear"
        ref = O.linear_ref(x.float().numpy(), O.gguf_dequantize(raw, name, (n, k)),
                           None if b is None else b.float().numpy())
        if odt == torch.bfloat16:
            ref = torch.from_numpy(ref.astype(np.float32)).bfloat16().double().numpy()
        rel = O.rel_fro(got.double().cpu().numpy(), ref)
        assert rel < 1e-3, f"{what}: rel_fro {rel:.3e}"


def test_noalloc_rejects_calls_beyond_the_scratch():
    """A call whose workspace exceeds the fixed scratch is refused before anything is launched."""
    L = _lib()
    name, m, n, k = "Q4_0", 4096, 64, 4096         # 32 MiB of normalized rows > 16 MiB
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=DEV)
    raw = torch.zeros(n * k // 32 * 18, dtype=torch.uint8, device=DEV)
    y = torch.zeros(m, n, dtype=torch.float16, device=DEV)
    st = L.load().qlin_gguf_linear_noalloc(L.desc(x), raw.data_ptr(), O.gguf_type_id(name), n, k, None, L.desc(y),
                                           L.stream_of(x.device))
    assert st == L.QLIN_EWORKSPACE
    assert b"scratch" in L.load().qlin_last_error()
    torch.cuda.synchronize()
    assert int(y.abs().sum().item()) == 0
