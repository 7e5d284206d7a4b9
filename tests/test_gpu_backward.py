"""Input gradient of the frozen packed linears on the GPU (qlin.int8_linear_grad_input,
qlin.w4a8_linear_grad_input) and the autograd wrappers.

The reference's check (bench/bench_int8_backward.py:46-50): dx against the float32 CPU product
dy @ W with W the dequantized weight in the original basis, as relative Frobenius error.  Here W
comes from the oracle (rotate(q * s), or the W4A8 grid times s_channel, rotated) and the product
is taken in float64.  Bar: relative Frobenius error < 1e-3 and max error < 2e-2 of max |dx|, with
bf16 / fp16 outputs compared against the reference rounded to the same dtype.  Gradients as small
as the reference's bf16 case (2e-5) keep that accuracy (the row normalization).
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


def check(dx, ref, what):
    got = dx.float().cpu().numpy().astype(np.float64)
    want = torch.from_numpy(ref).to(dx.dtype).double().numpy() if dx.dtype != torch.float32 else ref
    assert np.isfinite(got).all(), what
    rel = O.rel_fro(got, want)
    mx = float(np.abs(got - want).max()) / max(float(np.abs(want).max()), 1e-300)
    assert rel < 1e-3 and mx < 2e-2, f"{what}: rel_fro={rel:.3e} max_rel={mx:.3e}"


def grad_ref(dy, w):
    return np.asarray(dy.float().cpu().numpy(), np.float64).reshape(-1, w.shape[0]) @ w.astype(np.float64)


INT8_CASES = [
    # m, n, k, group, dy dtype, out dtype, scale form, gradient magnitude
    (1, 256, 256, 256, torch.float16, None, "f32", 1.0),
    (37, 200, 512, 128, torch.bfloat16, None, "f16", 1.0),
    (64, 512, 384, 128, torch.float32, torch.float32, "scalar", 1.0),
    (130, 1024, 768, 0, torch.bfloat16, torch.float16, "f32", 2e-5),
    (300, 96, 1024, 256, torch.float16, torch.bfloat16, "f32", 1.0),
    (65, 33, 272, 16, torch.float16, torch.float32, "f32", 3.0),
    (1100, 256, 8192, 256, torch.bfloat16, None, "f32", 1.0),  # 288 workgroups: the two-per-CU kernel
    (40, 128, 65536, 256, torch.float16, None, "f32", 1.0),    # wide rows: dx of 65536 and 196608 values
    (8, 64, 196608, 128, torch.bfloat16, torch.float32, "f32", 1.0),
]


@pytest.mark.parametrize("m,n,k,g,dt,odt,sform,mag", INT8_CASES)
def test_int8_grad_input(m, n, k, g, dt, odt, sform, mag):
    Q = qlin()
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(0)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, g) if g else qz().quantize_int8_rowwise(w)
    sn = np.asarray(sn, np.float32).reshape(-1)
    if sform == "scalar":
        sn = sn[:1]
    scale = torch.from_numpy(sn)
    if sform == "f16":
        scale = scale.half()
    dy = (torch.randn(m, n, generator=torch.Generator().manual_seed(1)) * mag).to(dt)
    if m > 2:
        dy[2] = 0  # a zero row
    dx = Q.int8_linear_grad_input(dy.to(DEV), torch.from_numpy(qn).to(DEV), scale.to(DEV), g > 0, g or 256,
                                  out_dtype=odt)
    assert dx.shape == (m, k) and dx.dtype == (odt or dt)
    sf = scale.float().numpy()
    w_orig = O.dequantize_int8_convrot(qn, np.broadcast_to(sf, (n,)).copy(), g) if g else \
        qn.astype(np.float32) * np.broadcast_to(sf, (n,))[:, None]
    check(dx, grad_ref(dy, w_orig), f"int8 m={m} n={n} k={k} g={g}")
    if m > 2:
        assert torch.count_nonzero(dx[2]) == 0


def test_int8_grad_input_strided_and_batched():
    Q = qlin()
    n, k = 192, 512
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(2)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, 256)
    q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(np.asarray(sn, np.float32).reshape(-1)).to(DEV)
    wide = torch.randn(40, n + 24, generator=torch.Generator().manual_seed(3)).half().to(DEV)
    dy = wide[:, 8:8 + n]  # rows with a stride wider than N
    dx = Q.int8_linear_grad_input(dy, q, s, True, 256)
    w_orig = O.dequantize_int8_convrot(qn, np.asarray(sn, np.float32).reshape(-1), 256)
    check(dx, grad_ref(dy, w_orig), "strided")
    dy3 = dy.contiguous().reshape(4, 10, n)
    dx3 = Q.int8_linear_grad_input(dy3, q, s, True, 256)
    assert dx3.shape == (4, 10, k)
    torch.testing.assert_close(dx3.reshape(40, k), dx, rtol=0, atol=0)
    assert Q.int8_linear_grad_input(dy[:0], q, s, True, 256).shape == (0, k)


# group sizes 16 and 32 decode the grid element by element; 64 and 128 take the forward's
# 64-code segment decode
@pytest.mark.parametrize("bits,codebook,g,m,gs", [(4, "auto", 256, 48, 16), (4, None, 128, 7, 16), (6, None, 256, 100, 32),
                                                  (4, "auto", 256, 33, 128), (6, None, 128, 20, 64)])
def test_w4a8_grad_input(bits, codebook, g, m, gs):
    Q = qlin()
    n, k = 256, 1024
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(4)) * 0.02).numpy()
    q, s_rel, s_ch, book = qz().quantize_w4a8_int8_weight(w, bits=bits, group_size=gs, convrot_groupsize=g,
                                                          codebook=codebook)
    dy = torch.randn(m, n, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    dev = lambda t: None if t is None else t.to(DEV)
    dx = Q.w4a8_linear_grad_input(dev(dy), dev(q), dev(s_rel), dev(s_ch), dev(book), None, gs, g)
    sr = O.srel_to_f32(s_rel.view(torch.uint8).numpy(), "e4m3") if s_rel.dtype == torch.float8_e4m3fn else \
        s_rel.float().numpy()
    w_orig = O.dequantize_w4a8(q.numpy(), sr, s_ch.numpy(), None if book is None else book.numpy(), gs, g, bits)
    check(dx, grad_ref(dy, w_orig), f"w{bits}a8 g={g} m={m}")


def test_int8_trainable_autograd():
    """train/train_lora.py:187-188: forward = int8_linear, backward = the input gradient; the
    frozen operands get no gradient."""
    Q = qlin()
    n, k = 256, 512
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(6)) * 0.02).numpy()
    qn, sn = qz().quantize_int8_convrot_weight(w, 256)
    q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(np.asarray(sn, np.float32).reshape(-1)).to(DEV)
    bias = torch.randn(n, device=DEV).half()
    x = torch.randn(3, 11, k, generator=torch.Generator().manual_seed(7)).half().to(DEV).requires_grad_(True)
    y = Q.int8_linear_trainable(x, q, s, bias, True, 256)
    torch.testing.assert_close(y, Q.int8_linear(x.detach(), q, s, bias, convrot=True), rtol=0, atol=0)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(8)).half().to(DEV)
    y.backward(g)
    assert x.grad.dtype == x.dtype and x.grad.shape == x.shape
    torch.testing.assert_close(x.grad, Q.int8_linear_grad_input(g, q, s, True, 256), rtol=0, atol=0)
    w_orig = O.dequantize_int8_convrot(qn, np.asarray(sn, np.float32).reshape(-1), 256)
    check(x.grad.reshape(-1, k), grad_ref(g, w_orig), "autograd")


def test_packed_chain_trains_lora():
    """tests/test_training_packed.py:77-92, on the GPU: a stack of packed layers (W4 with a
    codebook, W6, INT8-ConvRot) with LoRA beside each, tanh between them; the loss reaches the
    input and every LoRA factor through the packed layers' input gradients."""
    Q = qlin()
    torch.manual_seed(9)
    d = 256
    layers = []
    for kind in ("w4", "w6", "int8"):
        w = (torch.randn(d, d) * 0.05).numpy()
        if kind == "int8":
            qn, sn = qz().quantize_int8_convrot_weight(w, 256)
            q, s = torch.from_numpy(qn).to(DEV), torch.from_numpy(np.asarray(sn, np.float32).reshape(-1)).to(DEV)
            layers.append(lambda x, q=q, s=s: Q.int8_linear_trainable(x, q, s, None, True, 256))
        else:
            bits = 4 if kind == "w4" else 6
            q, sr, sc, cb = qz().quantize_w4a8_int8_weight(w, bits=bits, group_size=16 if bits == 4 else 32,
                                                           convrot_groupsize=256)
            dev = lambda t: None if t is None else t.to(DEV)
            layers.append(lambda x, q=dev(q), sr=dev(sr), sc=dev(sc), cb=dev(cb), gs=16 if bits == 4 else 32:
                          Q.w4a8_linear_trainable(x, q, sr, sc, cb, None, None, gs, 256))
    downs = [torch.nn.Parameter(torch.randn(4, d, device=DEV) / 4) for _ in layers]
    ups = [torch.nn.Parameter(torch.randn(d, 4, device=DEV) * 0.01) for _ in layers]
    x = torch.randn(2, d, device=DEV, requires_grad=True)
    h = x
    for f, dn, up in zip(layers, downs, ups):
        h = (f(h) + (h @ dn.t()) @ up.t()).tanh()
    loss = h.square().mean()
    loss.backward()
    assert x.grad is not None and torch.isfinite(x.grad).all() and x.grad.abs().max() > 0
    for p in downs + ups:
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().max() > 0
    with pytest.raises(Q.NoCapableBackendError):
        Q.w4a8_linear_trainable(x, q, sr, sc, None, torch.zeros(16, d), None, 16, 256)
