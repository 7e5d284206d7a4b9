"""The layout carriers (TensorWiseINT8Layout, AsymW4A8Int8Layout, QuantizedTensor) on the host:
they hold the reference's own packed tensors unchanged and hand them back through
get_plain_tensors (tests/test_training_packed.py:54-66, train/train_lora.py:208, 219)."""
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
RAW = np.load(os.path.join(HERE, "golden", "selftest_raw.npz"))


def fixture(case, fmt, name, dtype=None):
    """The reference's stored bytes of one tensor, viewed as `dtype`."""
    a = RAW[f"{case}/{fmt}/{name}"].copy()
    return torch.from_numpy(a.view(dtype) if dtype is not None else a)


@pytest.mark.parametrize("case", ["gauss_96x1024", "heavy_96x1024"])
def test_int8_carrier_round_trips_the_reference_tensors(case):
    from qlin.layouts import QuantizedTensor, TensorWiseINT8Layout
    q = fixture(case, "int8_convrot", "q", np.int8).reshape(96, 1024)
    s = fixture(case, "int8_convrot", "scale", np.float32)
    p = TensorWiseINT8Layout.Params(scale=s, orig_dtype=torch.float32, orig_shape=(96, 1024), convrot=True,
                                    convrot_groupsize=256)
    w = QuantizedTensor(q, "TensorWiseINT8Layout", p)
    qd, sd = TensorWiseINT8Layout.get_plain_tensors(w)
    assert qd is q and sd is s                      # the tensors themselves, not copies
    assert w._layout_cls == "TensorWiseINT8Layout" and w.shape == (96, 1024) and w.dtype == torch.float32
    assert qd.dtype == torch.int8 and sd.shape == (96,)


@pytest.mark.parametrize("case", ["gauss_96x1024", "heavy_96x1024"])
@pytest.mark.parametrize("fmt", ["w4a8", "w6a8"])
def test_w4a8_carrier_round_trips_the_reference_tensors(case, fmt):
    from qlin.layouts import AsymW4A8Int8Layout, QuantizedTensor
    q = fixture(case, fmt, "q", np.int8).reshape(96, -1)
    s_rel = fixture(case, fmt, "s_rel").reshape(96, -1).view(torch.float8_e4m3fn)
    s_ch = fixture(case, fmt, "s_channel", np.float32)
    key = f"{case}/{fmt}/codebook"
    cb = torch.from_numpy(RAW[key].copy().view(np.float32)) if key in RAW.files else None
    p = AsymW4A8Int8Layout.Params(scale=s_rel, s_channel=s_ch, codebook=cb, correction=None, group_size=16,
                                  convrot_groupsize=256, orig_dtype=torch.bfloat16, orig_shape=(96, 1024))
    w = QuantizedTensor(q, "AsymW4A8Int8Layout", p)
    qd, sr, sc, corr, book = AsymW4A8Int8Layout.get_plain_tensors(w)
    assert qd is q and sr is s_rel and sc is s_ch and corr is None and book is cb
    assert w.shape == (96, 1024) and w.dtype == torch.bfloat16
    bits = q.shape[1] * 8 // 1024
    assert bits == (4 if fmt == "w4a8" else 6)


def test_carrier_declines_and_errors():
    import qlin
    from qlin.layouts import AsymW4A8Int8Layout, QuantizedTensor, TensorWiseINT8Layout, linear
    with pytest.raises(ValueError):
        QuantizedTensor(torch.zeros(4, 4, dtype=torch.int8), "NoSuchLayout", None)
    p = TensorWiseINT8Layout.Params(scale=torch.ones(8))
    w = QuantizedTensor(torch.zeros(8, 256, dtype=torch.int8), "TensorWiseINT8Layout", p)
    assert w.shape == (8, 256)
    with pytest.raises(qlin.NoCapableBackendError):   # host tensors: the kernels need a ROCm device
        linear(torch.zeros(2, 256, dtype=torch.float16), w)
    pa = AsymW4A8Int8Layout.Params(scale=torch.ones(8, 16), s_channel=torch.ones(8), group_size=16,
                                   correction=torch.zeros(16, 8))
    wa = QuantizedTensor(torch.zeros(8, 128, dtype=torch.int8), "AsymW4A8Int8Layout", pa)
    with pytest.raises(qlin.NoCapableBackendError):   # the asymmetric `correction` variant is declined
        linear(torch.zeros(2, 256, dtype=torch.float16), wa)
    with pytest.raises(TypeError):
        linear(torch.zeros(2, 256), torch.zeros(8, 256))


def test_residual_arguments_are_checked_on_the_host():
    import qlin
    x = torch.zeros(2, 256, dtype=torch.float16)
    q = torch.zeros(8, 256, dtype=torch.int8)
    with pytest.raises(qlin.NoCapableBackendError):   # well-formed, on the host: declined
        qlin.int8_linear(x, q, torch.ones(8), residual=torch.zeros(2, 8))
