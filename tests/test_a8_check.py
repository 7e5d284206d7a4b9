"""CPU checks of the A8 activation comparisons (tests/a8_check.py): the exact rotation passes, and
a rotation over the wrong group, a dropped factor, a large value two ulps off or a changed code
fails, and a value far smaller than its group may be off by the fp32 error bound."""
import numpy as np
import pytest
import torch

import oracle as O
from a8_check import assert_quantized_like_oracle, assert_rotation_close, exact_rotation_bits


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rotation_check(dt):
    x = (torch.randn(4, 1024, generator=torch.Generator().manual_seed(0)) * 3).to(dt)
    good = torch.from_numpy(exact_rotation_bits(x, 128).view(np.int16)).view(dt)
    assert_rotation_close(x, good, 128, "exact")
    wrong_g = torch.from_numpy(exact_rotation_bits(x, 256).view(np.int16)).view(dt)
    with pytest.raises(AssertionError):
        assert_rotation_close(x, wrong_g, 128, "wrong group")
    unscaled = (good.float() * 2.0).to(dt)  # 1/sqrt(128) = 1/(8 sqrt 2): a dropped sqrt 2 is off by far more
    with pytest.raises(AssertionError):
        assert_rotation_close(x, unscaled, 128, "scale")
    one_ulp = good.clone().view(torch.int16)
    one_ulp[0, :5] += 1
    assert_rotation_close(x, one_ulp.view(dt), 128, "five values one ulp off")
    # a value far from zero moved by two ulps is beyond the fp32 bound
    two = good.clone().view(torch.int16)
    j = int(good[1].float().abs().argmax())
    two[1, j] += 2
    with pytest.raises(AssertionError):
        assert_rotation_close(x, two.view(dt), 128, "two ulps at the row's largest value")


def test_rotation_check_allows_the_fp32_bound_on_cancelled_values():
    """Outputs (x0 - x1) / sqrt(128) of 20 and 20 + 2^-6: 0.00138, while the group's L1 norm over
    sqrt(128) is 3.54; the fp32 butterflies may be off there by 1.7e-6, about two fp16 ulps."""
    xt = torch.zeros(1, 128, dtype=torch.float32)
    xt[0, 0], xt[0, 1] = 20.0, 20.0 + 2.0 ** -6
    xt = xt.half()
    r = torch.from_numpy(exact_rotation_bits(xt, 128).view(np.int16)).view(torch.float16)
    small = int(r[0].float().abs().argmin())
    bump = r.clone().view(torch.int16)
    bump[0, small] += 2
    assert_rotation_close(xt, bump.view(torch.float16), 128, "a cancelled value two ulps off", rare=0.1)
    big = r.clone().view(torch.int16)
    big[0, int(r[0].float().abs().argmax())] += 2
    with pytest.raises(AssertionError):
        assert_rotation_close(xt, big.view(torch.float16), 128, "a large value two ulps off", rare=0.1)


def test_quantize_check():
    xr = torch.from_numpy(O.rotate(np.random.default_rng(1).standard_normal((3, 512)).astype(np.float16), 256))
    q, s = O.quantize_int8_rowwise(xr.numpy())
    assert_quantized_like_oracle(xr, torch.from_numpy(q), torch.from_numpy(s), "oracle itself")
    q2 = q.copy()
    q2[1, 7] ^= 1
    with pytest.raises(AssertionError):
        assert_quantized_like_oracle(xr, torch.from_numpy(q2), torch.from_numpy(s), "one code")
    s2 = s.copy().reshape(-1)
    s2[2] = np.nextafter(s2[2], np.float32(1))
    with pytest.raises(AssertionError):
        assert_quantized_like_oracle(xr, torch.from_numpy(q), torch.from_numpy(s2), "one scale")
