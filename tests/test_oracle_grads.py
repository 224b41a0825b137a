"""Pins the oracle's stage-gradient restatement (accumulate_torch, norm_squared_torch).

accumulate_torch is the reference's own torch expression; it is pinned here against
numpy's IEEE binary32 arithmetic (a dropped unscale, a multiply instead of a
divide for a non-power-of-two scale, or a double-precision intermediate would all
change bits).  norm_squared_torch is pinned against exact integer arithmetic on
dyadic inputs, where every FP64 partial sum is exact in any order.
"""
import math

import numpy as np
import pytest
import torch

from oracle import reference as R


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("scale", [1.0, 128.0, 65536.0, 3.0, 0.1])
def test_accumulate_torch_is_ieee_binary32(dtype, scale):
    gen = torch.Generator().manual_seed(5)
    dst = torch.randn(4099, generator=gen) * 1e-2
    g = (torch.randn(4099, generator=gen) * (scale * 1e-3)).to(dtype)
    expect = dst.numpy().copy()
    R.accumulate_torch(dst, g, scale)
    gf = g.float().numpy()  # exact widening
    expect = (expect + gf / np.float32(scale)).astype(np.float32)
    assert np.array_equal(dst.numpy().view(np.uint32), expect.view(np.uint32))


def test_accumulate_torch_zero_plus_negative_zero_is_positive_zero():
    dst = torch.zeros(3)
    R.accumulate_torch(dst, torch.tensor([-0.0, 0.0, -0.0], dtype=torch.float16), 128.0)
    assert not torch.signbit(dst).any()


def test_norm_squared_torch_exact_on_dyadic_inputs():
    """k * 2^-10 with |k| < 2^11: squares k^2 2^-20, sums < 2^53 ulps -> exact in FP64."""
    gen = torch.Generator().manual_seed(9)
    ks = [torch.randint(-2047, 2048, (n,), generator=gen) for n in (1, 1048575, 1048577, 3000)]
    grads = [(k.double() / 1024).float() for k in ks]
    exact = sum(int((k.long() ** 2).sum()) for k in ks) / 2 ** 20
    assert R.norm_squared_torch(grads) == exact
    # chunking is part of the reference's order; the exact value is order-free
    assert R.norm_squared_torch(grads, chunk=4096) == exact


def test_norm_squared_torch_random_matches_fsum():
    gen = torch.Generator().manual_seed(10)
    grads = [torch.randn(n, generator=gen) * 1e-3 for n in (5, 70000, 1048577)]
    ref = math.fsum(float(x) ** 2 for g in grads for x in g.double().tolist())
    got = R.norm_squared_torch(grads)
    assert abs(got - ref) <= 1e-13 * ref


def test_norm_squared_torch_nonfinite():
    assert math.isinf(R.norm_squared_torch([torch.tensor([1.0, float("inf")])]))
    assert math.isnan(R.norm_squared_torch([torch.tensor([1.0, float("nan")])]))
