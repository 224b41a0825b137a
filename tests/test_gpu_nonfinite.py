"""GPU parity: the non-finite detector's decision equals the oracle's, exactly."""
import numpy as np
import pytest
import torch

from morph_amd import kernels
from tests.helpers import TORCH_TO_ORACLE, to_oracle

pytestmark = pytest.mark.gpu


def detect(grads):
    flag = kernels.new_flag()
    kernels.flag_clear(flag)
    kernels.nonfinite_or([g.cuda() for g in grads], flag)
    torch.cuda.synchronize()
    return bool(flag.item())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 8, 4096, 8191, 8192, 8193, 100003, 2 ** 20 + 5])
def test_single_poison_anywhere(dtype, n):
    from oracle import reference as R
    g = torch.randn(n, generator=torch.Generator().manual_seed(n)).to(dtype)
    assert not detect([g])
    positions = sorted({0, n - 1, n // 2, max(0, n - 8), min(n - 1, 8191)})
    for pos in positions:
        for bad in (float("inf"), float("-inf"), float("nan")):
            h = g.clone()
            h[pos] = bad
            expect = R.nonfinite_any(to_oracle(h), TORCH_TO_ORACLE[dtype])
            assert expect
            assert detect([h]), (pos, bad)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("offset", [1, 3])
def test_unaligned_views(dtype, offset):
    """A gradient view that starts off a 16-byte boundary takes the element path: a
    non-finite value is found at either end and in the middle, and a finite view
    (with a poisoned element just before it, outside the view) is not flagged."""
    n = 10001
    base = torch.randn(n + offset, generator=torch.Generator().manual_seed(offset)).to(dtype)
    base[offset - 1] = float("nan")  # outside the view
    dev = base.cuda()
    assert not detect([dev[offset:]])
    for pos in (0, n // 2, n - 1):
        h = dev.clone()
        h[offset + pos] = float("inf")
        assert detect([h[offset:]]), pos


def test_finite_extremes_never_flag():
    f16 = torch.tensor([65504., -65504., 6e-8, -6e-8, 0., -0.] * 1000, dtype=torch.float16)
    bf16 = torch.tensor([3.38e38, -3.38e38, 1e-38, 0.] * 1000, dtype=torch.bfloat16)
    f32 = torch.tensor([3.4028235e38, -3.4028235e38, 1e-45, 0.] * 1000, dtype=torch.float32)
    assert not detect([f16])
    assert not detect([bf16])
    assert not detect([f32])


def test_multi_tensor_or_and_flag_accumulates():
    gen = torch.Generator().manual_seed(0)
    grads = [torch.randn(int(n), generator=gen).half() for n in (5, 4096, 70001, 3, 0, 12345)]
    assert not detect(grads)
    grads[3][2] = float("nan")
    assert detect(grads)
    # several calls OR into one flag and nothing ever clears it but flag_clear
    flag = kernels.new_flag()
    kernels.flag_clear(flag)
    kernels.nonfinite_or([grads[3].cuda()], flag)
    kernels.nonfinite_or([grads[0].cuda()], flag)
    torch.cuda.synchronize()
    assert flag.item() == 1
    kernels.flag_clear(flag)
    torch.cuda.synchronize()
    assert flag.item() == 0


def test_random_poison_matches_oracle():
    from oracle import reference as R
    rng = np.random.RandomState(1)
    for trial in range(60):
        n = int(rng.randint(1, 200000))
        dtype = [torch.float16, torch.bfloat16, torch.float32][trial % 3]
        g = torch.from_numpy((rng.randn(n) * 10 ** rng.uniform(-6, 4)).astype(np.float32))
        g = g.to(dtype)
        for _ in range(int(rng.randint(0, 3))):
            g[int(rng.randint(n))] = float(rng.choice([np.inf, -np.inf, np.nan]))
        assert detect([g]) == R.nonfinite_any(to_oracle(g), TORCH_TO_ORACLE[dtype])


def test_many_tensors_beyond_one_launch():
    """More tensors than one launch descriptor holds; the poison is in the last one."""
    grads = [torch.ones(17 + i, dtype=torch.float16) for i in range(400)]
    assert not detect(grads)
    for k in (0, 159, 160, 399):  # first, last of a launch, first of the next, last
        h = [g.clone() for g in grads]
        h[k][-1] = float("inf")
        assert detect(h), k
