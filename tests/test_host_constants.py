"""The product's host constants (morph_amd.hyper) equal the oracle's, bit for bit."""
import ctypes
import itertools

import pytest

from morph_amd import hyper


def as_bytes(hp):
    return bytes(memoryview(hp).cast("B")) if hasattr(hp, "__buffer__") else ctypes.string_at(
        ctypes.addressof(hp), ctypes.sizeof(hp))


@pytest.mark.parametrize("lr,betas,eps,wd,scale", [
    (3e-4, (.9, .95), 1e-8, .1, 65536.), (3e-4, (.9, .95), 1e-8, 0., 1.),
    (1e-3, (.9, .999), 1e-8, .01, 128.), (2e-2, (.3, .5), 1e-6, .5, 3.),
    (1e-2, (.9, 0.), 1e-8, .1, 1024.)])
def test_adamw_constants_match_oracle(oracle, lr, betas, eps, wd, scale):
    for step in itertools.chain(range(1, 40), (100, 1000, 12345, 10 ** 6)):
        ours = hyper.adamw_constants(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps,
                                     weight_decay=wd, step=step, loss_scale=scale)
        ref = oracle.torch_adamw_hp(lr, betas[0], betas[1], eps, wd, step, scale=scale)
        assert as_bytes(ours) == as_bytes(ref), step


@pytest.mark.parametrize("lr,clip", [(.003, .25), (.001, 1.0), (3e-4, .037)])
def test_disk_constants_match_oracle(oracle, lr, clip):
    for step in range(1, 60):
        ours = hyper.disk_constants(step=step, lr=lr, clip=clip)
        ref = oracle.disk_adamw_hp(step, lr, clip)
        assert as_bytes(ours) == as_bytes(ref), step


def test_struct_layout_matches_header():
    """morph_adamw_hp is 10 floats + 2 uint32 = 48 bytes; morph_adamw_tensor is 56."""
    from morph_amd._lib import AdamwHP, AdamwTensor
    assert ctypes.sizeof(AdamwHP) == 48
    assert ctypes.sizeof(AdamwTensor) == 56


def test_rejects_bad_inputs():
    with pytest.raises(ValueError):
        hyper.adamw_constants(lr=1e-3, beta1=.9, beta2=.95, eps=1e-8, weight_decay=0, step=0)
    with pytest.raises(ValueError):
        hyper.adamw_constants(lr=1e-3, beta1=.9, beta2=.95, eps=1e-8, weight_decay=0, step=1,
                              loss_scale=0.)
