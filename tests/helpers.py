"""Shared helpers for the GPU parity tests (inputs are made on the CPU, seeded)."""
import numpy as np
import torch

from oracle import reference as R

TORCH_TO_ORACLE = {torch.float32: R.DTYPE_F32, torch.float16: R.DTYPE_F16,
                   torch.bfloat16: R.DTYPE_BF16, None: R.DTYPE_NONE}


def to_oracle(t):
    """A CPU tensor as the numpy array the oracle takes (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).ravel()
    return t.numpy().ravel()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype.itemsize == 4 else a.view(np.uint16)


def export_bits(t):
    """Raw bits of an export tensor (fp16/bf16 -> uint16, fp32 -> uint32)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy().ravel().view(np.uint32)
    return t.view(torch.int16).numpy().ravel().view(np.uint16)


def oracle_export_bits(out, out_dtype):
    if out_dtype == torch.float32:
        return out.view(np.uint32)
    return out.view(np.uint16)


def oracle_hp_for(kind, step, lr=3e-4, betas=(.9, .95), eps=1e-8, wd=.1, scale=1.0, clip=None):
    if kind == "disk":
        return R.disk_adamw_hp(step, lr, clip, scale=scale)
    return R.torch_adamw_hp(lr, betas[0], betas[1], eps, wd, step, scale=scale, clip=clip)


def assert_same_bits(a, b, what):
    a, b = bits(a), bits(b)
    bad = np.flatnonzero(a != b)
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} elements differ, first at {bad[:5]}"
