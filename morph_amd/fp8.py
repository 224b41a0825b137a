"""Block-scaled FP8 (E4M3FN) transport on the GPU: streamtrain/precision.py:20-37.

pack_fp8 / unpack_fp8 keep the reference's signatures and results: per block of
256 elements an FP32 scale max(amax / 448, 1e-30) and one E4M3FN byte per
element (round to nearest even), and the inverse scaled into FP16 / BF16 /
FP32.  Both run as one kernel over device tensors (morph_fp8_pack/unpack).
"""
import ctypes

import torch

from . import _lib
from ._lib import check, dtype_code, lib, require_device_tensor, stream_handle

FP8_SUFFIXES = ('ffn.gate.weight', 'ffn.up.weight', 'ffn.down.weight')


def fp8_eligible(name):
    """precision.py:20-21: only the SwiGLU matrices travel in FP8."""
    return any(name.endswith(suffix) for suffix in FP8_SUFFIXES)


def _check_block(block_size):
    if block_size != _lib.FP8_BLOCK:
        raise ValueError(f"block_size must be {_lib.FP8_BLOCK}")


def pack_fp8(value, block_size=256, stream=None):
    """E4M3FN bytes (uint8, value.numel()) + FP32 per-block scales (ceil(n / 256))."""
    _check_block(block_size)
    require_device_tensor(value, "value")
    flat = value.detach().reshape(-1)
    n = flat.numel()
    encoded = torch.empty(n, dtype=torch.uint8, device=flat.device)
    scales = torch.empty(-(-n // block_size), dtype=torch.float32, device=flat.device)
    check(lib().morph_fp8_pack(ctypes.c_void_p(flat.data_ptr()), dtype_code(flat.dtype), n,
                               ctypes.c_void_p(encoded.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
                               stream_handle(stream)))
    return encoded, scales


def unpack_fp8(encoded, scales, dtype=torch.float16, block_size=256, stream=None):
    """dtype(float(byte) * scale) for every byte, as a flat tensor of encoded.numel()."""
    _check_block(block_size)
    require_device_tensor(encoded, "encoded")
    require_device_tensor(scales, "scales")
    if encoded.dtype != torch.uint8 or scales.dtype != torch.float32:
        raise TypeError("encoded must be uint8 and scales float32")
    n = encoded.numel()
    if scales.numel() < -(-n // block_size):
        raise ValueError("one scale per 256-element block expected")
    out = torch.empty(n, dtype=dtype, device=encoded.device)
    check(lib().morph_fp8_unpack(ctypes.c_void_p(encoded.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
                                 n, ctypes.c_void_p(out.data_ptr()), dtype_code(dtype),
                                 stream_handle(stream)))
    return out
