"""Pins the oracle's FP8 restatement (precision.py:24-37) and torch's E4M3FN conversion.

- the reference's own assertion (tests/test_fp16.py:16-19): a packed/unpacked
  randn(519) is within 4% relative error;
- torch's decode of all 256 bytes equals the format definition (1-4-3, bias 7, no
  infinities, S.1111.111 = NaN);
- torch's encode is round-to-nearest-even: every representable value maps to its own
  byte, every midpoint between neighbours to the even one, values just off a midpoint
  to the nearer one.
"""
import math

import pytest
import torch

from oracle import reference as R


def test_reference_roundtrip_assertion():
    torch.manual_seed(2)
    values = torch.randn(519)
    encoded, scales = R.pack_fp8_torch(values)
    restored = R.unpack_fp8_torch(encoded, scales, torch.float32)
    assert (restored - values).norm() / values.norm() < .04
    assert encoded.dtype == torch.uint8 and encoded.numel() == 519 and scales.numel() == 3


def test_torch_decode_equals_format_definition():
    decoded = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().tolist()
    for b, v in enumerate(decoded):
        ref = R.e4m3fn_value(b)
        assert (math.isnan(v) and math.isnan(ref)) or v == ref, (b, v, ref)
    assert max(abs(R.e4m3fn_value(b)) for b in range(256) if not math.isnan(R.e4m3fn_value(b))) == 448


def test_torch_encode_is_round_to_nearest_even():
    finite = sorted({R.e4m3fn_value(b) for b in range(128) if not math.isnan(R.e4m3fn_value(b))})
    enc = lambda xs: torch.tensor(xs, dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).tolist()
    assert enc(finite) == [next(b for b in range(128) if R.e4m3fn_value(b) == v) for v in finite]
    lo, hi = finite[:-1], finite[1:]
    mids = [(a + b) / 2 for a, b in zip(lo, hi)]
    got = enc(mids)
    for a, b, g in zip(lo, hi, got):
        code_a, code_b = enc([a])[0], enc([b])[0]
        assert g == (code_a if code_a % 2 == 0 else code_b)
    above = enc([m * (1 + 2 ** -20) for m in mids])
    assert above == enc(hi)


@pytest.mark.parametrize("n", [1, 255, 256, 257])
def test_pack_sizes_and_zero_block_scale(n):
    encoded, scales = R.pack_fp8_torch(torch.zeros(n))
    assert encoded.numel() == n and scales.numel() == -(-n // 256)
    assert (encoded == 0).all() and (scales == torch.tensor(1e-30, dtype=torch.float32)).all()
