"""GPU FP8 block-scaled pack/unpack (morph_amd.fp8) against the oracle (precision.py:24-37).

Bytes (NaN codes included) and scales bit-exact for FP32/FP16/BF16 inputs, ragged sizes
and wide dynamic range (subnormal codes); exhaustive conversion sweeps over every finite FP16 value and
every FP32 value with |v| <= 448 at scale 1; zero and NaN blocks; unpack of all 256 codes at several
scales into FP16/BF16/FP32; the reference's 4% roundtrip bound.
"""
import numpy as np
import pytest
import torch

from morph_amd import fp8
from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def same(a, b):
    """Bitwise equality: exact for E4M3FN bytes (NaN codes and their signs included);
    for floats, with any NaN equal to any NaN (scales and unpacked values)."""
    a, b = a.cpu(), b.cpu()
    if a.dtype == torch.uint8:
        return torch.equal(a, b)
    an, bn = torch.isnan(a.float()), torch.isnan(b.float())
    view = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}[a.dtype]
    return torch.equal(an, bn) and torch.equal(a[~an].view(view), b[~bn].view(view))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 255, 256, 257, 519, 70001])
def test_pack_bitexact_vs_reference(dtype, n):
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=gen) * torch.exp(torch.randn(n, generator=gen) * 4)  # wide range
    x = x.to(dtype)
    enc, sc = fp8.pack_fp8(x.to(DEV))
    renc, rsc = R.pack_fp8_torch(x)
    assert same(sc, rsc) and same(enc, renc)


def test_conversion_exhaustive_over_fp16_values():
    """Blocks led by 448 have scale exactly 1, so bytes are the plain conversion of every
    finite FP16 value in [-448, 448] (and of random FP32 values)."""
    h = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(torch.float16).float()
    vals = h[torch.isfinite(h) & (h.abs() <= 448)]
    vals = torch.cat([vals, (torch.rand(100000, generator=torch.Generator().manual_seed(1)) - .5) * 896])
    blocks = vals.split(255)
    x = torch.cat([torch.cat([torch.tensor([448.0]), b, torch.zeros(255 - b.numel())]) for b in blocks])
    enc, sc = fp8.pack_fp8(x.to(DEV))
    assert torch.equal(sc.cpu(), torch.ones_like(sc.cpu()))
    assert torch.equal(enc.cpu(), x.to(torch.float8_e4m3fn).view(torch.uint8))


def test_conversion_every_fp32_value_in_range():
    """Every FP32 value in [-448, 448] (both signs of all 1,138,753,537 magnitudes up to
    448) in blocks led by 448, so the scale is 1 and the bytes are the plain E4M3FN
    conversion of each value (the kernel converts with gfx950's v_cvt_pk_fp8_f32),
    against torch's conversion on the GPU, which is checked against torch's CPU
    conversion on a sample."""
    top = 0x43E00000  # bits of 448.0
    sample = torch.randint(0, top + 1, (1 << 20,), generator=torch.Generator().manual_seed(9),
                           dtype=torch.int32).view(torch.float32)
    assert torch.equal(sample.to(DEV).to(torch.float8_e4m3fn).view(torch.uint8).cpu(),
                       sample.to(torch.float8_e4m3fn).view(torch.uint8))
    step = 255 << 19
    for lo in range(0, top + 1, step):
        x = torch.arange(lo, min(lo + step, top + 1), dtype=torch.int32, device=DEV).view(torch.float32)
        x = torch.cat([x, torch.zeros((-x.numel()) % 255, device=DEV)]).view(-1, 255)
        for sign in (1.0, -1.0):
            blocks = torch.cat([torch.full((x.shape[0], 1), 448.0, device=DEV), x * sign], 1).view(-1)
            enc, sc = fp8.pack_fp8(blocks)
            assert bool((sc == 1.0).all())
            assert torch.equal(enc, blocks.to(torch.float8_e4m3fn).view(torch.uint8)), (lo, sign)
        del x, blocks, enc, sc


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_blocks_with_infinities(dtype):
    """A block holding +-inf has scale inf: its finite elements encode as +-0 and the
    infinities as NaN (inf / inf), as the reference's division gives; -0 in a finite
    block stays -0."""
    x = torch.randn(1024, generator=torch.Generator().manual_seed(3))
    x[5], x[300], x[301], x[700] = float("inf"), float("-inf"), float("inf"), float("nan")
    x[800], x[801] = -0.0, 0.0  # signed zeros in a finite block keep their sign
    x = x.to(dtype)
    enc, sc = fp8.pack_fp8(x.to(DEV))
    renc, rsc = R.pack_fp8_torch(x)
    assert same(sc, rsc) and same(enc, renc)
    assert torch.isinf(sc[0].cpu()) and torch.isinf(sc[1].cpu()) and torch.isnan(sc[2].cpu())
    assert enc[800].item() == 0x80 and enc[801].item() == 0
    assert enc[5].item() == enc[300].item() == 0xFF  # inf / inf: the negative default NaN


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_zero_and_nan_blocks(dtype):
    """A zero block has scale 1e-30; a block with a NaN has a NaN scale and NaN bytes
    whose signs follow the reference's ops: 0x7F for every element but a NaN one,
    which keeps its own sign (x86 division returns its first NaN operand)."""
    x = torch.zeros(1024)
    x[256:512] = torch.linspace(-1, 1, 256)
    x[300], x[301] = float("nan"), -float("nan")
    x[600:700] = torch.linspace(-1, 1, 100)
    x[900] = -float("nan")
    x = x.to(dtype)
    enc, sc = fp8.pack_fp8(x.to(DEV))
    renc, rsc = R.pack_fp8_torch(x)
    assert same(sc, rsc) and same(enc, renc)
    assert sc[0].item() == np.float32(1e-30) and torch.isnan(sc[1].cpu())
    bits = x.float().view(torch.int32)  # the NaNs' signs after the cast to dtype
    assert enc[256].item() == 0x7F
    for i in (300, 301, 900):
        assert enc[i].item() == (0xFF if bits[i] < 0 else 0x7F)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("offset", [1, 3, 8])
def test_unaligned_views(dtype, offset):
    """Views that start off a 16-byte boundary take the element-wise loads (source) and
    byte-wise loads (encoded); bytes, scales and decoded values still equal the reference's."""
    gen = torch.Generator().manual_seed(offset)
    base = (torch.randn(5000 + offset, generator=gen) * 3).to(dtype)
    x = base[offset:]
    enc, sc = fp8.pack_fp8(base.to(DEV)[offset:])
    renc, rsc = R.pack_fp8_torch(x)
    assert same(sc, rsc) and same(enc, renc)
    padded = torch.cat([torch.zeros(offset, dtype=torch.uint8), renc]).to(DEV)
    for out in (torch.float16, torch.bfloat16, torch.float32):
        got = fp8.unpack_fp8(padded[offset:], rsc.to(DEV), out)
        assert same(got, R.unpack_fp8_torch(renc, rsc, out))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_unpack_all_codes_bitexact(dtype):
    codes = torch.arange(256, dtype=torch.uint8).repeat(5)
    scales = torch.tensor([1.0, 1e-30, 0.01, 3.5, 2.0 ** 20], dtype=torch.float32)
    got = fp8.unpack_fp8(codes.to(DEV), scales.to(DEV), dtype)
    assert same(got, R.unpack_fp8_torch(codes, scales, dtype))


def test_reference_roundtrip_bound_on_gpu():
    torch.manual_seed(2)
    values = torch.randn(519)
    enc, sc = fp8.pack_fp8(values.to(DEV))
    restored = fp8.unpack_fp8(enc, sc, torch.float32).cpu()
    assert (restored - values).norm() / values.norm() < .04
    assert not fp8.fp8_eligible('embedding.weight') and fp8.fp8_eligible('blocks.3.ffn.up.weight')


def test_config2_window_roundtrip_matches_reference_full_size():
    """A full [6144, 3072] FP16 weight against the reference's ops on the CPU, where the
    reference packs (disk.py:330-345 packs slot.host).  torch's GPU kernels would not do:
    they divide by the Python scalar 448 as a multiply by its rounded reciprocal."""
    gen = torch.Generator(device=DEV).manual_seed(4)
    w = (torch.randn(6144, 3072, generator=gen, device=DEV) * .02).half()
    enc, sc = fp8.pack_fp8(w)
    renc, rsc = R.pack_fp8_torch(w.cpu())
    assert same(sc, rsc) and same(enc, renc)
    assert same(fp8.unpack_fp8(enc, sc, torch.float16), R.unpack_fp8_torch(renc, rsc, torch.float16))
