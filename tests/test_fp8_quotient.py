"""The FP8 pack kernel's quotient for 16-bit inputs, checked exhaustively on the CPU.

morph_amd/csrc/fp8.hip divides a block's FP16/BF16 elements by the block scale
(streamtrain/precision.py:27-31) as Markstein's correction of |x| * (1 / s), with
x's sign put back, rather than one IEEE division per element.  tests/csrc/fp8_quotient_check.c runs that
sequence (binary32 multiply and fused multiply-adds, as on the device) against
the IEEE quotient for every block maximum and every element up to it: every
FP16 quotient is identical, and the BF16 quotients that differ are those of
subnormal elements, all below 2^-10, where E4M3FN encodes zero either way, so
every byte is identical.  The GPU tests then compare the kernel's bytes with
the reference's CPU ops (tests/test_gpu_fp8.py).
"""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).parent / "csrc" / "fp8_quotient_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path_factory.mktemp("fp8q") / "fp8_quotient_check"
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    return exe


def run(checker, fmt):
    out = subprocess.run([str(checker), fmt], check=True, capture_output=True, text=True).stdout
    pairs, qbad, bbad, worst = out.split()
    return int(pairs), int(qbad), int(bbad), float.fromhex(worst)


def test_fp16_quotients_identical(checker):
    pairs, qbad, bbad, _ = run(checker, "fp16")
    assert pairs == 503856640  # 31744 finite magnitudes: every (amax, x <= amax) pair
    assert qbad == 0 and bbad == 0


def test_bf16_bytes_identical(checker):
    pairs, qbad, bbad, worst = run(checker, "bf16")
    assert pairs == 32640 * 32641 // 2
    assert bbad == 0
    # the differing quotients are all far below E4M3FN's smallest rounding step (2^-10)
    assert qbad > 0 and worst < 2.0 ** -10
