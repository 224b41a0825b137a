"""The C-ABI library loads and exports every symbol include/*.h declares (no GPU calls)."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]

# These tests hand the entry points fake (never allocated) device addresses to show that
# validation rejects the call before anything is launched.  Should a check ever regress,
# a launch at those addresses must not reach a GPU: they run only where none is visible.
no_gpu_visible = pytest.mark.skipif(torch.cuda.is_available(),
                                    reason="passes fake device pointers; runs only without a GPU")


def declared_functions():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(morph_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_expected_entry_points():
    from morph_amd._lib import EXPORTS
    assert set(declared_functions()) == set(EXPORTS)


def test_library_exports_every_declared_symbol():
    from morph_amd import _lib
    lib = _lib.lib()  # loads; raises ImportError if not built
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_status_strings():
    from morph_amd import _lib
    lib = _lib.lib()
    assert lib.morph_abi_version() == _lib.ABI_VERSION == 9
    assert lib.morph_strerror(0) == b"ok"
    for code in (-1, -2, -3, -4, -5):
        assert lib.morph_strerror(code) not in (b"ok", b"unknown morph status")
    assert lib.morph_strerror(-99) == b"unknown morph status"


@no_gpu_visible
def test_argument_validation_happens_before_any_launch():
    """Invalid calls return a negative status and never reach the GPU."""
    from morph_amd import _lib
    lib = _lib.lib()
    assert lib.morph_flag_clear(None, None) == -1
    assert lib.morph_nonfinite_or(None, 1, 10, None, None) == -1
    flag = ctypes.c_uint32(0)
    assert lib.morph_nonfinite_or(None, 7, 0, ctypes.byref(flag), None) == -2
    hp = _lib.AdamwHP()
    assert lib.morph_adamw_fused(None, 1, None, None, None, None, -1, 10, ctypes.byref(hp),
                                 None, None) == -1
    assert lib.morph_adamw_fused(None, 9, None, None, None, None, -1, 0, ctypes.byref(hp),
                                 None, None) == -2
    assert lib.morph_adamw_multi(None, -1, 1, -1, None, 0, None, None, None, None) == -1
    # step slots are 0 or 1; the fused detector + close validates before any launch
    st = ctypes.c_void_p(0x10000)
    assert lib.morph_step_end(st, None, None, 0, 2, None) == -1
    assert lib.morph_step_end(None, None, None, 0, 0, None) == -1
    assert lib.morph_adamw_multi_dev(None, 0, 1, -1, None, None, 0, None, st, 2, None, None,
                                     None) == -1
    close = lambda *a: lib.morph_nonfinite_or_close(*a)
    assert close(None, None, 0, 1, None, 0, None, None, 0, None) == -1      # no state
    assert close(None, None, 0, 1, st, 2, None, None, 0, None) == -1        # bad slot
    assert close(None, None, 0, 1, st, 0, None, None, 3, None) == -1        # clock list missing
    assert close(None, None, 0, 7, st, 0, None, None, 0, None) == -2        # unknown dtype
    # allocation-free final pass: more partials than its array holds -> ERANGE, no launch
    big = (_lib.AccumTensor * 1)()
    big[0].grad, big[0].dst, big[0].numel = None, 0x10000, (1 << 31) + 1
    assert lib.morph_grad_partials(big, 1) == _lib.NOALLOC_MAX_PARTIALS + 1
    assert lib.morph_grad_accumulate_final_noalloc(big, 1, 1, 1.0, 0, st, st, None) == -4
    big[0].numel = 1 << 31
    assert lib.morph_grad_partials(big, 1) == _lib.NOALLOC_MAX_PARTIALS
    # conversion: grid limits of the copy (FP32) and of the 16-bit conversions -> ERANGE
    src, dst = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000)
    conv = lambda dtype, n: lib.morph_convert_f32(src, dst, dtype, ctypes.c_int64(n), None, None)
    assert conv(_lib.DTYPE_F32, 256 * (2 ** 31 - 1) + 1) == -4
    assert conv(_lib.DTYPE_F16, 2048 * (2 ** 31 - 1) + 1) == -4
    assert conv(5, 10) == -2 and conv(_lib.DTYPE_F32, -1) == -1
    # GEMM: validated on the host (fake, aligned pointers are never dereferenced)
    p = ctypes.c_void_p(0x10000)
    gemm = lambda M, N, K, flags, Ct=None: lib.morph_gemm_nt_bf16(
        p, p, None, p, Ct, M, N, K, 1, K, K, 0, N, M, 0, 0, 0, 0, 0, 1.0, 0.0, flags, None)
    assert gemm(256, 256, 64, 4) == -1                   # unknown flag bit
    assert gemm(256, 256, 64, _lib.GEMM_SYMMETRIC | _lib.GEMM_Q_KN) == -1
    assert gemm(256, 512, 64, _lib.GEMM_SYMMETRIC) == -1  # symmetric needs M == N
    assert gemm(256, 256, 64, _lib.GEMM_SYMMETRIC, Ct=p) == -1
    assert gemm(100, 256, 64, 0) == -4                    # not a tile multiple
    assert gemm(256, 256, 0, 0) == -1
    # the output may not overlap an operand (other tiles still read it); D may alias C
    q, c = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x200000)
    ok = lambda C, flags=0, D=None: lib.morph_gemm_nt_bf16(
        p, q, D, C, None, 256, 256, 64, 1, 64, 256 if flags else 64, 256, 256, 0, 0, 0, 0, 0, 0,
        1.0, 0.0, flags, None)
    assert ok(p) == -1 and ok(q) == -1 and ok(q, _lib.GEMM_Q_KN) == -1
    assert ok(ctypes.c_void_p(0x100000 + 2 * 64 * 256 - 16), _lib.GEMM_Q_KN) == -1  # last Q bytes


@no_gpu_visible
def test_muon_matrix_flags_are_validated():
    """transposed must be 0 or 1 and reserved 0, checked before any launch."""
    from morph_amd import _lib
    lib = _lib.lib()
    p = 0x10000
    hp = _lib.MuonHP()
    hp.ns_steps = 5
    for transposed, reserved in ((2, 0), (-1, 0), (0, 1)):
        arr = (_lib.MuonMatrix * 1)()
        arr[0].grad, arr[0].momentum, arr[0].param = p, p, p
        arr[0].transposed, arr[0].reserved = transposed, reserved
        assert lib.morph_muon_step(arr, 1, 256, 512, ctypes.byref(hp), ctypes.c_void_p(p),
                                   1 << 40, None) == -1


@no_gpu_visible
def test_muon_finish_range_rejects_ranges_outside_the_batch():
    """0 <= first, 0 <= n, first + n <= count: n = -1 is not "the rest of the batch"."""
    from morph_amd import _lib
    lib = _lib.lib()
    p = 0x10000
    hp = _lib.MuonHP()
    hp.ns_steps = 5
    arr = (_lib.MuonMatrix * 2)()
    for i in range(2):
        arr[i].grad, arr[i].momentum, arr[i].param = p, p, p
    fin = lambda first, n: lib.morph_muon_finish_range(arr, 2, 256, 512, ctypes.byref(hp), 0,
                                                       first, n, ctypes.c_void_p(p), 1 << 40, None)
    for first, n in ((0, -1), (-1, 1), (1, 2), (3, 0), (0, 3)):
        assert fin(first, n) == -1, (first, n)


# (ctypes class, C type) pairs whose layouts must agree field by field
STRUCTS = [("AdamwHP", "morph_adamw_hp"), ("AdamwTensor", "morph_adamw_tensor"),
           ("StepState", "morph_step_state"), ("AdamwSched", "morph_adamw_sched"),
           ("AccumTensor", "morph_accum_tensor"), ("MuonMatrix", "morph_muon_matrix"),
           ("MuonHP", "morph_muon_hp")]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs a host C compiler")
def test_ctypes_struct_layouts_match_the_header(tmp_path):
    """sizeof and every field offset of the ctypes mirrors equal the C compiler's."""
    from morph_amd import _lib
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "morph_optim.h"',
             'int main(void) {']
    for cls, ctype in STRUCTS:
        lines.append(f'  printf("{cls} size %zu\\n", sizeof({ctype}));')
        for field, *_ in getattr(_lib, cls)._fields_:
            lines.append(f'  printf("{cls} {field} %zu\\n", offsetof({ctype}, {field}));')
    lines += ['  return 0;', '}']
    (tmp_path / "layout.c").write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), "-o", str(tmp_path / "layout"),
                    str(tmp_path / "layout.c")], check=True)
    out = subprocess.run([str(tmp_path / "layout")], check=True, capture_output=True, text=True)
    for line in out.stdout.splitlines():
        cls, field, value = line.split()
        struct = getattr(_lib, cls)
        got = ctypes.sizeof(struct) if field == "size" else getattr(struct, field).offset
        assert got == int(value), (cls, field, got, value)


def test_gemm_flag_values_match_header():
    from morph_amd import _lib
    text = (ROOT / "include" / "morph_optim.h").read_text()
    for name, value in (("MORPH_GEMM_SYMMETRIC", _lib.GEMM_SYMMETRIC),
                        ("MORPH_GEMM_Q_KN", _lib.GEMM_Q_KN),
                        ("MORPH_GEMM_TILE_M", _lib.GEMM_TILE_M),
                        ("MORPH_GEMM_TILE_K", _lib.GEMM_TILE_K)):
        assert re.search(rf"#define {name} {value}\b", text), name


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from morph_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.lib()
