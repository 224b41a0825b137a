"""morph_host_copy: the library's host copy pool behind the pinned staging (host only, no GPU)."""
import ctypes
import os
import threading

import pytest
import torch

from morph_amd import _lib, staging

MIB = 1 << 20


def _copy(dst, src, nbytes, threads, dst_off=0, src_off=0):
    L = _lib.lib()
    return L.morph_host_copy(ctypes.c_void_p(dst.data_ptr() + dst_off),
                             ctypes.c_void_p(src.data_ptr() + src_off), nbytes, threads)


@pytest.mark.parametrize("nbytes", [0, 1, 63, MIB - 3, MIB + 17, 3 * MIB + 5, 37 * MIB + 1])
@pytest.mark.parametrize("threads", [1, 2, 3, 8, 16, 64])
def test_copies_every_byte(nbytes, threads):
    gen = torch.Generator().manual_seed(nbytes * 131 + threads)
    src = torch.randint(0, 256, (nbytes + 16,), dtype=torch.uint8, generator=gen)
    dst = torch.zeros(nbytes + 16, dtype=torch.uint8)
    # odd offsets: pieces start wherever the split falls, not at an alignment
    assert _copy(dst, src, nbytes, threads, dst_off=3, src_off=5) == 0
    assert torch.equal(dst[3:3 + nbytes], src[5:5 + nbytes])
    assert not dst[:3].any() and not dst[3 + nbytes:].any()  # nothing outside the range


def test_errors_are_reported_before_any_copy():
    L = _lib.lib()
    buf = torch.zeros(4 * MIB, dtype=torch.uint8)
    p = ctypes.c_void_p(buf.data_ptr())
    q = ctypes.c_void_p(buf.data_ptr() + 2 * MIB)
    assert L.morph_host_copy(None, p, 16, 4) == -1
    assert L.morph_host_copy(q, None, 16, 4) == -1
    assert L.morph_host_copy(q, p, 16, 0) == -1
    assert L.morph_host_copy(q, p, 16, 65) == -4
    assert L.morph_host_copy(None, None, 0, 0) == 0  # nothing to copy
    # overlapping ranges (memcpy semantics) are refused in both directions
    assert L.morph_host_copy(ctypes.c_void_p(buf.data_ptr() + 1), p, 2 * MIB, 4) == -1
    assert L.morph_host_copy(p, ctypes.c_void_p(buf.data_ptr() + 1), 2 * MIB, 4) == -1
    assert L.morph_host_copy(q, p, 2 * MIB, 4) == 0  # adjacent, not overlapping


def test_concurrent_callers_each_get_their_own_copy():
    """Calls from several threads are serialized; each one copies its own ranges."""
    n = 9 * MIB + 7
    srcs = [torch.full((n,), k + 1, dtype=torch.uint8) for k in range(6)]
    dsts = [torch.zeros(n, dtype=torch.uint8) for _ in range(6)]
    errors = []

    def run(k):
        for _ in range(5):
            rc = _copy(dsts[k], srcs[k], n, 1 + k % 5)
            if rc != 0:
                errors.append(rc)

    threads = [threading.Thread(target=run, args=(k,)) for k in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    for k in range(6):
        assert torch.equal(dsts[k], srcs[k])


@pytest.mark.skipif(not hasattr(os, "fork"), reason="needs fork")
def test_a_forked_child_copies_with_its_own_pool():
    """The parent's workers do not exist in a child; the child's copy still completes."""
    n = 6 * MIB + 1
    src = torch.arange(n, dtype=torch.int32).to(torch.uint8)
    dst = torch.zeros(n, dtype=torch.uint8)
    assert _copy(dst, src, n, 8) == 0  # the parent's pool now has workers
    dst.zero_()
    want, got = src.numpy(), dst.numpy()
    pid = os.fork()
    if pid == 0:
        # no torch op in the child: its intra-op (OpenMP) pool does not survive a fork
        ok = _copy(dst, src, n, 8) == 0 and bool((got == want).all())
        os._exit(0 if ok else 1)
    _, status = os.waitpid(pid, 0)
    assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0


def test_staging_host_copy_checks_its_tensors(monkeypatch):
    a = torch.randn(1000)
    b = torch.empty(1000)
    staging.host_copy(b, a)
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="dtype or size"):
        staging.host_copy(torch.empty(999), a)
    with pytest.raises(ValueError, match="dtype or size"):
        staging.host_copy(torch.empty(1000, dtype=torch.float64), a)
    with pytest.raises(ValueError, match="contiguous"):
        staging.host_copy(torch.empty(2000)[::2], a)
    monkeypatch.setattr(staging, "COPY_THREADS", 65)
    with pytest.raises(_lib.MorphError):
        staging.host_copy(torch.empty(4 * MIB), torch.randn(4 * MIB))


def test_default_copy_threads_leaves_cores_free(monkeypatch):
    for cores, want in ((1, 1), (4, 1), (6, 2), (12, 8), (16, 8), (64, 8)):
        monkeypatch.setattr(os, "sched_getaffinity", lambda pid, c=cores: set(range(c)))
        assert staging.default_copy_threads() == want
