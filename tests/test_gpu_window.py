"""GPU-resident stage window (morph_amd.window) and the master-weight conversion kernel.

- load(): the compute copy equals the reference's CPU cast of the FP32 weight row
  (disk.py:316-327: read FP32, destination.copy_(work)) bit for bit;
- update(): the [3, N] file equals the oracle's DiskState arithmetic bit for bit (the
  same bar as the per-chunk path), the new compute copy equals the cast of the new
  weights, and the fault hook fires after every partial write-back in file order;
- morph_convert_f32: FP16 bits equal numpy's astype('<f2') and BF16 bits torch's
  conversion on edge cases (ties, overflow, subnormals, inf/NaN); the range flag is
  export.py:33's condition; FP32 output is a bit copy;
- rollback (disk.py:110-128): after a fault before the stage's commit or inside an
  update, recover_stage() reloads the window from the restored files, the retried
  update matches the oracle, and an export from the window equals one from the files.
"""
import ctypes
import shutil

import numpy as np
import pytest
import torch

from morph_amd import _lib
from morph_amd.window import ResidentDiskUpdate, ResidentWindow
from tests.helpers import assert_same_bits
from tests.test_gpu_disk import Store, oracle_disk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def make_store(tmp_path, sizes, seed=0, moments=True):
    rng = np.random.RandomState(seed)
    weights = {f"p{i}": (rng.randn(n) * .02).astype(np.float32) for i, n in enumerate(sizes)}
    store = Store(tmp_path, weights)
    if moments:  # non-zero moments, as after some steps
        for name, e in store.entries.items():
            s = store.state(name)
            s[1] = (rng.randn(e["size"]) * 1e-3).astype(np.float32)
            s[2] = (np.abs(rng.randn(e["size"])) * 1e-6).astype(np.float32)
            s.tofile(store.root / e["file"])
    return store


def cpu_cast(w, dtype):
    """disk.py:316-327: FP32 window then destination.copy_(work) into the compute dtype."""
    return torch.from_numpy(np.array(w, np.float32)).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_load_compute_copy_matches_cpu_cast(tmp_path, dtype):
    sizes = [1, 4099, 70000, 1048577]
    store = make_store(tmp_path, sizes)
    win = ResidentWindow(store, list(store.entries), dtype, chunk_elements=40000)
    win.load()
    torch.cuda.synchronize()
    for name in store.entries:
        st = store.state(name)
        assert_same_bits(win.state[name].cpu().numpy(), st, "resident state")
        exp = cpu_cast(st[0], dtype).view(torch.int16 if dtype != torch.float32 else torch.int32)
        got = win.weights[name].cpu().reshape(-1).view(exp.dtype)
        assert torch.equal(got, exp)
    assert win.transfer_bytes["h2d_state"] == 12 * sum(sizes)


@pytest.mark.parametrize("chunk", [1000, 1048576])
def test_update_matches_oracle_and_refreshes_compute_copy(tmp_path, chunk):
    rng = np.random.RandomState(1)
    sizes = [3001, 250000]
    store = make_store(tmp_path, sizes, moments=False)
    w0 = {n: store.state(n)[0].copy() for n in store.entries}
    slot = torch.empty(sum(sizes), dtype=torch.bfloat16, device=DEV)
    win = ResidentWindow(store, list(store.entries), torch.bfloat16, weights=slot)
    win.load()
    ups = {n: [((rng.randn(e["size"]) * 1e-2).astype(np.float32), s, .001, c)
               for s, c in ((1, .5), (2, 1.0))] for n, e in store.entries.items()}
    for k in range(2):
        for name in store.entries:
            g, step, lr, clip = ups[name][k]
            win.update(name, torch.from_numpy(g).to(DEV), step, lr, clip, chunk_elements=chunk)
    for name, e in store.entries.items():
        expect = oracle_disk(w0[name], ups[name])
        assert_same_bits(store.state(name), expect, "state file")
        assert_same_bits(win.state[name].cpu().numpy(), expect, "resident state")
        got = win.weights[name].cpu().reshape(-1).view(torch.int16)
        assert torch.equal(got, cpu_cast(expect[0], torch.bfloat16).view(torch.int16))
    n_chunks = sum(-(-n // chunk) for n in sizes)
    assert store.points == ["partial_state_write"] * (2 * n_chunks)
    # the slot buffer is the compute copies, in stage order
    assert torch.equal(slot[:sizes[0]].cpu(), win.weights["p0"].cpu())


def test_fault_after_first_partial_write_drops_resident_state(tmp_path):
    rng = np.random.RandomState(4)
    n, chunk = 10000, 4096
    store = make_store(tmp_path, [n], moments=False)
    w0 = store.state("p0")[0].copy()
    g = (rng.randn(n) * 1e-2).astype(np.float32)
    win = ResidentWindow(store, ["p0"], torch.float16)
    win.load()

    def fail(point):
        raise OSError("partial")
    store.fault = fail
    with pytest.raises(OSError, match="partial"):
        win.update("p0", torch.from_numpy(g), 1, .003, 1.0, chunk_elements=chunk)
    got = store.state("p0")
    first = oracle_disk(w0[:chunk], [(g[:chunk], 1, .003, 1.0)])
    assert_same_bits(got[:, :chunk], first, "first chunk written")
    zeros = np.zeros(n - chunk, np.float32)
    assert_same_bits(got[:, chunk:], np.stack([w0[chunk:], zeros, zeros]), "untouched tail")
    assert "p0" not in win.state
    with pytest.raises(KeyError):
        win.update("p0", torch.from_numpy(g), 1, .003, 1.0)


def test_mixin_uses_window_when_resident_else_per_chunk_path(tmp_path):
    class GpuStore(ResidentDiskUpdate, Store):  # Store already mixes in GpuDiskUpdate
        pass

    rng = np.random.RandomState(6)
    sizes = [5000, 7000]
    a = GpuStore(tmp_path / "a", {"p0": (rng.randn(sizes[0]) * .02).astype(np.float32),
                                  "p1": (rng.randn(sizes[1]) * .02).astype(np.float32)})
    b = Store(tmp_path / "b", {n: a.state(n)[0] for n in a.entries})
    a.window = ResidentWindow(a, ["p0"], torch.float16)  # only p0 resident
    a.window.load()
    for name, n in zip(("p0", "p1"), sizes):
        g = torch.from_numpy((rng.randn(n) * 1e-2).astype(np.float32))
        a.update(name, g, 1, .002, .7, chunk_elements=3000)
        b.update(name, g, 1, .002, .7, chunk_elements=3000)
        assert (a.root / a.entries[name]["file"]).read_bytes() == \
            (b.root / b.entries[name]["file"]).read_bytes()
    assert a.window.transfer_bytes["d2h_state"] == 12 * sizes[0]


def convert(x, dtype, check=False):
    src = torch.as_tensor(x, dtype=torch.float32).to(DEV)
    dst = torch.empty(src.numel(), dtype=dtype, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.check(_lib.lib().morph_convert_f32(
        ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), _lib.dtype_code(dtype),
        src.numel(), ctypes.c_void_p(flag.data_ptr()) if check else None, None))
    return dst.cpu(), bool(flag.item())


EDGE = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, -6e-8,
                 5.96e-8, 2.98e-8, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 3e38, 1e-40, np.inf,
                 -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)


def test_convert_f16_bits_equal_numpy_and_range_flag():
    rng = np.random.RandomState(2)
    x = np.concatenate([EDGE, (rng.randn(100003) * 100).astype(np.float32),
                        rng.uniform(-70000, 70000, 5000).astype(np.float32)])
    got, _ = convert(x, torch.float16)
    with np.errstate(over="ignore"):  # values past 65504 become inf, as intended
        want = x.astype("<f2")
    assert np.array_equal(got.numpy().view(np.uint16), want.view(np.uint16))
    for values, bad in (([1.0, 65504.0, -65504.0], False), ([65504.5], True), ([np.inf], True),
                        ([np.nan], True), ([1.0] * 5000 + [-70000.0], True)):
        _, flag = convert(np.array(values, np.float32), torch.float16, check=True)
        a = np.asarray(values, np.float32)
        assert flag == bad == (not np.isfinite(a).all() or np.abs(a).max() > 65504)


def test_convert_bf16_bits_equal_torch_including_nan():
    """Non-NaN values: torch's bits.  NaN: 0x7FC0, c10::BFloat16's scalar definition (torch's
    vectorized CPU path writes 0xFFFF instead, so torch itself has two NaN encodings)."""
    rng = np.random.RandomState(3)
    x = np.concatenate([EDGE, [np.nan, -np.nan], (rng.randn(50001) * 1e3).astype(np.float32)]).astype(np.float32)
    got, _ = convert(x, torch.bfloat16)
    got = got.view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    exp = torch.from_numpy(x[~nan]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[~nan], exp)
    assert (got[nan] == 0x7FC0).all()


@pytest.mark.parametrize("n,offset", [(100003, 0), (3 * 2048, 0), (5000, 1)])
def test_convert_f32_copies_bits_and_flags_nonfinite(n, offset):
    """FP32 output is a bit copy (NaN payloads, -0, subnormals kept): whole blocks, a
    partial last block, and an unaligned source (element path); the flag is set exactly
    when some value is inf or NaN."""
    rng = np.random.RandomState(4)
    x = (rng.randn(n) * 10).astype(np.float32)
    x[:len(EDGE)] = EDGE
    bits = x.view(np.uint32)
    bits[len(EDGE)] = 0x7FC01234  # a NaN with a payload
    bits[len(EDGE) + 1] = 0x00000001  # the smallest subnormal
    base = torch.zeros(n + offset, dtype=torch.float32, device=DEV)
    base[offset:] = torch.from_numpy(x).to(DEV)
    src = base[offset:]
    for check in (False, True):
        dst = torch.empty(n, dtype=torch.float32, device=DEV)
        flag = torch.zeros(1, dtype=torch.int32, device=DEV)
        _lib.check(_lib.lib().morph_convert_f32(
            ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), _lib.DTYPE_F32, n,
            ctypes.c_void_p(flag.data_ptr()) if check else None, None))
        assert np.array_equal(dst.cpu().numpy().view(np.uint32), bits)
        assert bool(flag.item()) == check
    finite = torch.from_numpy(np.where(np.isfinite(x), x, 0).astype(np.float32)).to(DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty_like(finite)
    _lib.check(_lib.lib().morph_convert_f32(
        ctypes.c_void_p(finite.data_ptr()), ctypes.c_void_p(out.data_ptr()), _lib.DTYPE_F32, n,
        ctypes.c_void_p(flag.data_ptr()), None))
    assert torch.equal(out, finite) and not bool(flag.item())


class JournalBase(Store):
    """Store plus a minimal undo journal with the behaviour streamtrain/disk.py:110-174
    gives recover_stage: prepare_stage copies the stage's files into root/journal and
    records the stage in the transaction; commit_stage clears both; recover_stage copies
    the journaled files back when the transaction still names a journal."""

    def __init__(self, root, weights=None, entries=None):
        if entries is None:
            super().__init__(root, weights)
        else:
            self.root, self.entries, self.points = root, entries, []
        self.manifest = dict(transaction=None)
        self.fail_at = None

    def fault(self, point):
        self.points.append(point)
        if point == self.fail_at:
            raise RuntimeError(f"injected fault at {point}")

    def begin(self):
        self.manifest["transaction"] = dict(journal=None)

    def prepare_stage(self, index, names):
        journal = self.root / "journal"
        shutil.rmtree(journal, ignore_errors=True)
        journal.mkdir()
        for name in names:
            f = self.entries[name]["file"]
            shutil.copyfile(self.root / f, journal / f)
        self.fault("journal_durable")
        self.manifest["transaction"]["journal"] = index

    def commit_stage(self, index):
        self.fault("cursor_file_durable")
        self.manifest["transaction"]["journal"] = None
        shutil.rmtree(self.root / "journal", ignore_errors=True)

    def recover_stage(self):
        transaction = self.manifest.get("transaction")
        journal = self.root / "journal"
        if transaction and transaction.get("journal") is not None:
            for path in journal.glob("*.bin"):
                shutil.copyfile(path, self.root / path.name)
            transaction["journal"] = None
        shutil.rmtree(journal, ignore_errors=True)


class ResidentJournalStore(ResidentDiskUpdate, JournalBase):
    pass


def _grads(store, seed):
    rng = np.random.RandomState(seed)
    return {n: torch.from_numpy((rng.randn(e["size"]) * 1e-2).astype(np.float32)).to(DEV)
            for n, e in store.entries.items()}


@pytest.mark.parametrize("fail_at", ["cursor_file_durable", "partial_state_write"])
def test_rollback_reloads_the_window_from_the_restored_files(tmp_path, fail_at):
    """disk.py:110-128 / state_cache.py:147-156: a fault after the stage's updates
    (before its commit) or inside one (after a partial write-back) leaves the window --
    state and compute copy -- ahead of the files the journal restores.  recover_stage()
    on the same store reloads it; the retried update then equals the oracle applied to
    the restored file, and the compute copy equals the cast of the final weights."""
    sizes = [3001, 250000]
    store = ResidentJournalStore(tmp_path, {f"p{i}": (np.random.RandomState(i).randn(n) * .02)
                                            for i, n in enumerate(sizes)})
    names = list(store.entries)
    before = {n: store.state(n).copy() for n in names}
    slot = torch.empty(sum(sizes), dtype=torch.bfloat16, device=DEV)
    store.window = ResidentWindow(store, names, torch.bfloat16, weights=slot)
    store.window.load()
    store.begin()
    store.prepare_stage(0, names)
    store.fail_at = fail_at
    first = _grads(store, 5)
    with pytest.raises(RuntimeError, match="injected fault"):
        for name in names:
            store.update(name, first[name], 1, .002, .5, chunk_elements=100000)
        store.commit_stage(0)
    store.fail_at = None
    store.recover_stage()
    torch.cuda.synchronize()
    for name in names:
        assert_same_bits(store.state(name), before[name], "restored file")
        assert name in store.window.state
        assert_same_bits(store.window.state[name].cpu().numpy(), before[name], "reloaded state")
        got = store.window.weights[name].cpu().reshape(-1).view(torch.int16)
        assert torch.equal(got, cpu_cast(before[name][0], torch.bfloat16).view(torch.int16))
    # the retried stage
    store.begin()
    store.prepare_stage(0, names)
    retry = _grads(store, 6)
    for name in names:
        store.update(name, retry[name], 1, .002, .5, chunk_elements=100000)
    store.commit_stage(0)
    torch.cuda.synchronize()
    for name in names:
        expect = oracle_disk(before[name][0], [(retry[name].cpu().numpy(), 1, .002, .5)])
        assert_same_bits(store.state(name), expect, "file after the retried update")
        assert_same_bits(store.window.state[name].cpu().numpy(), expect, "resident state")
        got = store.window.weights[name].cpu().reshape(-1).view(torch.int16)
        assert torch.equal(got, cpu_cast(expect[0], torch.bfloat16).view(torch.int16))


def test_export_from_the_window_after_rollback_equals_the_files(tmp_path):
    """export_fp16(window=...) encodes the resident rows; after a rollback they must be the
    restored (committed) weights, so the shards equal an export from the files."""
    from morph_amd.export import export_fp16
    from tests.test_gpu_export import Tiny, make_state, same_dirs
    model = Tiny()
    state_dir = tmp_path / "state"
    entries = make_state(state_dir, model)
    store = ResidentJournalStore(state_dir, entries=entries)
    names = list(entries)
    store.window = ResidentWindow(store, names, torch.float16)
    store.window.load()
    store.begin()
    store.prepare_stage(0, names)
    store.fail_at = "cursor_file_durable"
    grads = _grads(store, 7)
    with pytest.raises(RuntimeError, match="injected fault"):
        for name in names:
            store.update(name, grads[name] * 100, 1, .5, 1.0)
        store.commit_stage(0)
    store.fail_at = None
    store.recover_stage()
    export_fp16(state_dir, tmp_path / "from_window", model=model, window=store.window,
                lock_held=True)
    export_fp16(state_dir, tmp_path / "from_files", model=model, lock_held=True)
    same_dirs(tmp_path / "from_window", tmp_path / "from_files")
