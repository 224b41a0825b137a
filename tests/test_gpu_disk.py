"""GPU DiskState.update drop-in (morph_amd.disk) vs the oracle, on real [3, N] files."""
import json
import threading
from collections import OrderedDict
from pathlib import Path

import numpy as np
import pytest
import torch

from morph_amd.disk import GpuDiskUpdate, gpu_disk_update
from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu


class Store(GpuDiskUpdate):
    """The attributes of streamtrain/disk.py:45-108 that update() uses."""

    def __init__(self, root, weights):
        self.root = Path(root)
        self.root.mkdir(parents=True, exist_ok=True)
        self.entries = {}
        for i, (name, w) in enumerate(weights.items()):
            w = np.asarray(w, np.float32).ravel()
            self.entries[name] = dict(shape=[w.size], size=w.size, file=f"{i:05}.bin")
            np.stack([w, np.zeros_like(w), np.zeros_like(w)]).tofile(self.root / f"{i:05}.bin")
        self.points = []

    def fault(self, point):
        self.points.append(point)

    def state(self, name):
        e = self.entries[name]
        return np.fromfile(self.root / e["file"], dtype=np.float32).reshape(3, e["size"])


class CachedStore(Store):
    """Plus the cache attributes of streamtrain/state_cache.py that update() uses."""

    def __init__(self, root, weights):
        super().__init__(root, weights)
        self._cache_lock = threading.RLock()
        self._cache = OrderedDict()
        self._cache_stats = dict(hits=0, misses=0, estimated_bytes_avoided=0)
        self.dropped = []

    def warm(self, name):
        self._cache[name] = self.state(name).copy()

    def _drop(self, name):
        self.dropped.append(name)
        self._cache.pop(name, None)


def oracle_disk(w0, updates):
    """C oracle with DiskState constants, applied to the whole vector."""
    from oracle import reference as R
    w, m, v = np.array(w0, np.float32), np.zeros(len(w0), np.float32), np.zeros(len(w0), np.float32)
    for grad, step, lr, clip in updates:
        R.adamw(np.asarray(grad, np.float32), w, m, v, R.disk_adamw_hp(step, lr, clip))
    return np.stack([w, m, v])


def test_state_cache_vectors_bitexact(tmp_path):
    """tests/test_state_cache.py:21-46's vectors, chunk 2, through the GPU update."""
    store = Store(tmp_path, {"weight": [1.0, -2.0, 0.5]})
    ups = [([2.0, -1.0, 0.5], 1, .003, .25), ([-.3, 1.2, 5.0], 3, .003, .1)]
    for grad, step, lr, clip in ups:
        store.update("weight", torch.tensor(grad), step, lr, clip, chunk_elements=2)
    assert_same_bits(store.state("weight"), oracle_disk([1.0, -2.0, 0.5], ups), "state file")
    assert store.points == ["partial_state_write"] * 4  # 2 chunks x 2 updates


@pytest.mark.parametrize("n,chunk", [(1, 1048576), (3001, 1000), (1048577, 1048576), (250000, 65536)])
def test_random_parameters_bitexact_and_torch_close(tmp_path, n, chunk):
    from oracle import reference as R
    rng = np.random.RandomState(n)
    w0 = (rng.randn(n) * .02).astype(np.float32)
    store = Store(tmp_path, {"p": w0})
    ups = [((rng.randn(n) * 1e-2).astype(np.float32), s, .001, c) for s, c in ((1, .5), (2, 1.0), (7, .03))]
    for g, step, lr, clip in ups:
        store.update("p", torch.from_numpy(g), step, lr, clip, chunk_elements=chunk)
    got = store.state("p")
    assert_same_bits(got, oracle_disk(w0, ups), "state file")
    # the reference's own torch-op sequence (disk.py:209-215): moments exact, masters close
    ref = np.stack([w0, np.zeros(n, np.float32), np.zeros(n, np.float32)])
    for g, step, lr, clip in ups:
        R.disk_update_torch(ref, torch.from_numpy(g), step, lr, clip, chunk_elements=chunk)
    assert_same_bits(got[1:], ref[1:], "moments vs torch ops")
    assert np.abs(got[0] - ref[0]).max() <= 1e-6 * np.abs(ref[0]).max()


class _Indexed:
    """A [3, N] array-like with only shape, dtype and indexing (not an ndarray)."""

    def __init__(self, a):
        self.a, self.shape, self.dtype = a, a.shape, a.dtype

    def __getitem__(self, key):
        return self.a[key]

    def __setitem__(self, key, value):
        self.a[key] = value


def test_states_the_copy_pool_cannot_take_go_through_indexing():
    """A writable C-ordered ndarray is read and written on the copy pool; any other [3, N]
    array-like (Fortran order, an object with indexing only) takes the indexing path, and a
    write-through target gets every chunk's result too.  All end bit-exact vs the oracle."""
    rng = np.random.RandomState(8)
    n, chunk = 5003, 1000
    w0 = (rng.randn(n) * .02).astype(np.float32)
    ups = [((rng.randn(n) * 1e-2).astype(np.float32), s, .001, .6) for s in (1, 2)]
    want = oracle_disk(w0, ups)

    def fresh():
        return np.stack([w0, np.zeros(n, np.float32), np.zeros(n, np.float32)])

    fortran = np.asfortranarray(fresh())
    indexed = _Indexed(fresh())
    cache, mirror = fresh(), _Indexed(fresh())
    for g, step, lr, clip in ups:
        gpu_disk_update(fortran, torch.from_numpy(g), step, lr, clip, chunk)
        gpu_disk_update(indexed, torch.from_numpy(g), step, lr, clip, chunk)
        gpu_disk_update(cache, torch.from_numpy(g), step, lr, clip, chunk, write_through=mirror)
    assert not fortran.flags.c_contiguous
    assert_same_bits(np.ascontiguousarray(fortran), want, "Fortran-ordered state")
    assert_same_bits(indexed.a, want, "indexed state")
    assert_same_bits(cache, want, "state with a write-through target")
    assert_same_bits(mirror.a, want, "write-through target")
    with pytest.raises(ValueError, match="write_through"):
        gpu_disk_update(fresh(), torch.from_numpy(ups[0][0]), 1, .001, .6, chunk,
                        write_through=np.zeros((3, n + 1), np.float32))


def test_updates_from_two_threads_at_once(tmp_path):
    """disk.py:287-300: the main thread calls update() while SlotPrefetch's worker works on
    other parameters.  Two threads updating their own stores at the same time (each
    chunk's launches and copies ordered on the calling thread's stream) both end
    bit-exact against the oracle."""
    rng = np.random.RandomState(21)
    n = 300001
    w0 = {k: (rng.randn(n) * .02).astype(np.float32) for k in ("a", "b")}
    ups = {k: [((rng.randn(n) * 1e-2).astype(np.float32), s, .001, .7) for s in (1, 2, 3)]
           for k in ("a", "b")}
    stores = {k: Store(tmp_path / k, {"p": w0[k]}) for k in ("a", "b")}
    errors = []

    def run(k):
        try:
            side = torch.cuda.Stream() if k == "b" else None  # one thread on its own stream
            with torch.cuda.stream(side) if side is not None else torch.cuda.stream(
                    torch.cuda.current_stream()):
                for g, step, lr, clip in ups[k]:
                    stores[k].update("p", torch.from_numpy(g), step, lr, clip, chunk_elements=65536)
        except Exception as e:  # surfaced on the main thread below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(k,)) for k in ("a", "b")]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for k in ("a", "b"):
        assert_same_bits(stores[k].state("p"), oracle_disk(w0[k], ups[k]), f"store {k}")


def test_device_gradient_input(tmp_path):
    rng = np.random.RandomState(3)
    w0 = (rng.randn(70000) * .02).astype(np.float32)
    g = (rng.randn(70000) * 1e-2).astype(np.float32)
    store = Store(tmp_path, {"p": w0})
    store.update("p", torch.from_numpy(g).cuda(), 1, .002, .8, chunk_elements=30000)
    assert_same_bits(store.state("p"), oracle_disk(w0, [(g, 1, .002, .8)]), "state file")


def test_fault_after_first_partial_write_leaves_later_chunks_untouched(tmp_path):
    """disk.py:216: the fault hook fires after each partial write-back."""
    rng = np.random.RandomState(4)
    n, chunk = 10000, 4096
    w0 = (rng.randn(n) * .02).astype(np.float32)
    g = (rng.randn(n) * 1e-2).astype(np.float32)
    store = Store(tmp_path, {"p": w0})

    def fail(point):
        raise OSError("partial")
    store.fault = fail
    with pytest.raises(OSError, match="partial"):
        store.update("p", torch.from_numpy(g), 1, .003, 1.0, chunk_elements=chunk)
    got = store.state("p")
    first = oracle_disk(w0[:chunk], [(g[:chunk], 1, .003, 1.0)])
    assert_same_bits(got[:, :chunk], first, "first chunk written")
    assert_same_bits(got[:, chunk:], np.stack([w0[chunk:], np.zeros(n - chunk, np.float32),
                                               np.zeros(n - chunk, np.float32)]), "untouched tail")


def test_cached_store_hit_writes_through_and_matches_plain(tmp_path):
    rng = np.random.RandomState(5)
    w0 = (rng.randn(5000) * .02).astype(np.float32)
    g = (rng.randn(5000) * 1e-2).astype(np.float32)
    plain = Store(tmp_path / "plain", {"p": w0})
    cached = CachedStore(tmp_path / "cached", {"p": w0})
    cached.warm("p")
    for s in (plain, cached):
        s.update("p", torch.from_numpy(g), 1, .003, .5, chunk_elements=2048)
    assert cached._cache_stats["hits"] == 1
    assert (plain.root / "00000.bin").read_bytes() == (cached.root / "00000.bin").read_bytes()
    assert_same_bits(cached._cache["p"], cached.state("p"), "cache == file")
    # a miss goes to the file path and does not populate the cache
    cached2 = CachedStore(tmp_path / "cached2", {"p": w0})
    cached2.update("p", torch.from_numpy(g), 1, .003, .5)
    assert cached2._cache_stats["misses"] == 1 and "p" not in cached2._cache


def test_cached_store_failed_write_drops_entry(tmp_path):
    """state_cache.py:138-140: an exception mid-update invalidates the cached entry."""
    w0 = np.arange(6000, dtype=np.float32) * 1e-3
    cached = CachedStore(tmp_path, {"p": w0})
    cached.warm("p")
    cached.fault = lambda point: (_ for _ in ()).throw(OSError("partial"))
    with pytest.raises(OSError):
        cached.update("p", torch.ones(6000), 1, .003, 1.0, chunk_elements=1000)
    assert cached.dropped == ["p"] and "p" not in cached._cache


def test_rejects_wrong_shapes(tmp_path):
    store = Store(tmp_path, {"p": np.zeros(10, np.float32)})
    with pytest.raises(ValueError):
        store.update("p", torch.ones(11), 1, .001, 1.0)
    with pytest.raises(TypeError):
        store.update("p", torch.ones(10, dtype=torch.float16), 1, .001, 1.0)
