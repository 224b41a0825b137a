"""A stage's canonical optimizer state resident in HBM.

The reference keeps every parameter's state on disk as one [3, N] float32 file
(rows: weight, exp_avg, exp_avg_sq; streamtrain/disk.py:45-70, 184-189).  For
each stage it reads the weight row, casts it on the CPU to the compute dtype
and copies it into the slot's device weights (disk.py:316-327), and after the
backward it updates every parameter on the CPU chunk by chunk
(DiskState.update, disk.py:203-223).

ResidentWindow moves the state of one stage onto the GPU once: load() streams
each [3, N] file through pinned staging into HBM (12 B/param host-to-device,
chunked and double-buffered) and writes the compute copy on the device
(morph_convert_f32), so the CPU cast and the separate weight copy disappear.
update() has DiskState.update's signature and arithmetic: one fused launch
over the resident state (FP32 gradient from the device window, DiskState's
constants), which also writes the new compute copy; then the [3, N] result is
written back to the file chunk by chunk with fault('partial_state_write')
after every partial write, flush and fsync -- the reference's durability and
fault order (disk.py:215-223).  If anything raises, the parameter's resident
state is dropped (it may be ahead of the file; the journal rolls the file
back) and must be loaded again.

The undo journal (disk.py:110-182) restores a stage's files when a fault hits
between its first update and its commit.  ResidentDiskUpdate.recover_stage()
keeps the window in step with that: the resident entries of the restored
files (and those dropped by a failed update) are reloaded from the restored
files, state and compute copy, as CachedDiskState drops its cache on the same
rollback (state_cache.py:147-156).
"""
import ctypes
import os
import time
import warnings

import numpy as np
import torch

from . import arena, kernels
from ._lib import check, dtype_code, lib, stream_handle
from .hyper import disk_constants
from .staging import host_copy, shared_stream, write_exact


def _fsync(path):
    fd = os.open(path, os.O_RDWR)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


class ResidentWindow:
    """One stage's [3, N] optimizer state in HBM plus its compute copy.

    store: the DiskState-like owner of the files (needs `root`, `entries`,
    `fault`).  names: the stage's canonical parameter names, in slot order.
    weights: optional flat device tensor (the slot's weights, dtype =
    compute_dtype) whose consecutive slices receive each parameter's compute
    copy, as Slot.weights does in the reference (engine.py:60-70, 128-140).
    """

    def __init__(self, store, names, compute_dtype=torch.float16, weights=None, device=None,
                 chunk_elements=1 << 22):
        self.store = store
        self.names = list(names)
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        self.compute_dtype = compute_dtype
        self.chunk = int(chunk_elements)
        if self.chunk < 1:
            raise ValueError("chunk_elements must be positive")
        sizes = [int(store.entries[n]["size"]) for n in self.names]
        total = sum(sizes)
        if weights is None:
            weights = torch.empty(total, dtype=compute_dtype, device=self.device)
        if weights.dtype != compute_dtype or weights.numel() < total or weights.device != self.device:
            raise ValueError("weights must be a device tensor of compute_dtype with room for the stage")
        self.weights, self.state, off = {}, {}, 0
        for name, n in zip(self.names, sizes):
            self.weights[name] = weights.reshape(-1)[off:off + n].view(store.entries[name]["shape"])
            off += n
        self.transfer_bytes = dict(h2d_state=0, d2h_state=0)
        self.timing = dict(file_read=0.0, d2h_wait=0.0, file_write=0.0, fsync=0.0)  # seconds
        self.kernel_timer = None  # optional list: (start, end) HIP events around each update launch
        self.dispatch_timer = None  # optional kernels.DispatchTimer: stamps each update launch
        self._copy = shared_stream(self.device, "up")  # one copy stream per device (HW queues)
        self._staging = None
        self.dropped_on_error = set()  # dropped by a failed update(); ahead of their files

    # -- staging buffers ----------------------------------------------------
    def _slots(self):
        if self._staging is None:
            c = self.chunk
            self._staging = [dict(host=torch.empty((3, c), dtype=torch.float32, pin_memory=True),
                                  event=torch.cuda.Event()) for _ in range(2)]
        return self._staging

    def _path(self, name):
        return self.store.root / self.store.entries[name]["file"]

    # -- load ---------------------------------------------------------------
    def load(self, names=None):
        """Read the [3, N] files into HBM and write the compute copies.  Synchronous on
        return for the host staging; the device work is ordered on the current stream."""
        compute = torch.cuda.current_stream(self.device)
        slots = self._slots()
        for name in (self.names if names is None else names):
            size = int(self.store.entries[name]["size"])
            dev = _state_rows(size, self.device)
            # allocated on the compute stream, which may still have work queued on this memory
            self._copy.wait_stream(compute)
            # A read-only mapping of the file; like the reference's memmap it refuses a file
            # shorter than [3, N].  The library's copy pool moves each chunk's rows into the
            # pinned buffer, its threads taking the page faults in parallel (one 226 MB file:
            # 2.9-3.4 ms against 10.4-10.8 ms by pread on one thread, on the MI355X box).
            rows = _read_only_rows(self._path(name), size)
            for k, start in enumerate(range(0, size, self.chunk)):
                end = min(start + self.chunk, size)
                n = end - start
                s = slots[k % 2]
                s["event"].synchronize()  # the H2D that last read this staging buffer is done
                t0 = time.perf_counter()
                for row in range(3):
                    host_copy(s["host"][row, :n], rows[row, start:end])
                self.timing["file_read"] += time.perf_counter() - t0
                with torch.cuda.stream(self._copy):
                    for row in range(3):
                        dev[row, start:end].copy_(s["host"][row, :n], non_blocking=True)
                    s["event"].record(self._copy)
            del rows
            compute.wait_stream(self._copy)
            self.state[name] = dev
            self.dropped_on_error.discard(name)
            self.transfer_bytes["h2d_state"] += 12 * size
            self._compute_copy(name, compute)
        for s in slots:
            s["event"].synchronize()

    def _compute_copy(self, name, stream):
        w, out = self.state[name][0], self.weights[name]
        check(lib().morph_convert_f32(ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                      dtype_code(self.compute_dtype), w.numel(), None,
                                      stream_handle(stream)))

    def drop(self, name):
        self.state.pop(name, None)

    # -- update (DiskState.update's contract) ---------------------------------
    def update(self, name, gradient, step, lr, clip, chunk_elements=1048576):
        """disk.py:203-223 on the resident state; the file is written back chunk by chunk."""
        if name not in self.state:
            raise KeyError(f"{name} is not resident; call load() first")
        if chunk_elements < 1:
            raise ValueError("chunk_elements must be positive")
        dev = self.state[name]
        size = dev.shape[1]
        flat = gradient.detach().reshape(-1)
        if flat.numel() != size:
            raise ValueError(f"gradient has {flat.numel()} elements, state has {size}")
        if flat.dtype != torch.float32:
            raise TypeError("DiskState.update takes an FP32 gradient")
        if flat.device != self.device:
            flat = flat.to(self.device)
        compute = torch.cuda.current_stream(self.device)
        try:
            if self.kernel_timer is not None:
                t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0.record(compute)
            events = self.dispatch_timer.next() if self.dispatch_timer is not None else None
            kernels.adamw_step(dev[0], dev[1], dev[2], flat, disk_constants(step=step, lr=lr, clip=clip),
                               out=self.weights[name].reshape(-1), stream=compute, events=events)
            if self.kernel_timer is not None:
                t1.record(compute)
                self.kernel_timer.append((t0, t1))
            self._write_back(name, dev, chunk_elements, compute)
        except BaseException:
            self.drop(name)
            self.dropped_on_error.add(name)
            compute.synchronize()
            raise

    def _write_back(self, name, dev, chunk_elements, compute):
        size = dev.shape[1]
        path = self._path(name)
        host = torch.empty((2, 3, min(chunk_elements, size)), dtype=torch.float32, pin_memory=True)
        hnp = host.numpy()
        done = [torch.cuda.Event(), torch.cuda.Event()]
        starts = list(range(0, size, chunk_elements))

        def fetch(k):
            start = starts[k]
            end = min(start + chunk_elements, size)
            with torch.cuda.stream(self._copy):
                if k == 0:
                    self._copy.wait_stream(compute)  # after the update
                for row in range(3):
                    host[k % 2, row, :end - start].copy_(dev[row, start:end], non_blocking=True)
                done[k % 2].record(self._copy)

        fd = os.open(path, os.O_RDWR)
        try:
            if starts:
                fetch(0)
            for k, start in enumerate(starts):
                end = min(start + chunk_elements, size)
                t0 = time.perf_counter()
                done[k % 2].synchronize()
                self.timing["d2h_wait"] += time.perf_counter() - t0
                if k + 1 < len(starts):
                    fetch(k + 1)  # overlaps this chunk's file write
                t0 = time.perf_counter()
                for row in range(3):  # the chunk's columns of all three rows, then the fault hook
                    write_exact(fd, hnp[k % 2, row, :end - start], (row * size + start) * 4)
                self.timing["file_write"] += time.perf_counter() - t0
                self.transfer_bytes["d2h_state"] += 12 * (end - start)
                self.store.fault('partial_state_write')
            t0 = time.perf_counter()
            os.fsync(fd)
            self.timing["fsync"] += time.perf_counter() - t0
        finally:
            self._copy.synchronize()
            os.close(fd)


def _read_only_rows(path, size):
    """The [3, size] float32 file at `path` as a CPU tensor over a read-only mapping (nothing
    writes through it; torch warns about any non-writable array, so that warning is muted)."""
    mapped = np.memmap(path, dtype=np.float32, mode="r", shape=(3, size))
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The given NumPy array is not writable")
        return torch.from_numpy(mapped)


def _state_rows(size, device):
    """A [3, size] float32 device view (weight, exp_avg, exp_avg_sq: the file's rows) laid
    out like a FusedAdamW arena (morph_amd.arena): when a row is 2 MiB or more, row k starts
    at a 2 MiB boundary + k * 64 KiB.  One plain [3, size] tensor puts the rows exactly
    size * 4 bytes apart -- for the config-2 matrices 36 x 2 MiB, every stream on the same
    2 MiB phase, the placement the fused pass streams slowest from."""
    nbytes = 4 * size
    if nbytes >= arena.ALIGN_LARGE:
        stride = (arena.align_up(nbytes, arena.ALIGN_LARGE) + arena.STAGGER) // 4
    else:
        stride = arena.align_up(max(nbytes, 4), arena.ALIGN_SMALL) // 4
    # room to move the first row up to the next 2 MiB boundary
    storage = torch.empty(2 * stride + size + arena.ALIGN_LARGE // 4, dtype=torch.float32,
                          device=device)
    base = ((-storage.data_ptr()) % arena.ALIGN_LARGE) // 4
    return storage.as_strided((3, size), (stride, 1), base)


class ResidentDiskUpdate:
    """DiskState mixin: update() runs on the stage window when the parameter is resident.

    class GpuDiskState(ResidentDiskUpdate, GpuDiskUpdate, DiskState): pass
    store.window = ResidentWindow(store, stage_names, torch.float16, slot.weights)
    store.window.load()          # when the stage is loaded (disk.py:316-327's place)
    ...
    store.update(name, grad, step, lr, clip)   # unchanged call sites (disk.py:464)
    """

    window = None

    def update(self, name, gradient, step, lr, clip, chunk_elements=1048576):
        if self.window is not None and name in self.window.state:
            return self.window.update(name, gradient, step, lr, clip, chunk_elements)
        return super().update(name, gradient, step, lr, clip, chunk_elements)

    def recover_stage(self):
        """disk.py:110-128, with the window kept in step with the restored files.

        A rollback (a transaction whose journal is set and present) copies the
        journaled [3, N] files back over the stage's files.  A resident entry of
        such a file may be one update ahead of it (the update succeeded, the commit
        did not happen), and the slot's compute copy with it; an entry dropped by a
        failed update left its compute copy ahead too.  Both are loaded again from
        the restored files once the host class has restored them.
        """
        window = self.window
        transaction = self.manifest.get("transaction")
        journal = self.root / "journal"
        reload = []
        if (window is not None and transaction is not None
                and transaction.get("journal") is not None and journal.exists()):
            restored = {path.name for path in journal.glob("*.bin")}
            reload = [n for n in window.names
                      if self.entries[n]["file"] in restored
                      and (n in window.state or n in window.dropped_on_error)]
            for name in reload:
                window.drop(name)
        result = super().recover_stage()
        if reload:
            window.load(reload)
        return result
