"""GPU AdamW behind DiskState.update's signature (streamtrain/disk.py:203-223).

The reference keeps each parameter's canonical state on disk as one [3, N]
float32 file (rows: weight, first moment, second moment) and updates it on
the CPU chunk by chunk.  This module keeps that contract -- same signature,
same file format, the chunk loop, fault('partial_state_write') after every
partial write-back (disk.py:216), flush + fsync at the end -- and moves the
arithmetic to the fused kernel with DiskState's constants (betas 0.9/0.999,
eps 1e-8, weight decay 0.01 on every parameter, gradient * clip).

Per chunk the [3, n] slice is staged through pinned host memory to the GPU,
updated in place by one launch, and copied back; this path is PCIe-bound
(16 B/param H2D, 12 B/param D2H), so it pipelines the transfers of chunk k+1
with the update of chunk k on separate streams while keeping the write-back
and fault order of the reference.

Use:  class GpuDiskState(GpuDiskUpdate, DiskState): pass
or    gpu_disk_update(mapped, gradient, step, lr, clip, chunk_elements, fault)
"""
import os

import numpy as np
import torch

from . import kernels
from .hyper import disk_constants
from .staging import host_copy, shared_stream


class _Staging:
    """Pinned host + device buffers for one chunk in flight."""

    def __init__(self, chunk, device):
        self.host_state = torch.empty((3, chunk), dtype=torch.float32, pin_memory=True)
        self.host_grad = torch.empty(chunk, dtype=torch.float32, pin_memory=True)
        self.dev_state = torch.empty((3, chunk), dtype=torch.float32, device=device)
        self.dev_grad = torch.empty(chunk, dtype=torch.float32, device=device)
        self.ready = torch.cuda.Event()
        self.done = torch.cuda.Event()


def _rows(a):
    """torch views sharing the memory of a writable C-ordered ndarray (an np.memmap of a state
    file, or a cached copy), else None."""
    if isinstance(a, np.ndarray) and a.flags.c_contiguous and a.flags.writeable:
        return torch.from_numpy(a)
    return None


def gpu_disk_update(mapped, gradient, step, lr, clip, chunk_elements=1048576, fault=None,
                    device=None, dispatch_timer=None, write_through=None):
    """Update a [3, N] float32 array-like (e.g. np.memmap) in place, chunk by chunk.

    gradient: FP32 tensor with N elements (CPU, pinned or on the GPU), already
    unscaled (disk.py:447).  Writes back each chunk before calling fault().
    dispatch_timer: optional kernels.DispatchTimer; each chunk's launch stamps a pair.
    write_through: optional second [3, N] float32 array-like that every chunk's result is
    also written to, after `mapped` (CachedDiskState's cache and its file).
    """
    if mapped.shape[0] != 3 or mapped.dtype != np.float32:
        raise ValueError("state must be a [3, N] float32 array")
    if write_through is not None and (tuple(write_through.shape) != tuple(mapped.shape)
                                      or write_through.dtype != np.float32):
        raise ValueError("write_through must be a [3, N] float32 array like the state")
    size = mapped.shape[1]
    flat = gradient.detach().reshape(-1)
    if flat.numel() != size:
        raise ValueError(f"gradient has {flat.numel()} elements, state has {size}")
    if flat.dtype != torch.float32:
        raise TypeError("DiskState.update takes an FP32 gradient")
    if chunk_elements < 1:
        raise ValueError("chunk_elements must be positive")
    device = torch.device(device) if device is not None else torch.device(
        "cuda", torch.cuda.current_device())
    # A writable C-ordered ndarray (the np.memmap of DiskState) is read and written row by row
    # on the library's copy pool, whose threads take the file's page faults in parallel; any
    # other array-like goes through its own indexing.
    targets = [mapped] if write_through is None else [mapped, write_through]
    views = [_rows(t) for t in targets]
    rows = views[0]
    hp = disk_constants(step=step, lr=lr, clip=clip)
    chunk = min(chunk_elements, max(size, 1))
    compute = torch.cuda.current_stream(device)
    copy_in = shared_stream(device, "up")  # one copy stream per device (HW queues)
    slots = [_Staging(chunk, device) for _ in range(2)]
    # The staging tensors come from the caching allocator on the compute stream, which may hand
    # out memory whose last reader is still queued there, and a device gradient may still be in
    # production on it: the copy stream starts after everything queued so far.
    copy_in.wait_stream(compute)
    starts = list(range(0, size, chunk_elements))

    def stage_in(k):
        s = slots[k % 2]
        start = starts[k]
        end = min(start + chunk_elements, size)
        n = end - start
        s.done.synchronize()  # the previous user of this slot has been written back
        if rows is not None:
            for r in range(3):
                host_copy(s.host_state[r, :n], rows[r, start:end])
        else:
            s.host_state[:, :n].copy_(torch.from_numpy(np.ascontiguousarray(mapped[:, start:end])))
        with torch.cuda.stream(copy_in):
            s.dev_state[:, :n].copy_(s.host_state[:, :n], non_blocking=True)
            if flat.device.type == "cuda":
                s.dev_grad[:n].copy_(flat[start:end], non_blocking=True)
            else:
                host_copy(s.host_grad[:n], flat[start:end])
                s.dev_grad[:n].copy_(s.host_grad[:n], non_blocking=True)
            s.ready.record(copy_in)
        return s, start, end, n

    try:
        pending = stage_in(0) if starts else None
        for k in range(len(starts)):
            s, start, end, n = pending
            compute.wait_event(s.ready)
            w, m, v = s.dev_state[0, :n], s.dev_state[1, :n], s.dev_state[2, :n]
            kernels.adamw_step(w, m, v, s.dev_grad[:n], hp, stream=compute,
                               events=dispatch_timer.next() if dispatch_timer is not None else None)
            s.host_state[:, :n].copy_(s.dev_state[:, :n], non_blocking=True)
            s.done.record(compute)
            if k + 1 < len(starts):
                pending = stage_in(k + 1)  # overlaps the update and copy-back of chunk k
            s.done.synchronize()
            for target, view in zip(targets, views):
                if view is not None:
                    for r in range(3):
                        host_copy(view[r, start:end], s.host_state[r, :n])
                else:
                    target[:, start:end] = s.host_state[:, :n].numpy()
            if fault is not None:
                fault('partial_state_write')
    finally:
        # an exception (e.g. an injected fault) may leave a staged copy in flight
        copy_in.synchronize()
        compute.synchronize()


class GpuDiskUpdate:
    """Mixin replacing DiskState.update (and CachedDiskState.update) with the GPU pass.

    Needs the host class's `root`, `entries` and `fault` (streamtrain/disk.py:45-108).
    When the host class keeps the CachedDiskState cache (state_cache.py:103-140),
    a cached [3, N] array is updated in the same pass and written through.
    """

    update_device = None  # None: the current CUDA device
    dispatch_timer = None  # optional kernels.DispatchTimer: stamps each chunk's launch

    def update(self, name, gradient, step, lr, clip, chunk_elements=1048576):
        if getattr(self, "_cache", None) is not None and hasattr(self, "_cache_lock"):
            return self._update_cached(name, gradient, step, lr, clip, chunk_elements)
        return self._update_plain(name, gradient, step, lr, clip, chunk_elements)

    def _update_plain(self, name, gradient, step, lr, clip, chunk_elements):
        entry = self.entries[name]
        path = self.root / entry['file']
        mapped = np.memmap(path, dtype='float32', mode='r+', shape=(3, entry['size']))
        gpu_disk_update(mapped, gradient, step, lr, clip, chunk_elements, self.fault,
                        self.update_device, self.dispatch_timer)
        mapped.flush()
        del mapped
        _fsync(path)

    def _update_cached(self, name, gradient, step, lr, clip, chunk_elements):
        # Bookkeeping of CachedDiskState.update (state_cache.py:103-140) around the GPU pass.
        with self._cache_lock:
            values = self._cache.get(name)
            if values is None:
                # dormant moments are not fetched just to populate the cache
                self._cache_stats["misses"] += 1
                return self._update_plain(name, gradient, step, lr, clip, chunk_elements)
            self._cache.move_to_end(name)
            self._cache_stats["hits"] += 1
            self._cache_stats["estimated_bytes_avoided"] += values.nbytes
            entry = self.entries[name]
            path = self.root / entry["file"]
            try:
                mapped = np.memmap(path, dtype=np.float32, mode="r+", shape=(3, entry["size"]))
                # the cached values are read, and each chunk's result goes to them, then the file
                gpu_disk_update(values, gradient, step, lr, clip, chunk_elements, self.fault,
                                self.update_device, self.dispatch_timer, write_through=mapped)
                mapped.flush()
                del mapped
                _fsync(path)
            except BaseException:
                self._drop(name)
                raise


def _fsync(path):
    descriptor = os.open(path, os.O_RDWR)
    try:
        os.fsync(descriptor)
    finally:
        os.close(descriptor)
