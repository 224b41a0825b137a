"""Device mirrors of host tensors and the pinned transfers that fill and drain them.

The reference's streamed engines keep the FP32 masters on the CPU
(morph/training/runner.py:41, StreamTrainEngine requires it, engine.py:92-93)
and leave each step's gradients in CPU `p.grad` (Slot.flush, engine.py:75-88);
HybridMuonAdamW / torch.optim.AdamW then update those CPU tensors in place.
Here the optimizer state stays resident in HBM and only the masters and the
gradients cross PCIe: HostStaging keeps one flat device buffer holding a
mirror of each host tensor (each at a 256-byte aligned offset) and moves data
between the host tensors and the mirrors in chunks through two pinned buffers
per direction, so the host-side copy of one chunk (pageable <-> pinned, on the
library's copy pool: host_copy) overlaps the DMA of the other.  Tensors whose mirrors are
adjacent travel in one DMA per chunk.  A host tensor that is already in
page-locked memory (pin_host_tensors, or a caller's own pinned allocation) is
reached by the DMA directly: its chunks skip the pinned buffers and the host
copy, which bounds the pageable transfers.  pipeline() streams chunks through a
device pass: chunk k goes up while chunk k - 1 comes back, on one copy stream
per direction (PCIe carries both directions at once: 88 GB/s together against
56 GB/s either way alone, measured on MI355X).
"""
import collections
import ctypes
import os
import threading

import torch

from ._lib import check, lib

ALIGN = 64  # elements of 4 bytes: mirrors start 256-byte aligned

_STREAMS = {}
_STREAMS_LOCK = threading.Lock()


def shared_stream(device, role):
    """The stream of `role` ('up', 'down', or 'side' for device work beside the
    caller's stream) on `device`, one per device for every user in the process.

    HIP multiplexes streams onto a few hardware queues (GPU_MAX_HW_QUEUES, 4 by
    default).  With a copy stream per staging object and direction, plus a side
    stream, streams end up sharing a queue, and work on one then waits for
    unrelated work on the other: measured on the streamed Muon step, the AdamW
    group's 4 MB gradient upload waited 21 ms for the Newton-Schulz chain running on
    the side stream.  The caller's stream and these three fit the four queues."""
    device = torch.device(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), role)
    with _STREAMS_LOCK:
        stream = _STREAMS.get(key)
        if stream is None:
            stream = _STREAMS[key] = torch.cuda.Stream(torch.device("cuda", key[0]))
    return stream


def read_exact(fd, out, offset):
    """Fill the contiguous array `out` (e.g. a view of pinned staging) from the file `fd` at
    byte `offset`, by pread; a file that ends first raises OSError."""
    view = memoryview(out).cast("B")
    got = 0
    while got < len(view):
        n = os.preadv(fd, [view[got:]], offset + got)
        if n <= 0:
            raise OSError(f"short read of a state file at offset {offset + got}")
        got += n


def write_exact(fd, data, offset):
    """Write all of the contiguous array `data` to the file `fd` at byte `offset`, by pwrite."""
    view = memoryview(data).cast("B")
    put = 0
    while put < len(view):
        put += os.pwrite(fd, view[put:], offset + put)


COPY_THREADS = None  # host_copy's thread count; None: default_copy_threads()


def default_copy_threads():
    """Threads for the host side of the staging copies: the cores this process may run
    on less four (left to the HIP runtime and the thread that queues the DMAs), at most 8,
    at least 1.  Measured on the MI355X box's 16 cores, streamed steps with CPU masters
    and gradients: config 2 11.0-11.8 ms per step with 8 threads against 12.4-13.4 with
    4, 11.9-12.2 with 12 and 12.0-12.6 with 16; config 5 139-140 ms with 8, 140-147
    with 6, 142-143 with 12."""
    return max(1, min(8, len(os.sched_getaffinity(0)) - 4))


_SMALL_COPY_BYTES = 64 << 10  # under this, torch's copy_ stays below its parallel grain (inline)
_default_threads = None


def _copy_threads():
    global _default_threads
    if COPY_THREADS is not None:
        return int(COPY_THREADS)
    if _default_threads is None:
        _default_threads = default_copy_threads()
    return _default_threads


def host_copy(dst, src):
    """dst <- src for two contiguous CPU tensors of one dtype and size: on the library's
    copy pool (morph_host_copy, COPY_THREADS threads), or inline on the calling thread
    for a copy under 64 KiB, where a pool call costs more than the copy."""
    if dst.dtype != src.dtype or dst.numel() != src.numel():
        raise ValueError("host_copy: dtype or size differs")
    if dst.device.type != "cpu" or src.device.type != "cpu":
        raise ValueError("host_copy: tensors must be on the CPU")
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("host_copy: tensors must be contiguous")
    _copy(dst, src)


def _copy(dst, src):
    """host_copy without its checks, for tensors the staging has validated already."""
    nbytes = dst.numel() * dst.element_size()
    if nbytes < _SMALL_COPY_BYTES:
        dst.copy_(src)
        return
    check(lib().morph_host_copy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                                nbytes, _copy_threads()))


def _align(x):
    return (x + ALIGN - 1) // ALIGN * ALIGN


def pin_host_tensors(tensors):
    """Move the data of CPU tensors (e.g. a streamed model's FP32 master parameters) into
    page-locked host memory in place: t.data becomes a pinned copy, so every reference
    to the tensor (a module's Parameter, an optimizer's parameter list) sees it.  The
    staging of the optimizers then moves these tensors by DMA alone.  Tensors already
    pinned are left alone.  Two distinct tensors that share storage cannot both be moved
    without losing the sharing, so that raises ValueError before anything is moved.
    Returns the number of bytes moved."""
    tensors = [t for t in tensors if t.device.type == "cpu"]
    owners = {}
    for t in tensors:
        key = t.untyped_storage().data_ptr()
        if key in owners and owners[key] is not t:
            raise ValueError("two tensors share host storage; pin the storage's owner instead")
        owners[key] = t
    moved = 0
    for t in owners.values():
        if t.is_pinned():
            continue
        t.data = t.data.pin_memory()
        moved += t.numel() * t.element_size()
    return moved


class HostStaging:
    """Device mirrors of `count` host tensors of the given shapes and one dtype.

    views[i] is the device mirror of tensor i.  upload()/download() move the
    listed tensors; both are ordered after the work already queued on
    `stream` and return with the host side finished (download: the host
    tensors hold the data; upload: the pinned buffers are free again), the
    device side ordered before later work on `stream`.
    """

    _DOWN_BUFFERS = 3  # pipeline(): pinned buffers (downloads in flight) on the way back

    def __init__(self, shapes, dtype, device, chunk_elements=1 << 22):
        self.device = torch.device(device)
        self.dtype = dtype
        self.shapes = [tuple(s) for s in shapes]
        self.numels = [int(torch.Size(s).numel()) for s in self.shapes]
        self.offsets, off = [], 0
        for n in self.numels:
            self.offsets.append(off)
            off = _align(off + n)
        self.flat = torch.empty(max(off, 1), dtype=dtype, device=self.device)
        self.views = [self.flat[o:o + n].view(s)
                      for o, n, s in zip(self.offsets, self.numels, self.shapes)]
        self.chunk = max(int(chunk_elements), ALIGN)
        self._copy = shared_stream(self.device, "up")
        self._copy_down = None
        self._pinned = None
        self._pinned_down = None
        self.bytes_h2d = 0
        self.bytes_d2h = 0

    def _new_buffers(self, count=2):
        return [dict(buf=torch.empty(self.chunk, dtype=self.dtype, pin_memory=True),
                     event=torch.cuda.Event()) for _ in range(count)]

    def _buffers(self):
        if self._pinned is None:
            self._pinned = self._new_buffers()
        return self._pinned

    def _chunks(self, which):
        """Device ranges [lo, hi) of at most `chunk` elements, each with the pieces
        (index, tensor start, tensor end) of the listed tensors it holds.  A range only
        spans tensors that are all listed (padding between them rides along)."""
        chunks = []
        which = sorted(set(which))
        run = []
        for k, i in enumerate(which):
            if run and i != run[-1] + 1:
                chunks += self._split(run)
                run = []
            run.append(i)
        if run:
            chunks += self._split(run)
        return chunks

    def _split(self, run):
        lo = self.offsets[run[0]]
        hi = self.offsets[run[-1]] + self.numels[run[-1]]
        out = []
        for a in range(lo, hi, self.chunk):
            b = min(a + self.chunk, hi)
            pieces = []
            for i in run:
                s = max(a, self.offsets[i])
                e = min(b, self.offsets[i] + self.numels[i])
                if s < e:
                    pieces.append((i, s - self.offsets[i], e - self.offsets[i]))
            out.append((a, b, pieces))
        return out

    def _check(self, tensors, which):
        for i, t in zip(which, tensors):
            if t.device.type != "cpu" or t.dtype != self.dtype or t.numel() != self.numels[i]:
                raise ValueError(f"host tensor {i}: expected a CPU {self.dtype} tensor of "
                                 f"{self.numels[i]} elements")
            if not t.is_contiguous():
                raise ValueError(f"host tensor {i} must be contiguous")

    @staticmethod
    def _pinned_of(host):
        """Indices of the host tensors in page-locked memory (DMA reaches them directly)."""
        return {i for i, t in host.items() if t.is_pinned()}

    @staticmethod
    def _direct(pieces, pinned):
        return all(i in pinned for i, _, _ in pieces)

    def _up_direct(self, pieces, host):
        """DMA of each piece from its pinned host tensor (on the current stream)."""
        for i, s, e in pieces:
            at = self.offsets[i] + s
            self.flat[at:at + e - s].copy_(host[i][s:e], non_blocking=True)
            self.bytes_h2d += (e - s) * self.flat.element_size()

    def _down_direct(self, pieces, host):
        """DMA of each piece into its pinned host tensor (on the current stream)."""
        for i, s, e in pieces:
            at = self.offsets[i] + s
            host[i][s:e].copy_(self.flat[at:at + e - s], non_blocking=True)
            self.bytes_d2h += (e - s) * self.flat.element_size()

    def upload(self, tensors, which=None, stream=None, wait=True, current=()):
        """views[which[k]] <- tensors[k] (host, contiguous).

        wait=False: the copies do not wait for the work already queued on
        `stream`; only for a caller that knows no queued work reads or writes
        these mirrors (later work on `stream` still waits for the copies).
        current: indices whose mirrors already hold their host tensors' values;
        a chunk made of such tensors only is not copied."""
        which = list(range(len(self.numels))) if which is None else list(which)
        tensors = list(tensors)
        self._check(tensors, which)
        src = {i: t.detach().reshape(-1) for i, t in zip(which, tensors)}
        pinned = self._pinned_of(src)
        stream = stream or torch.cuda.current_stream(self.device)
        if wait:
            self._copy.wait_stream(stream)  # earlier kernels may still read the mirrors
        bufs = None
        staged = 0
        current = set(current)
        for lo, hi, pieces in self._chunks(which):
            if self._direct(pieces, current):
                continue
            if self._direct(pieces, pinned):
                with torch.cuda.stream(self._copy):
                    self._up_direct(pieces, src)
                continue
            bufs = bufs or self._buffers()
            slot = bufs[staged % 2]
            staged += 1
            slot["event"].synchronize()  # the DMA that last read this buffer is done
            buf = slot["buf"]
            for i, s, e in pieces:
                at = self.offsets[i] + s - lo
                _copy(buf[at:at + e - s], src[i][s:e])
            with torch.cuda.stream(self._copy):
                self.flat[lo:hi].copy_(buf[:hi - lo], non_blocking=True)
                slot["event"].record(self._copy)
            self.bytes_h2d += (hi - lo) * self.flat.element_size()
        stream.wait_stream(self._copy)
        # the caller may change the host tensors on return
        if pinned:
            self._copy.synchronize()
        for slot in bufs or ():
            slot["event"].synchronize()

    def download(self, tensors, which=None, stream=None):
        """tensors[k] (host, contiguous) <- views[which[k]], after the work queued on `stream`."""
        which = list(range(len(self.numels))) if which is None else list(which)
        tensors = list(tensors)
        self._check(tensors, which)
        dst = {i: t.detach().view(-1) for i, t in zip(which, tensors)}
        pinned = self._pinned_of(dst)
        stream = stream or torch.cuda.current_stream(self.device)
        self._copy.wait_stream(stream)
        chunks = []
        for lo, hi, pieces in self._chunks(which):
            if self._direct(pieces, pinned):
                with torch.cuda.stream(self._copy):
                    self._down_direct(pieces, dst)
            else:
                chunks.append((lo, hi, pieces))
        bufs = self._buffers() if chunks else []

        def fetch(k):
            lo, hi, _ = chunks[k]
            slot = bufs[k % 2]
            with torch.cuda.stream(self._copy):
                slot["buf"][:hi - lo].copy_(self.flat[lo:hi], non_blocking=True)
                slot["event"].record(self._copy)
            self.bytes_d2h += (hi - lo) * self.flat.element_size()

        for k in range(min(2, len(chunks))):
            fetch(k)
        for k, (lo, hi, pieces) in enumerate(chunks):
            slot = bufs[k % 2]
            slot["event"].synchronize()
            for i, s, e in pieces:
                at = self.offsets[i] + s - lo
                _copy(dst[i][s:e], slot["buf"][at:at + e - s])
            if k + 2 < len(chunks):
                fetch(k + 2)  # this buffer is free again
        if pinned:
            self._copy.synchronize()  # the host tensors hold the data on return
        stream.wait_stream(self._copy)

    def pipeline(self, tensors, which, launch, stream=None, wait=True, current=()):
        """Per chunk of the listed mirrors: upload it from the host tensors, run
        launch(lo, hi, pieces, stream) (device work on those elements, enqueued on
        `stream`), then download it back into the same host tensors.  Uploads go
        ahead as fast as the link takes them; each chunk comes back (one of
        _DOWN_BUFFERS pinned buffers, a second copy stream) once its launch has run,
        and the host copies finished downloads out between uploads, so chunks go
        up and come back at the same time.  Returns with every host tensor
        updated, later work on `stream` ordered after the downloads.  wait=False:
        the uploads do not wait for the work already queued on `stream` (for a
        caller that knows none of it touches these mirrors; the launches still
        follow it).  pieces: (index, start, end) of each listed tensor's elements
        in the chunk.  current: indices whose mirrors already hold their host
        tensors' values (kept resident since the last pass); a chunk made of such
        tensors only is launched without its upload and still comes back."""
        which = list(which)
        tensors = list(tensors)
        self._check(tensors, which)
        host = {i: t.detach().view(-1) for i, t in zip(which, tensors)}
        pinned = self._pinned_of(host)
        stream = stream or torch.cuda.current_stream(self.device)
        if self._copy_down is None:
            self._copy_down = shared_stream(self.device, "down")
        chunks = self._chunks(which)
        staged_chunks = sum(not self._direct(pieces, pinned) for _, _, pieces in chunks)
        if staged_chunks and self._pinned_down is None:
            self._pinned_down = self._new_buffers(self._DOWN_BUFFERS)
        up = self._buffers() if staged_chunks else []
        free = list(self._pinned_down) if staged_chunks else []
        if wait:
            self._copy.wait_stream(stream)  # earlier kernels may still read the mirrors
        size = self.flat.element_size()
        launched = collections.deque()   # chunks whose download is not enqueued yet
        inflight = collections.deque()   # downloads not copied out yet

        def copy_out(item):
            lo, hi, pieces, slot = item
            slot["event"].synchronize()
            for i, s, e in pieces:
                at = self.offsets[i] + s - lo
                _copy(host[i][s:e], slot["buf"][at:at + e - s])
            free.append(slot)

        def service(block):
            done = False
            while inflight and inflight[0][3]["event"].query():
                copy_out(inflight.popleft())
                done = True
            if block and not done and inflight:
                copy_out(inflight.popleft())
            while launched and free:
                lo, hi, pieces = launched.popleft()
                slot = free.pop(0)
                self._copy_down.wait_stream(stream)  # after this chunk's launch
                with torch.cuda.stream(self._copy_down):
                    slot["buf"][:hi - lo].copy_(self.flat[lo:hi], non_blocking=True)
                    slot["event"].record(self._copy_down)
                self.bytes_d2h += (hi - lo) * size
                inflight.append((lo, hi, pieces, slot))

        staged = 0
        current = set(current)
        for lo, hi, pieces in chunks:
            resident = self._direct(pieces, current)
            if self._direct(pieces, pinned):
                # pinned host tensors: DMA up, the launch, DMA back, nothing for the host
                if not resident:
                    with torch.cuda.stream(self._copy):
                        self._up_direct(pieces, host)
                    stream.wait_stream(self._copy)
                launch(lo, hi, pieces, stream)
                self._copy_down.wait_stream(stream)
                with torch.cuda.stream(self._copy_down):
                    self._down_direct(pieces, host)
                service(block=False)
                continue
            if not resident:
                slot = up[staged % 2]
                staged += 1
                slot["event"].synchronize()  # the upload that last read this buffer is done
                for i, s, e in pieces:
                    at = self.offsets[i] + s - lo
                    _copy(slot["buf"][at:at + e - s], host[i][s:e])
                with torch.cuda.stream(self._copy):
                    self.flat[lo:hi].copy_(slot["buf"][:hi - lo], non_blocking=True)
                    slot["event"].record(self._copy)
                self.bytes_h2d += (hi - lo) * size
                stream.wait_stream(self._copy)
            launch(lo, hi, pieces, stream)
            launched.append((lo, hi, pieces))
            service(block=False)
        while launched or inflight:
            service(block=True)
        for slot in up:
            slot["event"].synchronize()  # the caller may change the host tensors on return
        if pinned:
            self._copy_down.synchronize()  # the direct downloads have landed
        stream.wait_stream(self._copy_down)

    def whole_tensor_chunks(self, which):
        """True when every chunk of the listed mirrors holds whole tensors only."""
        return all(s == 0 and e == self.numels[i]
                   for _, _, pieces in self._chunks(which) for i, s, e in pieces)
