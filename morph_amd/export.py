"""FP16 shard export from the FP32 canonical state, with the encoding on the GPU.

Reference: streamtrain/export.py:16-43 (`export_fp16`).  For every parameter it
reads the weight row of the [3, N] state file chunk by chunk, raises
ValueError('weights cannot be represented by finite FP16') at the first chunk
holding a non-finite value or one beyond +-65504, encodes the chunk with
numpy (`astype('<f2')`, round to nearest even), appends it to the shard file
and to the shard's SHA-256, fsyncs the shard, and finally writes the
`morph-fp16-shards-v1` manifest durably.

Here the FP32 rows go to the GPU segment by segment (or are already there: a
ResidentWindow's state), one conversion launch per chunk encodes them and sets
a per-chunk range flag (morph_convert_f32 -- the same bits as numpy, the same
condition as export.py:33), and the FP16 bytes come back at 2 B/param.  The
host keeps the reference's order per shard -- check, write, hash chunk by
chunk, so a bad chunk leaves exactly the reference's partial output -- while
SHA-256 (serial within a shard) runs for different shards on different
threads.  Memory is bounded by fixed-size segment buffers and bounded queues,
as the reference's chunked loop is ("Bounded FP16 model export", export.py:1).

The reference builds the model from its own factory (morph.factory) to get the
parameter schema, the tied-parameter aliases and config.to_dict(); that
package is the caller's, so `model` is passed in.
"""
import ctypes
import fcntl
import hashlib
import json
import os
import queue
import threading
from contextlib import nullcontext
from pathlib import Path

import torch

from . import _lib
from ._lib import check, lib, stream_handle
from .staging import read_exact

FP16_ERROR = "weights cannot be represented by finite FP16"


def _durable_json(path, value):
    """streamtrain/disk.py:durable_json: write a temp file, fsync, replace, fsync the directory."""
    path = Path(path)
    temp = path.with_suffix(".tmp")
    with temp.open("w") as handle:
        json.dump(value, handle)
        handle.flush()
        os.fsync(handle.fileno())
    os.replace(temp, path)
    fd = os.open(path.parent, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def _entries(model):
    """DiskState's schema (disk.py:46-49): name -> shape, size, file name by position."""
    return {name: dict(shape=list(p.shape), size=p.numel(), file=f"{i:05}.bin")
            for i, (name, p) in enumerate(model.named_parameters())}


class _Encoder:
    """FP32 row segments (host file or device tensor) -> FP16 bytes + one range flag per chunk.

    Fixed-size buffers (one segment of pinned FP32 staging, the device FP32 and FP16
    segment, pinned FP16 and flags), so the memory used does not depend on the
    parameter sizes.  Segments are whole multiples of the chunk, so each flag covers
    exactly one of the reference's chunks (export.py:29-33)."""

    def __init__(self, device, chunk_elements, segment_elements):
        self.device = device
        self.chunk = chunk_elements
        self.segment = chunk_elements * max(1, segment_elements // chunk_elements)
        self.stream = torch.cuda.Stream(device)
        per = -(-self.segment // self.chunk)
        self.src_host = torch.empty(self.segment, dtype=torch.float32, pin_memory=True)
        self.src_dev = torch.empty(self.segment, dtype=torch.float32, device=device)
        self.out_dev = torch.empty(self.segment, dtype=torch.float16, device=device)
        self.flags_dev = torch.zeros(per, dtype=torch.int32, device=device)
        self.out_host = torch.empty(self.segment, dtype=torch.float16, pin_memory=True)
        self.flags_host = torch.empty(per, dtype=torch.int32, pin_memory=True)

    def encode(self, lo, hi, fd=None, row_dev=None):
        """Encode elements [lo, hi) of a weight row -- row 0 of the [3, N] state file open
        as `fd` (read straight into the pinned staging), or the device tensor `row_dev` --
        and return (fp16 numpy array, per-chunk flags)."""
        n = hi - lo
        chunks = -(-n // self.chunk)
        L, sh = lib(), stream_handle(self.stream)
        with torch.cuda.stream(self.stream):
            if row_dev is None:
                read_exact(fd, self.src_host[:n].numpy(), 4 * lo)  # row 0 starts the file
                self.src_dev[:n].copy_(self.src_host[:n], non_blocking=True)
                src = self.src_dev
            else:
                self.stream.wait_stream(torch.cuda.current_stream(self.device))
                src = row_dev[lo:hi]
            self.flags_dev[:chunks].zero_()
            for k in range(chunks):
                a, b = k * self.chunk, min((k + 1) * self.chunk, n)
                check(L.morph_convert_f32(
                    ctypes.c_void_p(src.data_ptr() + 4 * a), ctypes.c_void_p(self.out_dev.data_ptr() + 2 * a),
                    _lib.DTYPE_F16, b - a, ctypes.c_void_p(self.flags_dev.data_ptr() + 4 * k), sh))
            self.out_host[:n].copy_(self.out_dev[:n], non_blocking=True)
            self.flags_host[:chunks].copy_(self.flags_dev[:chunks], non_blocking=True)
        self.stream.synchronize()
        return self.out_host[:n].numpy().copy(), self.flags_host[:chunks].numpy().copy()


class _ShardWriter(threading.Thread):
    """Writes and hashes one shard in the reference's order (export.py:29-35): per chunk,
    check its flag, write, update the SHA-256; fsync at the end.  Segments arrive through
    a bounded queue (None ends the shard); after an error the queue is still drained so
    the producer never blocks."""

    def __init__(self, path, chunk, slots):
        super().__init__(daemon=True)
        self.path, self.chunk, self.slots = path, chunk, slots
        self.queue = queue.Queue(maxsize=2)
        self.digest = None
        self.error = None

    def run(self):
        item = ()
        try:
            digest = hashlib.sha256()
            with self.path.open("wb") as handle:
                while True:
                    item = self.queue.get()
                    if item is None:
                        break
                    encoded, flags = item
                    for k, start in enumerate(range(0, encoded.size, self.chunk)):
                        if flags[k]:
                            raise ValueError(FP16_ERROR)
                        data = encoded[start:start + self.chunk].astype("<f2", copy=False).tobytes()
                        handle.write(data)
                        digest.update(data)
                handle.flush()
                os.fsync(handle.fileno())
            self.digest = digest.hexdigest()
        except BaseException as e:  # reported by result()
            self.error = e
            while item is not None:
                item = self.queue.get()
        finally:
            self.slots.release()

    def result(self):
        self.join()
        if self.error is not None:
            raise self.error
        return self.digest


def export_fp16(state_dir, output, chunk_elements=1048576, lock_held=False, *, model, window=None,
                device=None, hash_threads=8, segment_elements=1 << 22):
    """export.py:16-43 with the encoding on the GPU.  Same files, hashes and manifest.

    model: the meta-device model the reference builds from the manifest's config
    (`model_from_config(config_from_dict(manifest['config']))`).  window: an optional
    ResidentWindow whose resident FP32 rows are used instead of reading the files.
    Memory stays bounded like the reference's chunked loop: rows move in segments of
    about `segment_elements` (whole chunks), at most `hash_threads` shards are written
    and hashed at once, each with at most two encoded segments queued.
    """
    state_dir, output = Path(state_dir), Path(output)
    device = torch.device(device) if device is not None else torch.device(
        "cuda", torch.cuda.current_device())
    lock_ctx = nullcontext(None) if lock_held else (state_dir.parent / "run.lock").open("a+")
    with lock_ctx as lock:
        if lock is not None:
            try:
                fcntl.flock(lock, fcntl.LOCK_EX | fcntl.LOCK_NB)
            except BlockingIOError:
                raise RuntimeError("stop training safely before exporting a consistent model")
        manifest = json.loads((state_dir / "manifest.json").read_text())
        if manifest["dirty"]:
            raise ValueError("cannot export an incomplete optimizer transaction")
        entries = _entries(model)
        if entries != manifest["entries"]:  # DiskState.__init__ (disk.py:50-51)
            raise ValueError("disk state tensor schema differs")
        output.mkdir(parents=True, exist_ok=False)
        encoder = _Encoder(device, chunk_elements, segment_elements)
        slots = threading.Semaphore(max(1, hash_threads))
        writers = []

        def failed():
            # a writer's error ends production: the reference's serial loop stops at its
            # first error, so no shard is started, and no segment encoded, after one
            return any(w.error is not None for _, _, w in writers)

        try:
            for name, entry in entries.items():
                size = entry["size"]
                resident = window is not None and name in window.state
                row_dev = window.state[name][0] if resident else None
                fd = None if resident else os.open(state_dir / entry["file"], os.O_RDONLY)
                try:
                    if fd is not None and os.fstat(fd).st_size < 12 * size:
                        # where the reference's np.memmap of the [3, N] file refuses it
                        raise ValueError("mmap length is greater than file size")
                    slots.acquire()
                    if failed():
                        slots.release()
                        break
                    writer = _ShardWriter(output / entry["file"], chunk_elements, slots)
                    writer.start()
                    writers.append((name, entry, writer))
                    bad = False
                    try:
                        for lo in range(0, size, encoder.segment):
                            if failed():
                                bad = True
                                break
                            hi = min(lo + encoder.segment, size)
                            encoded, flags = encoder.encode(lo, hi, fd=fd, row_dev=row_dev)
                            writer.queue.put((encoded, flags))
                            if flags.any():
                                bad = True  # the reference stops at this parameter's first bad chunk
                                break
                    finally:
                        writer.queue.put(None)
                finally:
                    if fd is not None:
                        os.close(fd)
                if bad:
                    break
        finally:
            for _, _, writer in writers:
                writer.join()
        weights = {}
        for name, entry, writer in writers:
            digest = writer.result()  # re-raises the bad chunk's ValueError
            weights[name] = dict(file=entry["file"], shape=entry["shape"], dtype="float16",
                                 sha256=digest)
        canonical = {id(p): n for n, p in model.named_parameters()}
        aliases = {n: canonical[id(p)] for n, p in model.named_parameters(remove_duplicate=False)
                   if canonical[id(p)] != n}
        result = dict(format="morph-fp16-shards-v1", config=model.config.to_dict(),
                      step=manifest["step"], weights=weights, aliases=aliases,
                      lm_head=dict(kind="tied_embedding_projection", weight="embedding.weight"),
                      parameters=sum(e["size"] for e in entries.values()),
                      optimizer_included=False,
                      buffers="deterministically reconstructed from config",
                      source_precision="float32 masters", export_precision="float16")
        _durable_json(output / "manifest.json", result)
        return result
