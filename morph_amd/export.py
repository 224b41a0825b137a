"""FP16 shard export from the FP32 canonical state, with the encoding on the GPU.

Reference: streamtrain/export.py:16-43 (`export_fp16`).  For every parameter it
reads the weight row of the [3, N] state file chunk by chunk, raises
ValueError('weights cannot be represented by finite FP16') at the first chunk
holding a non-finite value or one beyond +-65504, encodes the chunk with
numpy (`astype('<f2')`, round to nearest even), appends it to the shard file
and to the shard's SHA-256, fsyncs the shard, and finally writes the
`morph-fp16-shards-v1` manifest durably.

Here the FP32 rows go to the GPU (or are already there: a ResidentWindow's
state), one conversion launch per chunk encodes them and sets a per-chunk
range flag (morph_convert_f32 -- the same bits as numpy, the same condition as
export.py:33), and the FP16 bytes come back at 2 B/param.  The host keeps the
reference's order per shard -- check, write, hash chunk by chunk, so a bad
chunk leaves exactly the reference's partial output -- while SHA-256 (serial
within a shard) runs for different shards on different threads.

The reference builds the model from its own factory (morph.factory) to get the
parameter schema, the tied-parameter aliases and config.to_dict(); that
package is the caller's, so `model` is passed in.
"""
import ctypes
import fcntl
import hashlib
import json
import os
from concurrent.futures import ThreadPoolExecutor
from contextlib import nullcontext
from pathlib import Path

import numpy as np
import torch

from . import _lib
from ._lib import check, lib, stream_handle

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
    """FP32 row (host file or device tensor) -> FP16 bytes + one range flag per chunk."""

    def __init__(self, device, chunk_elements):
        self.device = device
        self.chunk = chunk_elements
        self.stream = torch.cuda.Stream(device)

    def encode(self, row_dev):
        n = row_dev.numel()
        chunks = max(1, -(-n // self.chunk))
        out = torch.empty(n, dtype=torch.float16, device=self.device)
        flags = torch.zeros(chunks, dtype=torch.int32, device=self.device)
        L, sh = lib(), stream_handle(self.stream)
        with torch.cuda.stream(self.stream):
            self.stream.wait_stream(torch.cuda.current_stream(self.device))
            for k in range(chunks):
                a, b = k * self.chunk, min((k + 1) * self.chunk, n)
                if b > a:
                    check(L.morph_convert_f32(
                        ctypes.c_void_p(row_dev.data_ptr() + 4 * a), ctypes.c_void_p(out.data_ptr() + 2 * a),
                        _lib.DTYPE_F16, b - a, ctypes.c_void_p(flags.data_ptr() + 4 * k), sh))
            host = torch.empty(n, dtype=torch.float16, pin_memory=True)
            host.copy_(out, non_blocking=True)
            hflags = flags.to("cpu", non_blocking=True)
        self.stream.synchronize()
        return host.numpy(), hflags.numpy()


def _write_shard(path, encoded, flags, chunk):
    """Check, write and hash chunk by chunk in the reference's order (export.py:29-35)."""
    digest = hashlib.sha256()
    with path.open("wb") as handle:
        for k, start in enumerate(range(0, encoded.size, chunk)):
            if flags[k]:
                raise ValueError(FP16_ERROR)
            data = encoded[start:start + chunk].astype("<f2", copy=False).tobytes()
            handle.write(data)
            digest.update(data)
        handle.flush()
        os.fsync(handle.fileno())
    return digest.hexdigest()


def export_fp16(state_dir, output, chunk_elements=1048576, lock_held=False, *, model, window=None,
                device=None, hash_threads=8):
    """export.py:16-43 with the encoding on the GPU.  Same files, hashes and manifest.

    model: the meta-device model the reference builds from the manifest's config
    (`model_from_config(config_from_dict(manifest['config']))`).  window: an optional
    ResidentWindow whose resident FP32 rows are used instead of reading the files.
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
        encoder = _Encoder(device, chunk_elements)
        weights, pending = {}, []
        inflight = max(2, 2 * hash_threads)  # bounds the FP16 bytes held in host memory
        with ThreadPoolExecutor(max_workers=max(1, hash_threads)) as pool:
            try:
                for name, entry in entries.items():
                    size = entry["size"]
                    if window is not None and name in window.state:
                        row = window.state[name][0]
                    else:
                        mapped = np.memmap(state_dir / entry["file"], dtype=np.float32, mode="r",
                                           shape=(3, size))
                        row = torch.from_numpy(np.ascontiguousarray(mapped[0])).to(device)
                        del mapped
                    encoded, flags = encoder.encode(row)
                    while sum(not f.done() for _, _, f in pending) >= inflight:
                        next(f for _, _, f in pending if not f.done()).result()
                    # shards are independent: written and hashed in parallel; only the last
                    # submitted one can hold a bad chunk, since encoding stops there
                    pending.append((name, entry, pool.submit(_write_shard, output / entry["file"],
                                                             encoded, flags, chunk_elements)))
                    if flags.any():
                        break  # the reference stops at this parameter's first bad chunk
                for name, entry, fut in pending:
                    digest = fut.result()  # re-raises the bad chunk's ValueError
                    weights[name] = dict(file=entry["file"], shape=entry["shape"], dtype="float16",
                                         sha256=digest)
            finally:
                for _, _, fut in pending:
                    fut.cancel()
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
