"""FP16 shard export (morph_amd.export) against the oracle's restatement of export.py:16-43.

Shard files byte-identical (numpy's FP16 encoding), SHA-256 and manifest equal, the
same ValueError at the same chunk with the same partial output, the same refusals
(dirty state, existing output, held run lock), and the same result when the FP32 rows
come from an HBM-resident window instead of the files.
"""
import fcntl
import json

import numpy as np
import pytest
import torch
from torch import nn

from morph_amd.export import export_fp16
from morph_amd.window import ResidentWindow
from oracle import reference as R

pytestmark = pytest.mark.gpu


class Config:
    def to_dict(self):
        return dict(vocab=64, width=32, layers=1)


class Tiny(nn.Module):
    """Parameter layout with a tied head, like the reference model's (export.py:37-38)."""

    def __init__(self):
        super().__init__()
        self.config = Config()
        self.embedding = nn.Embedding(64, 32)
        self.gate = nn.Linear(32, 48, bias=False)
        self.norm = nn.LayerNorm(32)
        self.lm_head = nn.Linear(32, 64, bias=False)
        self.lm_head.weight = self.embedding.weight


def make_state(root, model, seed=0, step=7, dirty=False, edits=None):
    root.mkdir(parents=True)
    entries = {n: dict(shape=list(p.shape), size=p.numel(), file=f"{i:05}.bin")
               for i, (n, p) in enumerate(model.named_parameters())}
    rng = np.random.RandomState(seed)
    for name, e in entries.items():
        state = np.zeros((3, e["size"]), np.float32)
        state[0] = (rng.randn(e["size"]) * 3).astype(np.float32)
        state[1:] = rng.randn(2, e["size"]).astype(np.float32)  # moments are never exported
        for (ename, idx), value in (edits or {}).items():
            if ename == name:
                state[0, idx] = value
        state.tofile(root / e["file"])
    (root / "manifest.json").write_text(json.dumps(dict(entries=entries, step=step, dirty=dirty,
                                                        config=Config().to_dict())))
    return entries


def same_dirs(a, b):
    fa, fb = sorted(p.name for p in a.iterdir()), sorted(p.name for p in b.iterdir())
    assert fa == fb, (fa, fb)
    for name in fa:
        if name == "manifest.json":
            assert json.loads((a / name).read_text()) == json.loads((b / name).read_text())
        else:
            assert (a / name).read_bytes() == (b / name).read_bytes(), name


@pytest.mark.parametrize("chunk,segment", [(100, 1 << 22), (100, 250), (1048576, 1 << 22)])
def test_export_matches_reference_bytes_and_manifest(tmp_path, chunk, segment):
    """segment 250 with chunk 100: rows move in segments of two chunks (bounded memory)."""
    model = Tiny()
    make_state(tmp_path / "run" / "state", model,
               edits={("gate.weight", 5): 65504.0, ("gate.weight", 6): -65504.0,
                      ("norm.weight", 0): 65503.9, ("norm.weight", 1): 1e-8})
    got = export_fp16(tmp_path / "run" / "state", tmp_path / "gpu", chunk, model=model,
                      segment_elements=segment)
    ref = R.export_fp16_reference(tmp_path / "run" / "state", tmp_path / "cpu", model, chunk)
    assert got == ref
    assert got["aliases"] == {"lm_head.weight": "embedding.weight"}
    same_dirs(tmp_path / "gpu", tmp_path / "cpu")


@pytest.mark.parametrize("bad", [65504.5, 65519.0, float("inf"), float("nan")])
@pytest.mark.parametrize("segment", [1 << 22, 512])
def test_unrepresentable_weight_raises_at_the_same_chunk(tmp_path, bad, segment):
    """65519 rounds to 65504 in FP16 but the reference still refuses it (|w| > 65504).
    segment 512: the bad chunk (elements 512-767) opens the row's second segment."""
    model = Tiny()
    make_state(tmp_path / "run" / "state", model, edits={("gate.weight", 700): bad})
    with pytest.raises(ValueError, match="finite FP16"):
        export_fp16(tmp_path / "run" / "state", tmp_path / "gpu", 256, model=model,
                    segment_elements=segment)
    with pytest.raises(ValueError, match="finite FP16"):
        R.export_fp16_reference(tmp_path / "run" / "state", tmp_path / "cpu", model, 256)
    same_dirs(tmp_path / "gpu", tmp_path / "cpu")  # same complete and partial shards


def test_refusals(tmp_path):
    model = Tiny()
    make_state(tmp_path / "run" / "state", model, dirty=True)
    with pytest.raises(ValueError, match="incomplete optimizer transaction"):
        export_fp16(tmp_path / "run" / "state", tmp_path / "out", model=model)
    assert not (tmp_path / "out").exists()
    make_state(tmp_path / "run2" / "state", model)
    (tmp_path / "exists").mkdir()
    with pytest.raises(FileExistsError):
        export_fp16(tmp_path / "run2" / "state", tmp_path / "exists", model=model)
    with open(tmp_path / "run2" / "run.lock", "a+") as held:
        fcntl.flock(held, fcntl.LOCK_EX | fcntl.LOCK_NB)
        with pytest.raises(RuntimeError, match="stop training"):
            export_fp16(tmp_path / "run2" / "state", tmp_path / "out2", model=model)
    other = nn.Linear(3, 3)
    other.config = Config()
    with pytest.raises(ValueError, match="schema differs"):
        export_fp16(tmp_path / "run2" / "state", tmp_path / "out3", model=other)


def test_export_from_resident_window_equals_file_export(tmp_path):
    model = Tiny()
    entries = make_state(tmp_path / "run" / "state", model)

    class Store:
        root = tmp_path / "run" / "state"

        def fault(self, point):
            return None
    store = Store()
    store.entries = entries
    win = ResidentWindow(store, list(entries), torch.float16)
    win.load()
    export_fp16(tmp_path / "run" / "state", tmp_path / "win", 300, model=model, window=win,
                segment_elements=600)
    R.export_fp16_reference(tmp_path / "run" / "state", tmp_path / "cpu", model, 300)
    same_dirs(tmp_path / "win", tmp_path / "cpu")


def test_a_failed_shard_write_stops_the_export(tmp_path, monkeypatch):
    """The reference's serial loop (export.py:26-36) stops at its first I/O error, so the
    output holds the shards up to the failing one.  With one shard writer at a time the
    GPU export ends the same way: the first shard's fsync fails, the error propagates,
    and no later shard is started."""
    import os as os_mod
    from morph_amd import export as export_mod
    model = Tiny()
    make_state(tmp_path / "run" / "state", model)
    real_fsync = os_mod.fsync
    calls = []

    def failing_fsync(fd):
        calls.append(fd)
        if len(calls) == 1:
            raise OSError(5, "injected I/O error")
        return real_fsync(fd)

    monkeypatch.setattr(export_mod.os, "fsync", failing_fsync)
    with pytest.raises(OSError, match="injected"):
        export_fp16(tmp_path / "run" / "state", tmp_path / "gpu", 100, model=model, hash_threads=1)
    assert sorted(p.name for p in (tmp_path / "gpu").iterdir()) == ["00000.bin"]


def test_a_truncated_state_file_is_refused_where_the_reference_refuses_it(tmp_path):
    """The reference maps each [3, N] file with np.memmap before it opens that shard, so a file
    shorter than its schema raises ValueError there and the output holds the shards before it.
    The GPU export reads the rows with pread and checks the size at the same point."""
    model = Tiny()
    entries = make_state(tmp_path / "run" / "state", model)
    victim = tmp_path / "run" / "state" / entries["gate.weight"]["file"]
    victim.write_bytes(victim.read_bytes()[:-4])
    with pytest.raises(ValueError, match="mmap length"):
        export_fp16(tmp_path / "run" / "state", tmp_path / "gpu", 100, model=model)
    with pytest.raises(ValueError, match="mmap length"):
        R.export_fp16_reference(tmp_path / "run" / "state", tmp_path / "cpu", model, 100)
    same_dirs(tmp_path / "gpu", tmp_path / "cpu")
