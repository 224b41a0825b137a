"""Pins the oracle's restatement of export.py:16-43 with the reference's own assertions.

tests/test_fp16.py:16-26 exports with chunk_elements=17 and checks every shard against
numpy's float16 conversion of the weights and the parameter count; the manifest's
SHA-256 must be the digest of the shard bytes, and the tied head must appear as an alias.
"""
import hashlib
import json

import numpy as np
import pytest
import torch
from torch import nn

from oracle import reference as R


class Config:
    def to_dict(self):
        return dict(width=8)


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.config = Config()
        self.embedding = nn.Embedding(40, 8)
        self.gate = nn.Linear(8, 19)
        self.lm_head = nn.Linear(8, 40, bias=False)
        self.lm_head.weight = self.embedding.weight


def write_state(root, model, dirty=False):
    root.mkdir(parents=True)
    entries = {n: dict(shape=list(p.shape), size=p.numel(), file=f"{i:05}.bin")
               for i, (n, p) in enumerate(model.named_parameters())}
    for name, p in model.named_parameters():
        e = entries[name]
        w = p.detach().numpy().reshape(-1).astype(np.float32)
        np.stack([w, np.ones_like(w), np.ones_like(w)]).tofile(root / e["file"])
    (root / "manifest.json").write_text(json.dumps(dict(entries=entries, step=3, dirty=dirty,
                                                        config=model.config.to_dict())))


def test_reference_assertions_on_the_oracle_export(tmp_path):
    torch.manual_seed(2)
    model = Tiny()
    write_state(tmp_path / "state", model)
    manifest = R.export_fp16_reference(tmp_path / "state", tmp_path / "export", model, chunk_elements=17)
    assert manifest["parameters"] == sum(p.numel() for p in model.parameters())
    assert manifest["aliases"] == {"lm_head.weight": "embedding.weight"}
    assert manifest["format"] == "morph-fp16-shards-v1" and manifest["step"] == 3
    for name, p in model.named_parameters():
        entry = manifest["weights"][name]
        data = (tmp_path / "export" / entry["file"]).read_bytes()
        values = np.frombuffer(data, dtype="<f2")
        np.testing.assert_array_equal(values, p.detach().numpy().astype(np.float16).flatten())
        assert entry["sha256"] == hashlib.sha256(data).hexdigest()
        assert entry["shape"] == list(p.shape) and entry["dtype"] == "float16"
    assert json.loads((tmp_path / "export" / "manifest.json").read_text()) == manifest


def test_oracle_export_refuses_dirty_and_out_of_range(tmp_path):
    model = Tiny()
    write_state(tmp_path / "a", model, dirty=True)
    with pytest.raises(ValueError, match="incomplete"):
        R.export_fp16_reference(tmp_path / "a", tmp_path / "ea", model)
    with torch.no_grad():
        model.gate.weight[3, 2] = 70000.0
    write_state(tmp_path / "b", model)
    with pytest.raises(ValueError, match="finite FP16"):
        R.export_fp16_reference(tmp_path / "b", tmp_path / "eb", model)
