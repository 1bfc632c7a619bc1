"""Prompt-cache files: the reference's savePromptCache / loadPromptCache
layout (Libraries/MLXLMCommon/KVCache.swift:1244-1388): tensors "i.j",
metadata "0.i.j" (metaState), "1.key" (user), "2.i" (class name).  CPU: a
stand-in cache object with the same state / metaState surface; the GPU test
round-trips real caches."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from bsattn.prompt_cache import CLASS_NAME, loadPromptCache, savePromptCache


class StandIn:
    """The state / metaState surface savePromptCache and loadPromptCache use."""

    def __init__(self, state=None, meta=None, bits=0, offset=0, group=64):
        self.state = list(state or [])
        self.metaState = list(meta or [])
        self.bits, self.offset, self.groupSize = bits, offset, group
        self.device = None


def _layers():
    g = torch.Generator().manual_seed(3)
    k0 = torch.randn(2, 4, 40, 128, generator=g).to(torch.bfloat16)
    v0 = torch.randn(2, 4, 40, 128, generator=g).to(torch.bfloat16)
    k1 = torch.randn(2, 4, 40, 128, generator=g).to(torch.bfloat16)
    v1 = torch.randn(2, 4, 40, 128, generator=g).to(torch.bfloat16)
    meta = ["64", "32", "1", "1", "40", "0", "64"]
    return [StandIn([k0, v0], meta, offset=40), StandIn([k1, v1], meta, offset=40)]


def test_file_layout_matches_the_reference(tmp_path):
    path = str(tmp_path / "p.safetensors")
    layers = _layers()
    savePromptCache(path, layers, {"model": "llama", "step": "7"})
    with safe_open(path, framework="pt") as f:
        keys = sorted(f.keys())
        meta = f.metadata()
        assert keys == ["0.0", "0.1", "1.0", "1.1"]
        assert torch.equal(f.get_tensor("1.0"), layers[1].state[0])
    assert meta["2.0"] == CLASS_NAME and meta["2.1"] == CLASS_NAME
    assert [meta[f"0.1.{j}"] for j in range(7)] == layers[1].metaState
    assert meta["1.model"] == "llama" and meta["1.step"] == "7"
    assert len(meta) == 2 * 7 + 2 + 2


def test_round_trip(tmp_path):
    path = str(tmp_path / "p.safetensors")
    layers = _layers()
    savePromptCache(path, layers, {"a": "b"})
    seen = []

    def make(i, cls, ms, state):
        seen.append((i, cls, ms, [tuple(t.shape) for t in state]))
        return StandIn()

    caches, user = loadPromptCache(path, make)
    assert user == {"a": "b"}
    assert [s[:2] for s in seen] == [(0, CLASS_NAME), (1, CLASS_NAME)]
    for a, b in zip(caches, layers):
        assert len(a.state) == 2 and all(torch.equal(x, y) for x, y in zip(a.state, b.state))
        assert a.metaState == b.metaState


def test_dense_compatible_names_and_meta_state(tmp_path):
    path = str(tmp_path / "d.safetensors")
    q = StandIn([torch.zeros(1, 2, 8, 16, dtype=torch.int32)] * 6, ["x"] * 7, bits=4, offset=8)
    savePromptCache(path, _layers()[:1] + [q], dense_compatible=True)
    with safe_open(path, framework="pt") as f:
        meta = f.metadata()
        assert len(list(f.keys())) == 2 + 6
    # KVCacheSimple: metaState [""] (KVCache.swift:141-147); QuantizedKVCache:
    # [step, offset, groupSize, bits] (KVCache.swift:935-943)
    assert meta["2.0"] == "KVCache" and meta["0.0.0"] == "" and "0.0.1" not in meta
    assert meta["2.1"] == "QuantizedKVCache"
    assert [meta[f"0.1.{j}"] for j in range(4)] == ["256", "8", "64", "4"]


def test_loads_a_reference_written_dense_file(tmp_path):
    """The exact keys the reference writes for two KVCacheSimple layers."""
    path = str(tmp_path / "r.safetensors")
    k = torch.arange(2 * 3 * 5 * 128, dtype=torch.float32).reshape(2, 3, 5, 128).to(torch.float16)
    save_file({"0.0": k, "0.1": k + 1, "1.0": k + 2, "1.1": k + 3},
              path, metadata={"0.0.0": "", "0.1.0": "", "2.0": "KVCache", "2.1": "KVCache", "1.m": "v"})
    got = []
    caches, user = loadPromptCache(path, lambda i, cls, ms, st: got.append((cls, ms)) or StandIn())
    assert got == [("KVCache", [""]), ("KVCache", [""])]
    assert user == {"m": "v"}
    assert torch.equal(caches[1].state[1], k + 3)


@pytest.mark.parametrize("meta", [
    {"0.0.0": "", "2.1": "KVCache"},                    # class indices not 0..n-1
    {"0.0.0": "", "0.3.0": "", "2.0": "KVCache"},       # metaState for a cache that has no class
])
def test_malformed_metadata_is_rejected(tmp_path, meta):
    path = str(tmp_path / "m.safetensors")
    save_file({"0.0": torch.zeros(1, 1, 1, 128), "0.1": torch.zeros(1, 1, 1, 128)}, path, metadata=meta)
    with pytest.raises(ValueError):
        loadPromptCache(path, lambda *a: StandIn())
