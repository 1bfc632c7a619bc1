"""Prompt-cache files in the reference's savePromptCache / loadPromptCache
format (Libraries/MLXLMCommon/KVCache.swift:1244-1300 and :1307-1388).

A safetensors file whose tensors are "i.j" = state[j] of layer cache i, and
whose string metadata holds
  "0.i.j" = metaState[j] of layer cache i,
  "1.key" = user metadata,
  "2.i"   = the class name of layer cache i
(the flattened [cache_info, metadata, cache_classes] triple the reference
writes, KVCache.swift:1280-1300).

A BlockSparseKVCache is written under its own class name with its seven
metaState values, or, with dense_compatible=True, under the reference's
"KVCache" / "QuantizedKVCache" names and metaState conventions
(KVCache.swift:141-147, :935-943), so that the reference loads the file as a
dense cache.  Loading takes a factory that builds the empty cache for each
layer (the block-sparse geometry and the query head count are not part of
a dense cache's file) and fills it through its `state` setter.
"""
from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch
from safetensors import safe_open
from safetensors.torch import save_file

CLASS_NAME = "BlockSparseKVCache"
DENSE = "KVCache"
QUANTIZED = "QuantizedKVCache"
QUANTIZED_STEP = 256  # QuantizedKVCache.step (KVCache.swift:731, :739)


def _entries(cache, dense_compatible: bool) -> Tuple[List[torch.Tensor], List[str], str]:
    state = list(cache.state)
    if not dense_compatible:
        return state, list(cache.metaState), CLASS_NAME
    if cache.bits:
        return state, [str(QUANTIZED_STEP), str(cache.offset), str(cache.groupSize),
                       str(cache.bits)], QUANTIZED
    return state, [""], DENSE


def savePromptCache(path: str, cache: Sequence, metadata: Optional[Dict[str, str]] = None,
                    dense_compatible: bool = False) -> None:
    """Writes the layer caches' state and metaState to a safetensors file."""
    arrays: Dict[str, torch.Tensor] = {}
    meta: Dict[str, str] = {}
    for i, c in enumerate(cache):
        state, info, cls = _entries(c, dense_compatible)
        for j, a in enumerate(state):
            arrays[f"{i}.{j}"] = a.detach().to("cpu", copy=True).contiguous()
        for j, v in enumerate(info):
            meta[f"0.{i}.{j}"] = v
        meta[f"2.{i}"] = cls
    for k, v in (metadata or {}).items():
        meta[f"1.{k}"] = v
    save_file(arrays, path, metadata=meta)


def _indexed(keys, prefix: str) -> Dict[int, Dict[int, str]]:
    """{i: {j: key}} for keys "prefix i.j"."""
    out: Dict[int, Dict[int, str]] = {}
    for k in keys:
        if not k.startswith(prefix):
            continue
        parts = k[len(prefix):].split(".")
        if len(parts) != 2 or not (parts[0].isdigit() and parts[1].isdigit()):
            raise ValueError(f"malformed prompt-cache key {k!r}")
        out.setdefault(int(parts[0]), {})[int(parts[1])] = k
    return out


def _ordered(d: Dict[int, str], what: str) -> List[str]:
    if sorted(d) != list(range(len(d))):
        raise ValueError(f"{what} indices are not 0..{len(d) - 1}")
    return [d[j] for j in range(len(d))]


def loadPromptCache(path: str, make_cache: Callable[[int, str, List[str], List[torch.Tensor]], object],
                    device: Optional[torch.device] = None) -> Tuple[list, Dict[str, str]]:
    """Reads a prompt-cache file: (layer caches, user metadata).

    make_cache(i, class_name, metaState, state) returns the empty cache for
    layer i; it is filled with cache.state = state (moved to `device`, or to
    the cache's device), and a BlockSparseKVCache-class entry then checks
    its metaState against the cache (geometry and token count)."""
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = dict(f.metadata() or {})
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    data = _indexed(tensors.keys(), "")
    info = _indexed(meta.keys(), "0.")
    classes = {int(k[2:]): v for k, v in meta.items() if k.startswith("2.") and k[2:].isdigit()}
    user = {k[2:]: v for k, v in meta.items() if k.startswith("1.")}
    n = len(classes)
    if sorted(classes) != list(range(n)):
        raise ValueError("invalid cache metadata format")
    if any(i >= n for i in data) or any(i >= n for i in info):
        raise ValueError("mismatch in cache counts")
    caches = []
    for i in range(n):
        state = [tensors[k] for k in _ordered(data.get(i, {}), f"cache {i} state")]
        ms = [meta[k] for k in _ordered(info.get(i, {}), f"cache {i} metaState")]
        c = make_cache(i, classes[i], ms, state)
        dev = device if device is not None else getattr(c, "device", None)
        c.state = [t.to(dev) if dev is not None else t for t in state]
        if classes[i] == CLASS_NAME:
            c.metaState = ms
        caches.append(c)
    return caches, user


__all__ = ["savePromptCache", "loadPromptCache", "CLASS_NAME"]
