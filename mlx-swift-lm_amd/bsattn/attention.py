"""attentionWithCacheUpdate for the block-sparse cache.

Mirrors Libraries/MLXLMCommon/AttentionUtils.swift:37-77: the function a
model's attention module calls with freshly projected queries / keys /
values.  The reference routes on the cache's dynamic type; the block-sparse
cache is one more branch that appends the new token(s) and runs the
HIP select + gather-attention path.  Other cache types stay on the
reference's own dense path and are not handled here.
"""
from __future__ import annotations

import torch

from .cache import BlockSparseKVCache


MAX_QUERIES = 16  # query tokens per sequence of one multi-token pass


def attentionWithCacheUpdate(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                             cache, scale: float, mask="none") -> torch.Tensor:
    """queries [B, Hq, L, D], keys / values [B, Hkv, L, D] -> [B, Hq, L, D]."""
    if not isinstance(cache, BlockSparseKVCache):
        raise TypeError("attentionWithCacheUpdate here handles BlockSparseKVCache only; "
                        "other caches use the reference's dense path")
    L = queries.shape[2]
    if L == 1:
        if mask not in ("none", None):
            raise ValueError("decode (L == 1) takes no mask (BaseKVCache.makeMask returns .none)")
        cache.append(keys, values)
        return cache.decode(queries, scale)
    if L > MAX_QUERIES:
        raise NotImplementedError(f"block-sparse attention serves decode and verify passes of up to "
                                  f"{MAX_QUERIES} tokens; a {L}-token prefill is not provided")
    if mask != "causal":
        raise ValueError("a multi-token pass takes the causal mask (BaseKVCache.makeMask(n > 1))")
    cache.append(keys, values)
    return cache.decodeMulti(queries, scale)


__all__ = ["attentionWithCacheUpdate"]
