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


# A pass of up to MAX_QUERIES tokens (the speculative-verify shape, L =
# numDraft + 1) runs block-sparse, each query on its own prefix, so that its
# outputs equal token-by-token decoding; longer passes (prefill chunks) run
# dense causal attention, as the reference computes for L > 1.
MAX_QUERIES = 16


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
        return cache.appendDecode(keys, values, queries, scale)
    if mask != "causal":
        raise ValueError("a multi-token pass takes the causal mask (BaseKVCache.makeMask(n > 1))")
    cache.append(keys, values)
    if L <= MAX_QUERIES:
        return cache.decodeMulti(queries, scale)
    return cache.prefill(queries, scale)


__all__ = ["attentionWithCacheUpdate"]
