import MLX
import MLXLMCommon

/// Passes of up to this many query tokens (the speculative-verify shape,
/// L = numDraft + 1) run block-sparse, each query on its own prefix, so that
/// they equal token-by-token decoding; longer passes (prefill chunks) run
/// dense causal attention over the whole cache.
public let blockSparseMaxQueries = 16

/// attentionWithCacheUpdate (Libraries/MLXLMCommon/AttentionUtils.swift:37-77)
/// with one more dynamic-type branch, taken before the quantized one: a
/// BlockSparseKVCache appends the new tokens and attends on the GPU through
/// libbsattn.  Every other cache, and no cache, goes to the reference's
/// function unchanged, so a model swaps its call for this one and nothing
/// else.  queries [B, Hq, L, D], keys / values [B, Hkv, L, D].
public func blockSparseAttentionWithCacheUpdate(
    queries: MLXArray,
    keys: MLXArray,
    values: MLXArray,
    cache: KVCache?,
    scale: Float,
    mask: MLXFast.ScaledDotProductAttentionMaskMode = .none
) -> MLXArray {
    guard let bs = cache as? BlockSparseKVCache else {
        return attentionWithCacheUpdate(
            queries: queries, keys: keys, values: values, cache: cache, scale: scale, mask: mask)
    }
    let L = queries.dim(2)
    if L == 1 {
        guard case .none = mask else {
            fatalError("decode (L == 1) takes no mask (BaseKVCache.makeMask returns .none)")
        }
        return bs.appendDecode(keys: keys, values: values, queries: queries, scale: scale)
    }
    guard case .causal = mask else {
        fatalError("a multi-token pass over a BlockSparseKVCache takes the causal mask")
    }
    bs.append(keys: keys, values: values)
    if L <= blockSparseMaxQueries {
        return bs.decodeMulti(queries: queries, scale: scale)
    }
    return bs.prefill(queries: queries, scale: scale)
}
