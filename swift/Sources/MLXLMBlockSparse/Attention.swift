import MLX
import MLXLMCommon

/// Passes of up to this many query tokens (the speculative-verify shape,
/// L = numDraft + 1) run block-sparse, each query on its own prefix, so that
/// they equal token-by-token decoding; longer passes (prefill chunks) run
/// dense causal attention over the whole cache.
public let blockSparseMaxQueries = 16

/// The block-sparse branch of attentionWithCacheUpdate
/// (Libraries/MLXLMCommon/AttentionUtils.swift:37-77): MLXLMCommon's entry
/// point checks AttendingKVCache before its quantized branch and hands a
/// block-sparse cache (16-bit or quantized) the new tokens here, so models
/// keep calling attentionWithCacheUpdate unchanged.
extension BlockSparseKVCache: AttendingKVCache {
    /// queries [B, Hq, L, D], keys / values [B, Hkv, L, D].  L = 1 is one
    /// decode step (mask .none, as BaseKVCache.makeMask gives for n = 1);
    /// a longer pass takes the causal mask and runs as a speculative-verify
    /// pass up to blockSparseMaxQueries tokens, else as a prefill chunk.
    public func updateAndAttend(
        queries: MLXArray, keys: MLXArray, values: MLXArray, scale: Float,
        mask: MLXFast.ScaledDotProductAttentionMaskMode
    ) -> MLXArray {
        let L = queries.dim(2)
        if L == 1 {
            guard case .none = mask else {
                fatalError("decode (L == 1) takes no mask (BaseKVCache.makeMask returns .none)")
            }
            return appendDecode(keys: keys, values: values, queries: queries, scale: scale)
        }
        guard case .causal = mask else {
            fatalError("a multi-token pass over a BlockSparseKVCache takes the causal mask")
        }
        append(keys: keys, values: values)
        if L <= blockSparseMaxQueries {
            return decodeMulti(queries: queries, scale: scale)
        }
        return prefill(queries: queries, scale: scale)
    }
}
