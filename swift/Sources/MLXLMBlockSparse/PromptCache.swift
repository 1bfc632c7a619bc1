import MLX
import MLXLMCommon

/// A prompt-cache entry that cannot become a block-sparse cache.
public struct BlockSparsePromptCacheError: Error, CustomStringConvertible {
    public let description: String
}

extension BlockSparse {
    /// The class name block-sparse caches carry in prompt-cache files
    /// (savePromptCache, Libraries/MLXLMCommon/KVCache.swift:1244-1300).
    public static let promptCacheClassName = "BlockSparseKVCache"

    /// Makes loadPromptCache (KVCache.swift:1307-1388) rebuild
    /// "BlockSparseKVCache" entries.
    ///
    /// A file entry holds the cache's `state` ([keys, values] of 16-bit
    /// caches, [kw, ks, kb, vw, vs, vb] of quantized ones, rows = sequences)
    /// and its seven `metaState` values [blockSize, topK, sinkBlocks,
    /// recentBlocks, offset, kvBits, groupSize].  The query head count and
    /// the capacity are the model's, not the file's: `qHeads`, `maxTokens`
    /// per sequence and `maxSeqs` (default: the rows in the file) size the
    /// new cache.  loadPromptCache then sets `state` (the tokens) and
    /// `metaState` (which checks the geometry and the token count of row 0).
    public static func registerPromptCacheClass(
        qHeads: Int, maxTokens: Int, maxSeqs: Int? = nil, device: BlockSparseDevice? = nil
    ) {
        PromptCacheClasses.register(promptCacheClassName) { metaState, state in
            let v = metaState.compactMap { Int($0) }
            guard metaState.count == 7, v.count == 7 else {
                throw BlockSparsePromptCacheError(
                    description: "BlockSparseKVCache metaState must hold 7 integers, got \(metaState)")
            }
            let (blockSize, topK, sinkBlocks, recentBlocks, kvBits, groupSize) =
                (v[0], v[1], v[2], v[3], v[5], v[6])
            guard state.count == (kvBits == 0 ? 2 : 6), state[0].ndim == 4 else {
                throw BlockSparsePromptCacheError(
                    description: "BlockSparseKVCache state must be 2 (16-bit) or 6 (kvBits \(kvBits)) "
                        + "arrays [B, Hkv, T, ...], got \(state.count)")
            }
            let rows = maxSeqs ?? state[0].dim(0)
            let kvHeads = state[0].dim(1)
            let headDim = kvBits == 0 ? state[0].dim(3) : state[0].dim(3) * 32 / kvBits
            let blocks = (max(maxTokens, state[0].dim(2)) + blockSize - 1) / blockSize
            if kvBits == 0 {
                return BlockSparseKVCache(
                    maxSeqs: rows, qHeads: qHeads, kvHeads: kvHeads, headDim: headDim,
                    blockSize: blockSize, dtype: state[0].dtype, topK: topK, sinkBlocks: sinkBlocks,
                    recentBlocks: recentBlocks, maxBlocksPerSeq: blocks, device: device)
            }
            return QuantizedBlockSparseKVCache(
                maxSeqs: rows, qHeads: qHeads, kvHeads: kvHeads, headDim: headDim,
                blockSize: blockSize, topK: topK, sinkBlocks: sinkBlocks, recentBlocks: recentBlocks,
                maxBlocksPerSeq: blocks, bits: kvBits, groupSize: groupSize, device: device)
        }
    }
}
