import CBSAttn
import Foundation
import MLX
import MLXLMCommon

/// A paged KV cache whose decode attends only to the blocks that matter.
///
/// Tokens live in pages of `blockSize` tokens per sequence and KV head in
/// HBM, each completed block with a summary (the mean of its keys).  A decode
/// step scores every block of a sequence with max over the GQA group of
/// q · summary, keeps `sinkBlocks` leading, `recentBlocks` trailing and the
/// `topK` best blocks, and computes softmax(q kᵀ · scale) v over the tokens of
/// those blocks only (libbsattn, `include/bsattn.h`).
///
/// Conforms to the reference's `KVCache` (Libraries/MLXLMCommon/KVCache.swift:38-77)
/// with the semantics of `KVCacheSimple` (:328-437) for `update`, `state`,
/// `trim` and `copy`, and of `BaseKVCache.makeMask` (:160-174).  Rows of a
/// batch are independent sequences with their own lengths; `offset` is the
/// length of row 0, as the reference keeps one offset per cache (:40).
public class BlockSparseKVCache: KVCache {
    let handle: OpaquePointer
    public let desc: bsattn_desc
    public let device: BlockSparseDevice

    /// The cache a library handle belongs to; `copy()` makes its subclass's
    /// instances through this initializer.
    public required init(adopting handle: OpaquePointer, desc: bsattn_desc, device: BlockSparseDevice) {
        self.handle = handle
        self.desc = desc
        self.device = device
    }

    /// A cache for `maxSeqs` sequences of at most `maxBlocksPerSeq` blocks.
    /// `dtype` is the dtype of queries, keys, values and outputs (.float16 or
    /// .bfloat16); `kvBits` 4 or 8 stores keys and values as MLX-affine codes
    /// with fp16 scales and biases per `groupSize` elements (fp16 only; see
    /// `QuantizedBlockSparseKVCache`).  `numPages` 0 sizes the pool for every
    /// sequence at full length.
    public convenience init(
        maxSeqs: Int, qHeads: Int, kvHeads: Int, headDim: Int = 128, blockSize: Int = 64,
        dtype: DType = .bfloat16, topK: Int = 32, sinkBlocks: Int = 1, recentBlocks: Int = 1,
        maxBlocksPerSeq: Int, numPages: Int = 0, kvBits: Int = 0, groupSize: Int = 64,
        device: BlockSparseDevice? = nil
    ) {
        guard let dev = device ?? BlockSparse.device else {
            fatalError("BlockSparseKVCache: no BlockSparseDevice given and BlockSparse.device is unset")
        }
        precondition(dtype == .float16 || dtype == .bfloat16, "BlockSparseKVCache holds float16 or bfloat16")
        var d = bsattn_desc()
        d.max_seqs = Int32(maxSeqs)
        d.num_q_heads = Int32(qHeads)
        d.num_kv_heads = Int32(kvHeads)
        d.head_dim = Int32(headDim)
        d.block_size = Int32(blockSize)
        d.dtype = dtype == .bfloat16 ? 1 : 0  // BSATTN_BF16 : BSATTN_F16
        d.kv_bits = Int32(kvBits)
        d.group_size = Int32(groupSize)
        d.top_k = Int32(topK)
        d.sink_blocks = Int32(sinkBlocks)
        d.recent_blocks = Int32(recentBlocks)
        d.max_blocks_per_seq = Int32(maxBlocksPerSeq)
        d.num_pages = Int64(numPages)
        d.device = dev.ordinal
        var h: OpaquePointer? = nil
        bsCheck(bsattn_cache_create(&d, &h), "bsattn_cache_create")
        self.init(adopting: h!, desc: d, device: dev)
    }

    deinit {
        _ = bsattn_cache_destroy(handle)
    }

    // MARK: geometry

    public var dtype: DType { desc.dtype == 1 ? .bfloat16 : .float16 }
    public var kvHeads: Int { Int(desc.num_kv_heads) }
    public var qHeads: Int { Int(desc.num_q_heads) }
    public var headDim: Int { Int(desc.head_dim) }
    public var blockSize: Int { Int(desc.block_size) }
    public var topK: Int { Int(desc.top_k) }
    public var sinkBlocks: Int { Int(desc.sink_blocks) }
    public var recentBlocks: Int { Int(desc.recent_blocks) }

    var info: bsattn_info {
        var i = bsattn_info()
        bsCheck(bsattn_cache_info(handle, &i), "bsattn_cache_info")
        return i
    }

    /// Width of selected-block index outputs: sink + recent + topK.
    public var nselMax: Int { Int(info.nsel_max) }
    /// Pages no sequence holds.
    public var freePages: Int { Int(info.free_pages) }

    var stream: UnsafeMutableRawPointer? { device.stream }

    /// Tokens held by sequence `seq`.
    public func seqLen(_ seq: Int) -> Int {
        var n: Int32 = 0
        bsCheck(bsattn_seq_len(handle, Int32(seq), &n), "bsattn_seq_len")
        return Int(n)
    }

    /// Number of leading sequences that hold tokens.
    public var batchSize: Int {
        var n = 0
        while n < Int(desc.max_seqs) && seqLen(n) > 0 { n += 1 }
        return n
    }

    // MARK: KVCache

    public var offset: Int { seqLen(0) }
    public var maxSize: Int? { nil }
    public func innerState() -> [MLXArray] { [] }

    /// Appends keys / values [B, Hkv, L, D] to sequences `seqIds` (default
    /// rows 0..<B); completed blocks get their summaries.
    public func append(keys: MLXArray, values: MLXArray, seqIds: [Int]? = nil) {
        precondition(keys.shape == values.shape && keys.ndim == 4, "keys / values must both be [B, Hkv, L, D]")
        let (kp, vp) = (device.pointer(keys), device.pointer(values))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_append(handle, kp, vp, ids, Int32(keys.dim(0)), Int32(keys.dim(2)), stream),
                    "bsattn_append")
        }
    }

    /// KVCacheSimple.update (KVCache.swift:328-371): append, then every
    /// cached key / value [B, Hkv, offset, D].
    public func update(keys: MLXArray, values: MLXArray) -> (MLXArray, MLXArray) {
        append(keys: keys, values: values)
        return export(rows: keys.dim(0))
    }

    /// Keys and values of rows 0..<n, which must hold equal lengths.
    public func export(rows n: Int) -> (MLXArray, MLXArray) {
        let shape = [n, kvHeads, seqLen(0), headDim]
        let k = device.empty(shape, dtype: dtype)
        let v = device.empty(shape, dtype: dtype)
        if shape[2] > 0 {
            bsCheck(bsattn_export(handle, nil, Int32(n), device.pointer(k), device.pointer(v), stream),
                    "bsattn_export")
        }
        return (k, v)
    }

    /// [keys, values] of the rows that hold tokens (KVCacheSimple.state,
    /// KVCache.swift:373-384); setting it replaces the whole cache.
    public var state: [MLXArray] {
        get {
            let n = batchSize
            if n == 0 { return [] }
            let (k, v) = export(rows: n)
            return [k, v]
        }
        set {
            precondition(newValue.count == 2, "BlockSparseKVCache state must have exactly 2 arrays")
            resetAll()
            if newValue[0].dim(2) > 0 { append(keys: newValue[0], values: newValue[1]) }
        }
    }

    /// [blockSize, topK, sinkBlocks, recentBlocks, offset, kvBits, groupSize].
    public var metaState: [String] {
        get {
            [desc.block_size, desc.top_k, desc.sink_blocks, desc.recent_blocks, Int32(offset),
             desc.kv_bits, desc.group_size].map { String($0) }
        }
        set {
            precondition(newValue.count == 7, "BlockSparseKVCache metaState must have exactly 7 values")
            let want = newValue.map { Int32($0) ?? -1 }
            let have: [Int32] = [desc.block_size, desc.top_k, desc.sink_blocks, desc.recent_blocks,
                                 Int32(offset), desc.kv_bits, desc.group_size]
            precondition(want == have, "metaState \(newValue) does not match this cache (\(have))")
        }
    }

    public var isTrimmable: Bool { true }

    /// Drops the last `n` tokens of every sequence that holds tokens
    /// (KVCacheSimple.trim, KVCache.swift:396-402); returns the number
    /// trimmed from row 0.
    @discardableResult
    public func trim(_ n: Int) -> Int {
        let rows = max(batchSize, 1)
        var trimmed = [Int32](repeating: 0, count: rows)
        bsCheck(bsattn_trim(handle, nil, Int32(rows), Int32(n), &trimmed, stream), "bsattn_trim")
        return Int(trimmed[0])
    }

    /// Empties sequences `seqIds` and returns their pages to the pool.
    public func reset(_ seqIds: [Int]) {
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_reset(handle, ids, Int32(seqIds.count), stream), "bsattn_reset")
        }
    }

    func resetAll() { reset(Array(0 ..< Int(desc.max_seqs))) }

    /// BaseKVCache.makeMask (KVCache.swift:160-174): decode takes no mask,
    /// a multi-token pass the causal one.
    public func makeMask(n: Int, windowSize: Int?, returnArray: Bool)
        -> MLXFast.ScaledDotProductAttentionMaskMode
    {
        if n == 1 { return .none }
        if returnArray || (windowSize != nil && n > windowSize!) {
            return .array(createCausalMask(n: n, offset: offset, windowSize: windowSize))
        }
        return .causal
    }

    /// A deep copy on the same device (KVCacheSimple.copy, KVCache.swift:429-437).
    public func copy() -> any KVCache {
        var h: OpaquePointer? = nil
        bsCheck(bsattn_copy(handle, &h, stream), "bsattn_copy")
        return type(of: self).init(adopting: h!, desc: desc, device: device)
    }

    // MARK: block-sparse attention

    func checkQueries(_ q: MLXArray, multi: Bool = false) {
        precondition(q.ndim == 4 && q.dim(1) == qHeads && q.dim(3) == headDim && q.dtype == dtype,
                     "queries must be [B, Hq, L, D] in the cache's dtype")
        precondition(multi || q.dim(2) == 1, "decode takes one query token per sequence")
    }

    /// Selected blocks [B, Hkv, nselMax] int32 of queries [B, Hq, 1, D]:
    /// ascending block indices, -1 padded.
    public func selectBlocks(queries: MLXArray, seqIds: [Int]? = nil) -> MLXArray {
        checkQueries(queries)
        let idx = device.empty([queries.dim(0), kvHeads, nselMax], dtype: .int32)
        let (qp, ip) = (device.pointer(queries), device.pointer(idx))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_select(handle, qp, ids, Int32(queries.dim(0)), ip.assumingMemoryBound(to: Int32.self),
                                  stream), "bsattn_select")
        }
        return idx
    }

    /// Attention of queries [B, Hq, 1, D] over the blocks of `indices`.
    public func attend(queries: MLXArray, indices: MLXArray, scale: Float, seqIds: [Int]? = nil) -> MLXArray {
        checkQueries(queries)
        precondition(indices.dtype == .int32 && indices.shape == [queries.dim(0), kvHeads, nselMax],
                     "indices must be int32 [B, Hkv, nselMax]")
        let out = device.empty(queries.shape, dtype: dtype)
        let (qp, ip, op) = (device.pointer(queries), device.pointer(indices), device.pointer(out))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_attend(handle, qp, ids, Int32(queries.dim(0)), ip.assumingMemoryBound(to: Int32.self),
                                  scale, op, stream), "bsattn_attend")
        }
        return out
    }

    /// Decode of queries [B, Hq, 1, D] over the cached tokens (scoring,
    /// selection and attention) -> [B, Hq, 1, D].
    public func decode(queries: MLXArray, scale: Float, seqIds: [Int]? = nil) -> MLXArray {
        checkQueries(queries)
        let out = device.empty(queries.shape, dtype: dtype)
        let (qp, op) = (device.pointer(queries), device.pointer(out))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_decode(handle, qp, ids, Int32(queries.dim(0)), scale, op, nil, stream), "bsattn_decode")
        }
        return out
    }

    /// One decode step of attentionWithCacheUpdate (L = 1): appends keys /
    /// values [B, Hkv, 1, D] and decodes queries over the caches that now
    /// hold them, in one call (bit-identical to append then decode).
    public func appendDecode(keys: MLXArray, values: MLXArray, queries: MLXArray, scale: Float,
                             seqIds: [Int]? = nil) -> MLXArray
    {
        checkQueries(queries)
        precondition(keys.shape == values.shape && keys.shape == [queries.dim(0), kvHeads, 1, headDim],
                     "keys / values must both be [B, Hkv, 1, D]")
        let out = device.empty(queries.shape, dtype: dtype)
        let (kp, vp, qp, op) = (device.pointer(keys), device.pointer(values), device.pointer(queries),
                                device.pointer(out))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_append_decode(handle, kp, vp, qp, ids, Int32(queries.dim(0)), scale, op, nil, stream),
                    "bsattn_append_decode")
        }
        return out
    }

    /// The speculative-verify pass (Evaluate.swift:862-870): queries
    /// [B, Hq, L, D] (L <= 16) for the L tokens appended last; query i sees
    /// the first T - L + 1 + i tokens and selects its own blocks there.
    public func decodeMulti(queries: MLXArray, scale: Float, seqIds: [Int]? = nil) -> MLXArray {
        checkQueries(queries, multi: true)
        let out = device.empty(queries.shape, dtype: dtype)
        let (qp, op) = (device.pointer(queries), device.pointer(out))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_decode_multi(handle, qp, ids, Int32(queries.dim(0)), Int32(queries.dim(2)), scale, op,
                                        nil, stream), "bsattn_decode_multi")
        }
        return out
    }

    /// Dense causal attention of the last L tokens (a prefill chunk appended
    /// just before): query i sees tokens [0, T - L + i].
    public func prefill(queries: MLXArray, scale: Float, seqIds: [Int]? = nil) -> MLXArray {
        checkQueries(queries, multi: true)
        let out = device.empty(queries.shape, dtype: dtype)
        let (qp, op) = (device.pointer(queries), device.pointer(out))
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_prefill(handle, qp, ids, Int32(queries.dim(0)), Int32(queries.dim(2)), scale, op,
                                   stream), "bsattn_prefill")
        }
        return out
    }

    /// KVCacheSimple.toQuantized (KVCache.swift:407-427): a cache of the same
    /// geometry holding every sequence as `bits`-bit MLX-affine codes.
    public func toQuantized(groupSize: Int = 64, bits: Int = 4) -> QuantizedBlockSparseKVCache {
        let q = QuantizedBlockSparseKVCache(
            maxSeqs: Int(desc.max_seqs), qHeads: qHeads, kvHeads: kvHeads, headDim: headDim,
            blockSize: blockSize, topK: topK, sinkBlocks: sinkBlocks, recentBlocks: recentBlocks,
            maxBlocksPerSeq: Int(desc.max_blocks_per_seq), numPages: Int(desc.num_pages), bits: bits,
            groupSize: groupSize, device: device)
        for s in 0 ..< Int(desc.max_seqs) where seqLen(s) > 0 {
            let shape = [1, kvHeads, seqLen(s), headDim]
            var k = device.empty(shape, dtype: dtype)
            var v = device.empty(shape, dtype: dtype)
            withSeqIds([s]) { ids in
                bsCheck(bsattn_export(handle, ids, 1, device.pointer(k), device.pointer(v), stream), "bsattn_export")
            }
            if dtype != .float16 {
                k = k.asType(.float16)
                v = v.asType(.float16)
            }
            q.append(keys: k, values: v, seqIds: [s])
        }
        return q
    }
}

/// The quantized form (QuantizedKVCache, KVCache.swift:728-988): keys and
/// values held as MLX-affine codes (LSB-first in uint32 words) with fp16
/// scales and biases per `groupSize` elements; queries and outputs fp16.
/// Decode reads the codes directly (dequantization fused into scoring and
/// attention).
public final class QuantizedBlockSparseKVCache: BlockSparseKVCache, QuantizedKVCacheProtocol {
    public convenience init(
        maxSeqs: Int, qHeads: Int, kvHeads: Int, headDim: Int = 128, blockSize: Int = 64,
        topK: Int = 32, sinkBlocks: Int = 1, recentBlocks: Int = 1, maxBlocksPerSeq: Int,
        numPages: Int = 0, bits: Int = 4, groupSize: Int = 64, device: BlockSparseDevice? = nil
    ) {
        precondition(bits == 4 || bits == 8, "QuantizedBlockSparseKVCache stores 4- or 8-bit codes")
        self.init(maxSeqs: maxSeqs, qHeads: qHeads, kvHeads: kvHeads, headDim: headDim, blockSize: blockSize,
                  dtype: .float16, topK: topK, sinkBlocks: sinkBlocks, recentBlocks: recentBlocks,
                  maxBlocksPerSeq: maxBlocksPerSeq, numPages: numPages, kvBits: bits, groupSize: groupSize,
                  device: device)
    }

    public var groupSize: Int { Int(desc.group_size) }
    public var bits: Int { Int(desc.kv_bits) }
    public var mode: QuantizationMode { .affine }

    /// QuantizedKVCache.update traps (KVCache.swift:891-896).
    public override func update(keys: MLXArray, values: MLXArray) -> (MLXArray, MLXArray) {
        fatalError("`update` was called on a quantized cache. Use `updateQuantized` instead.")
    }

    func quantizedShapes(rows n: Int, tokens t: Int) -> ([Int], [Int]) {
        ([n, kvHeads, t, headDim * bits / 32], [n, kvHeads, t, headDim / groupSize])
    }

    /// ((wq, scales, biases), (wq, scales, biases)) of rows 0..<n.
    func exportQuantized(rows n: Int) -> ((MLXArray, MLXArray, MLXArray?), (MLXArray, MLXArray, MLXArray?)) {
        let (ws, ss) = quantizedShapes(rows: n, tokens: seqLen(0))
        let a = [device.empty(ws, dtype: .uint32), device.empty(ss, dtype: .float16),
                 device.empty(ss, dtype: .float16), device.empty(ws, dtype: .uint32),
                 device.empty(ss, dtype: .float16), device.empty(ss, dtype: .float16)]
        if ws[2] > 0 {
            let p = a.map { device.pointer($0) }
            bsCheck(bsattn_export_quantized(handle, nil, Int32(n), p[0].assumingMemoryBound(to: UInt32.self), p[1],
                                            p[2], p[3].assumingMemoryBound(to: UInt32.self), p[4], p[5], stream),
                    "bsattn_export_quantized")
        }
        return ((a[0], a[1], a[2]), (a[3], a[4], a[5]))
    }

    /// Appends already-quantized tokens in the MLX layout.
    public func appendQuantized(keys: (MLXArray, MLXArray, MLXArray?), values: (MLXArray, MLXArray, MLXArray?),
                                seqIds: [Int]? = nil)
    {
        guard let kb = keys.2, let vb = values.2 else { fatalError("affine codes carry biases") }
        let (ws, ss) = quantizedShapes(rows: keys.0.dim(0), tokens: keys.0.dim(2))
        precondition(keys.0.shape == ws && values.0.shape == ws && keys.1.shape == ss && kb.shape == ss
                     && values.1.shape == ss && vb.shape == ss, "quantized tuples must be MLX-layout \(ws) / \(ss)")
        let p = [keys.0, keys.1, kb, values.0, values.1, vb].map { device.pointer($0) }
        withSeqIds(seqIds) { ids in
            bsCheck(bsattn_append_quantized(handle, p[0].assumingMemoryBound(to: UInt32.self), p[1], p[2],
                                            p[3].assumingMemoryBound(to: UInt32.self), p[4], p[5], ids,
                                            Int32(ws[0]), Int32(ws[2]), stream), "bsattn_append_quantized")
        }
    }

    /// QuantizedKVCache.updateQuantized (KVCache.swift:816-889): quantize and
    /// append fp16 keys / values, return the tuples of every cached token.
    public func updateQuantized(keys: MLXArray, values: MLXArray)
        -> ((MLXArray, MLXArray, MLXArray?), (MLXArray, MLXArray, MLXArray?))
    {
        append(keys: keys, values: values)
        return exportQuantized(rows: keys.dim(0))
    }

    /// QuantizedKVCache.getQuantizedState (KVCache.swift:797-806).
    public func getQuantizedState() -> ((MLXArray, MLXArray, MLXArray?), (MLXArray, MLXArray, MLXArray?))? {
        let n = batchSize
        return n == 0 ? nil : exportQuantized(rows: n)
    }

    /// [kw, ks, kb, vw, vs, vb] (QuantizedKVCache.state, KVCache.swift:906-925).
    public override var state: [MLXArray] {
        get {
            guard let (k, v) = getQuantizedState() else { return [] }
            return [k.0, k.1, k.2!, v.0, v.1, v.2!]
        }
        set {
            precondition(newValue.count == 6, "QuantizedBlockSparseKVCache state must have exactly 6 arrays")
            resetAll()
            if newValue[0].dim(2) > 0 {
                appendQuantized(keys: (newValue[0], newValue[1], newValue[2]),
                                values: (newValue[3], newValue[4], newValue[5]))
            }
        }
    }
}

/// maybeQuantizeKVCache (KVCache.swift:1637-1660) for block-sparse caches:
/// once layer 0 holds more than `quantizedKVStart` tokens, every 16-bit
/// BlockSparseKVCache becomes its quantized form.
public func maybeQuantizeBlockSparseKVCache(
    cache: inout [KVCache], kvBits: Int?, kvGroupSize: Int = 64, quantizedKVStart: Int = 0
) {
    guard let kvBits, !cache.isEmpty, !(cache[0] is QuantizedBlockSparseKVCache),
          cache[0].offset > quantizedKVStart
    else { return }
    for i in 0 ..< cache.count {
        if let c = cache[i] as? BlockSparseKVCache, !(c is QuantizedBlockSparseKVCache) {
            cache[i] = c.toQuantized(groupSize: kvGroupSize, bits: kvBits)
        }
    }
}

/// The block-sparse form of LanguageModel.newCache(parameters:)
/// (LanguageModel.swift:215-230): one cache per layer, layer i with
/// kvHeads[i] KV heads, for up to `maxSeqs` sequences of `maxTokens` tokens.
/// The caches start 16-bit even when parameters.kvBits is set, as in the
/// reference; maybeQuantizeBlockSparseKVCache converts them once
/// quantizedKVStart is passed.  A maxKVSize asks for the reference's
/// RotatingKVCache (a bounded window), which stays on the dense path.
public func newBlockSparseCache(
    kvHeads: [Int], qHeads: Int, parameters: GenerateParameters? = nil, maxSeqs: Int, maxTokens: Int,
    dtype: DType = .bfloat16, blockSize: Int = 64, topK: Int = 32, sinkBlocks: Int = 1,
    recentBlocks: Int = 1, device: BlockSparseDevice? = nil
) -> [KVCache] {
    precondition(parameters?.maxKVSize == nil,
                 "maxKVSize selects RotatingKVCache (KVCache.swift:445-578), which stays on the dense path")
    let blocks = (maxTokens + blockSize - 1) / blockSize
    return kvHeads.map { h in
        BlockSparseKVCache(
            maxSeqs: maxSeqs, qHeads: qHeads, kvHeads: h, blockSize: blockSize, dtype: dtype, topK: topK,
            sinkBlocks: sinkBlocks, recentBlocks: recentBlocks, maxBlocksPerSeq: blocks, device: device)
    }
}
