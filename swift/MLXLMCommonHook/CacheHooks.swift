import Foundation
import MLX

// A source file for Libraries/MLXLMCommon: the two extension points through
// which a KV cache defined outside MLXLMCommon (here the block-sparse cache
// of the MLXLMBlockSparse target, which depends on MLXLMCommon) takes part in
// the entry point models call and in prompt-cache loading, without
// MLXLMCommon depending on it.  Two insertions use them:
//
//  - attentionWithCacheUpdate (AttentionUtils.swift:37-77), after the
//    `guard let cache` (:45-53) and before the quantized branch (:54):
//
//        if let attending = cache as? AttendingKVCache {
//            return attending.updateAndAttend(
//                queries: queries, keys: keys, values: values, scale: scale, mask: mask)
//        }
//
//  - loadPromptCache (KVCache.swift:1307-1388), the `default:` case of the
//    class switch (:1380-1381):
//
//        default:
//            guard let made = try PromptCacheClasses.make(
//                className, metaState: i < cacheInfo.count ? cacheInfo[i] : [],
//                state: cacheData[i])
//            else { throw KVCacheError(message: "Unknown cache class: \(className)") }
//            cache = made

/// A KV cache that computes its own attention.
///
/// attentionWithCacheUpdate hands such a cache the new keys / values and the
/// queries and returns what it returns, without calling `update`.  The check
/// comes before the quantized branch, so a cache may conform to this and to
/// QuantizedKVCacheProtocol at once and still attend itself.  Models keep
/// calling attentionWithCacheUpdate unchanged.
public protocol AttendingKVCache: KVCache {
    /// Appends keys / values [B, Hkv, L, D] and returns the attention of
    /// queries [B, Hq, L, D] over the cache that now holds them, in the
    /// queries' dtype; `mask` as attentionWithCacheUpdate receives it.
    func updateAndAttend(
        queries: MLXArray, keys: MLXArray, values: MLXArray, scale: Float,
        mask: MLXFast.ScaledDotProductAttentionMaskMode
    ) -> MLXArray
}

/// Cache classes that live outside MLXLMCommon, by the class name their
/// prompt-cache files carry.  loadPromptCache asks here for a class name its
/// own switch does not know, then sets the cache's `state` and `metaState`
/// from the file as it does for its own classes.
public enum PromptCacheClasses {
    /// Builds the empty cache of a file entry from its metaState and state
    /// (the arrays are what `state` will be set to; a maker reads shapes and
    /// dtypes from them, not contents).
    public typealias Maker = (_ metaState: [String], _ state: [MLXArray]) throws -> KVCache

    private final class Registry {
        let lock = NSLock()
        var makers: [String: Maker] = [:]
    }

    private static let registry = Registry()

    /// Makes `className` loadable; a later registration of the same name
    /// replaces the earlier one.
    public static func register(_ className: String, _ make: @escaping Maker) {
        registry.lock.lock()
        defer { registry.lock.unlock() }
        registry.makers[className] = make
    }

    /// The cache for a file entry of `className`, or nil when no maker is
    /// registered for it.
    public static func make(_ className: String, metaState: [String], state: [MLXArray]) throws
        -> KVCache?
    {
        registry.lock.lock()
        let make = registry.makers[className]
        registry.lock.unlock()
        return try make?(metaState, state)
    }
}
