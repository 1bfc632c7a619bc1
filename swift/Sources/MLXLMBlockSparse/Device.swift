import CBSAttn
import MLX

/// How MLX arrays reach the GPU that libbsattn runs on.
///
/// libbsattn reads and writes device memory and orders its work on a HIP
/// stream.  An MLX backend for MI355X keeps array storage in HBM; this
/// protocol is the three things the cache needs from it.  Arrays passed in are
/// row-major and contiguous; arrays handed back are written by kernels that
/// run on `stream` and are ready once the backend's next operation on that
/// stream runs.
public protocol BlockSparseDevice: AnyObject {
    /// Device address of the evaluated, contiguous storage of `array`.
    func pointer(_ array: MLXArray) -> UnsafeMutableRawPointer
    /// A new device array of `shape` and `dtype`; its contents are undefined
    /// until a library call writes them.
    func empty(_ shape: [Int], dtype: DType) -> MLXArray
    /// The HIP stream (`hipStream_t`) the backend orders array work on; nil
    /// is the null stream.
    var stream: UnsafeMutableRawPointer? { get }
    /// HIP device ordinal of that stream.
    var ordinal: Int32 { get }
}

/// Process-wide defaults of the binding.
public enum BlockSparse {
    /// The device new caches use unless one is given to their initializer.
    public static var device: BlockSparseDevice?
}

/// Traps with the library's message when a call fails, as the reference's
/// caches trap on misuse (`fatalError` / `precondition` in KVCache.swift).
@inline(__always)
func bsCheck(_ rc: Int32, _ what: StaticString) {
    if rc != 0 {
        let msg = bsattn_last_error().map { String(cString: $0) } ?? ""
        fatalError("\(what) failed (\(rc)): \(msg)")
    }
}

/// Calls `body` with a pointer to `ids` as int32, or nil for rows 0..<n.
func withSeqIds<R>(_ ids: [Int]?, _ body: (UnsafePointer<Int32>?) -> R) -> R {
    guard let ids else { return body(nil) }
    let ids32 = ids.map { Int32($0) }
    return ids32.withUnsafeBufferPointer { body($0.baseAddress) }
}
