// swift-tools-version: 5.9
//
// Swift binding of libbsattn.so, the block-sparse KV cache and decode
// attention for AMD Instinct MI355X.  Two targets:
//
//  - CBSAttn, a system library: the C ABI of include/bsattn.h through a
//    module map, linked against libbsattn.so (put its directory on the linker
//    and loader paths: swift build -Xlinker -L<dir>, LD_LIBRARY_PATH=<dir>).
//  - MLXLMBlockSparse: BlockSparseKVCache, a KVCache of mlx-swift-lm's
//    MLXLMCommon (Libraries/MLXLMCommon/KVCache.swift:38-77) that conforms to
//    AttendingKVCache, so the attentionWithCacheUpdate models call
//    (Libraries/MLXLMCommon/AttentionUtils.swift:37-77) routes to it, and
//    registers its class with PromptCacheClasses for loadPromptCache.
//
// AttendingKVCache and PromptCacheClasses are declared by
// MLXLMCommonHook/CacheHooks.swift, a file added to Libraries/MLXLMCommon
// together with the two short insertions its header comment gives (one
// branch in attentionWithCacheUpdate, one `default:` case in
// loadPromptCache).  The dependency below is a checkout of mlx-swift-lm with
// that change applied.  Inside mlx-swift-lm itself the two targets go into
// its Package.swift (Package.swift:7-150) beside MLXLMCommon, with
// "MLXLMCommon" as a target dependency instead of the package product.
import PackageDescription

let package = Package(
    name: "mlx-swift-lm-blocksparse",
    products: [
        .library(name: "MLXLMBlockSparse", targets: ["MLXLMBlockSparse"])
    ],
    dependencies: [
        .package(path: "../mlx-swift-lm"),  // with MLXLMCommonHook/CacheHooks.swift applied
        .package(url: "https://github.com/ml-explore/mlx-swift", .upToNextMinor(from: "0.31.3")),
    ],
    targets: [
        .systemLibrary(name: "CBSAttn", path: "Sources/CBSAttn"),
        .target(
            name: "MLXLMBlockSparse",
            dependencies: [
                "CBSAttn",
                .product(name: "MLXLMCommon", package: "mlx-swift-lm"),
                .product(name: "MLX", package: "mlx-swift"),
            ],
            path: "Sources/MLXLMBlockSparse"
        ),
    ]
)
