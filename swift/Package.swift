// swift-tools-version: 5.9
//
// Swift binding of libbsattn.so, the block-sparse KV cache and decode
// attention for AMD Instinct MI355X.  Two targets:
//
//  - CBSAttn, a system library: the C ABI of include/bsattn.h through a
//    module map, linked against libbsattn.so (put its directory on the linker
//    and loader paths: swift build -Xlinker -L<dir>, LD_LIBRARY_PATH=<dir>).
//  - MLXLMBlockSparse: BlockSparseKVCache, a KVCache of mlx-swift-lm's
//    MLXLMCommon (Libraries/MLXLMCommon/KVCache.swift:38-77), and
//    blockSparseAttentionWithCacheUpdate, the attentionWithCacheUpdate of
//    Libraries/MLXLMCommon/AttentionUtils.swift:37-77 with one more
//    dynamic-type branch.
//
// Inside mlx-swift-lm itself the same two targets go into its Package.swift
// (Package.swift:7-150) beside MLXLMCommon, with "MLXLMCommon" as a target
// dependency instead of the package product.
import PackageDescription

let package = Package(
    name: "mlx-swift-lm-blocksparse",
    products: [
        .library(name: "MLXLMBlockSparse", targets: ["MLXLMBlockSparse"])
    ],
    dependencies: [
        .package(url: "https://github.com/ml-explore/mlx-swift-lm", from: "3.0.0"),
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
