// swift-tools-version: 5.9
// The Linux C target of the MI355X linear path and the operator layer over it: a system
// library module for libmingtts_hip.so and a library target holding the Linux Encoder.
// Build (where a Swift toolchain is installed) with
//   swift build -Xcc -I../include -Xlinker -L../ming-tts_amd/csrc
import PackageDescription

let package = Package(
    name: "MingTTSHIP",
    products: [
        .library(name: "MingTTSHIP", targets: ["MingTTSHIP"]),
    ],
    targets: [
        .systemLibrary(name: "CMingHIP", path: "Sources/CMingHIP"),
        .target(name: "MingTTSHIP", dependencies: ["CMingHIP"], path: "Sources/MingTTSHIP"),
    ]
)
