// swift-tools-version:5.9
// SwiftPM package that puts libanima_hip behind the AnimaXS executor surfaces:
// AttentionExecutor (AnimaXS/Runtime/Metal/AttentionExecutor.swift:77-848),
// LinearExecutor (LinearExecutor.swift:43-459) and QuantDecoders
// (Runtime/Animapk/QuantDecoders.swift:17-164).  CAnimaHIP is a system-library
// target whose module map names include/anima_hip.h of this repository itself, so
// Swift imports exactly the declarations the C layout test compiles.
//
// Build the library first (python -m animaxs_amd.build); set ANIMA_HIP_LIB_DIR to
// the directory holding libanima_hip.so (default: the animaxs_amd package directory
// next to this file).
import Foundation
import PackageDescription

let here = URL(fileURLWithPath: #filePath).deletingLastPathComponent()
let libDir = ProcessInfo.processInfo.environment["ANIMA_HIP_LIB_DIR"]
    ?? here.deletingLastPathComponent().path

let package = Package(
    name: "AnimaHIP",
    products: [
        .library(name: "AnimaHIP", targets: ["AnimaHIP"]),
    ],
    targets: [
        .systemLibrary(name: "CAnimaHIP", path: "Sources/CAnimaHIP"),
        .target(
            name: "AnimaHIP",
            dependencies: ["CAnimaHIP"],
            path: "Sources/AnimaHIP",
            linkerSettings: [
                .linkedLibrary("anima_hip"),
                .unsafeFlags(["-L\(libDir)", "-Xlinker", "-rpath", "-Xlinker", libDir]),
            ]),
    ]
)
