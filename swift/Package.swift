// swift-tools-version:5.9
// The Swift side of the drop-in: the reference's FlashVSRMLX target depends on FlashVSRLCSA, which calls
// libfvsr_lcsa.so (built by mlx-flashvsr-swift_amd/build_lib.py) through the C module CFlashVSRLCSA.
// Build with: swift build -Xlinker -L<repo>/mlx-flashvsr-swift_amd/lib
import PackageDescription

let package = Package(
    name: "FlashVSRLCSA",
    products: [.library(name: "FlashVSRLCSA", targets: ["FlashVSRLCSA"])],
    targets: [
        .systemLibrary(name: "CFlashVSRLCSA", path: "Sources/CFlashVSRLCSA"),
        .target(name: "FlashVSRLCSA", dependencies: ["CFlashVSRLCSA"], path: "Sources/FlashVSRLCSA",
                linkerSettings: [.linkedLibrary("fvsr_lcsa")]),
    ]
)
