"""MI355X (gfx950) implementation of PromptMoGe's sparse 3-D refiner step.

    promptmoge_amd.ops        torch wrappers of the C ABI (include/pmg.h): voxelise, neighbour maps, convolutions,
                              row ops, metric fit
    promptmoge_amd.refiner    RefinerStep, the fused step (one HIP graph per step, no host round trip)
    promptmoge_amd.flex_gemm  drop-in for the reference's `flex_gemm` plugin package
    promptmoge_amd.spec       seeded synthetic scenes and weights of the benchmark configurations
"""
__version__ = "0.1.0"
