"""hip_backend: the MI355X (gfx950) MoE backend of llama-rs-metal behind a C ABI.

`api` mirrors metal_backend's Gpu / Batch op surface over libmoe_hip.so;
`synth` builds the seeded synthetic inputs of the benchmark configurations.
"""
from .api import (BF16, F16, F32, PATH_AUTO, PATH_GROUPED, PATH_MFMA, PATH_OPS, SIGNATURES, AllocationError,
                  Batch, BlockWeights, Buffer, Gpu, GpuError, MoeError, PackedWeight, ShapeError, Tensor,
                  UnavailableError, Weight, load_library, pack_size, LIB_PATH)

__all__ = [
    "BF16", "F16", "F32", "PATH_AUTO", "PATH_GROUPED", "PATH_MFMA", "PATH_OPS", "SIGNATURES",
    "AllocationError", "Batch", "BlockWeights", "Buffer", "Gpu", "GpuError", "MoeError",
    "PackedWeight", "ShapeError", "Tensor", "UnavailableError", "Weight", "load_library", "pack_size",
    "LIB_PATH",
]
