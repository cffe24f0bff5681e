"""MI355X-native EXL3 trellis tile encoder (gfx950 HIP kernels behind the
reference encoder API of alpha2beta/EXL3_Intel_Arc_quantizer).

Importing the package does not touch the GPU; the native library is loaded on
first use (``build_quantize_extension``) and must have been built with
``python -m exl3_intel_arc_quantizer_amd.build``.
"""

from .memory_policy import MemoryPolicy, MemoryPressureError, MemorySnapshot, capture_snapshot
from .reference_encoder import H_INF, EncodingResult
from .scratch_estimator import ScratchAllocation, ScratchEstimator
from .trellis_format import CB_3INST, CB_MCG, CB_MUL1, tensor_core_perm, tensor_core_perm_inv

__all__ = [
    "CB_3INST", "CB_MCG", "CB_MUL1", "H_INF", "EncodingResult", "MemoryPolicy",
    "MemoryPressureError", "MemorySnapshot", "ScratchAllocation", "ScratchEstimator",
    "capture_snapshot", "tensor_core_perm", "tensor_core_perm_inv",
    "XPUTrellisEncoder", "GPUTrellisEncoder", "ScratchArena", "build_quantize_extension",
]


def __getattr__(name):
    # Lazy: the encoder module imports torch only when used.
    if name in ("XPUTrellisEncoder", "GPUTrellisEncoder", "ScratchArena",
                "build_quantize_extension", "BatchEncodingBreakdown",
                "verify_tile_encoding_quality"):
        from . import gpu_quantizer
        return getattr(gpu_quantizer, name)
    raise AttributeError(name)
