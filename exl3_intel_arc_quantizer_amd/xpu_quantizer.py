"""Module-name alias of :mod:`.gpu_quantizer` for callers written against the
reference's ``exl3_quant.xpu_quantizer`` (same public names)."""

from .gpu_quantizer import (  # noqa: F401
    TRACEBACK_MODES,
    BatchEncodingBreakdown,
    GPUTrellisEncoder,
    ScratchArena,
    ScratchArenaLogEntry,
    XPUTrellisEncoder,
    build_quantize_extension,
    get_build_timings,
    verify_tile_encoding_quality,
)
from .memory_policy import MemoryPolicy, MemoryPressureError, MemorySnapshot, capture_snapshot  # noqa: F401
from .reference_encoder import H_INF, EncodingResult  # noqa: F401
from .trellis_format import CB_3INST, CB_MCG, CB_MUL1  # noqa: F401
