"""EdgeForge's quantized decode hot path on MI355X (gfx950).

libedgeforge_hip.so (edgeforge_amd/csrc, C-ABI in include/ef_hip.h) holds the HIP kernels: packed
Q4_0 / Q8_0 GEMV, the sampler, the quantizer and a device decode engine.  ``edgeforge_amd.hip`` is
the Python view of that C-ABI; ``edgeforge_amd.build`` compiles it for gfx950.
"""
from ._lib import HipError, LIB_PATH  # noqa: F401

__version__ = "0.1.0"
