"""FanarVSE throughput-mode search path, MI355X-native (gfx950 HIP kernels behind a C ABI).

Modules:
    enginei8  EngineI8 (search entry point, graph capture, fallback)
    index     index build (cells, means, PCA basis, int8 codes, static work list)
    s2lut     uniform tiered refinement code, LUT stage-2 entry points
    datagen   synthetic base/query generator of the benchmark configurations
    metrics   recall and read statistics
    _lib      ctypes binding of libfvs.so (include/fvs.h)
"""
from . import datagen, metrics  # noqa: F401
