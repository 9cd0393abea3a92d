"""MI355X (gfx950) backend for DiskMule's quantized-matrix path.

The compute lives in ``libdmhip.so`` (hand-written HIP for gfx950 behind the
C ABI of ``include/dmhip.h``).  :mod:`diskmule_amd.hip` binds that ABI with
ctypes and mirrors the method names of the reference's ``MetalContext``
(``src/metal.rs``) and ``ExpertCache`` (``src/expert.rs``).

There is no CPU fallback: when the library is missing or no GPU is present,
every entry point raises.
"""
from .hip import (  # noqa: F401
    HipContext,
    HipError,
    OwnedBuffer,
    MappedBuffer,
    ExpertCache,
    ExpertLayerLayout,
    KvLayer,
    BackendSelection,
    library_path,
    load_library,
    EXPORTED_SYMBOLS,
)
