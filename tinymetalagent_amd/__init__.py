"""TinyEngine's attention step on AMD Instinct MI355X (gfx950).

libtinyengine.so (built by tinymetalagent_amd.build) exports the engine's C ABI
(include/tinyengine.h) and the HIP backend slot (include/te_hip_backend.h).
`runtime` is the ctypes binding; `attention` wraps the device-level entry points
for torch tensors.  `attention` imports torch lazily, so the binding itself
works without it.
"""
from .runtime import (
    TE_ABI_VERSION,
    TinyEngineError,
    capabilities,
    check,
    detect_arch,
    device_info,
    hip_available,
    library_path,
    load_library,
    strerror,
)

__all__ = [
    "TE_ABI_VERSION",
    "TinyEngineError",
    "capabilities",
    "check",
    "detect_arch",
    "device_info",
    "hip_available",
    "library_path",
    "load_library",
    "strerror",
]
