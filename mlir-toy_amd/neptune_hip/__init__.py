"""neptune_hip — MI355X (gfx950) backend for Neptune's HTile hot path.

The compute lives in libneptune_hip.so (hand-written HIP kernels behind the
C-ABI of include/neptune_hip.h); this package only locates that library,
passes device pointers and streams to it, and offers the HTile front end
(``translate_file``) that binds an HTile attention tile program to it.
"""

from ._abi import (  # noqa: F401
    LIBRARY_ENV,
    NeptuneError,
    NeptuneHipError,
    NeptuneInvalidArgument,
    NeptuneNoDevice,
    NeptuneUnsupported,
    NeptuneWorkspaceTooSmall,
    backend_info,
    find_library_path,
    load_library,
)

__all__ = [
    "LIBRARY_ENV",
    "NeptuneError",
    "NeptuneHipError",
    "NeptuneInvalidArgument",
    "NeptuneNoDevice",
    "NeptuneUnsupported",
    "NeptuneWorkspaceTooSmall",
    "backend_info",
    "find_library_path",
    "load_library",
]
