"""ctypes view of include/neptune_hip.h and the library locator.

The locator searches where the reference's plugin finder searches
(src/neptune_mlir/plugin.py:28-55), in the same order. Failures of the
C-ABI map onto the exception classes the reference raises for the same
situations: ``NotImplementedError`` for valid requests the backend does not
cover (translators/common.py:187-197) and ``RuntimeError`` for
toolchain/runtime failures (common.py:217-224).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Iterator

LIBRARY_ENV = "NEPTUNE_HIP_LIB"
LIBRARY_FILE = "libneptune_hip.so"

ABI_VERSION = 1

# neptune_status
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_HIP = 3
ERR_NO_DEVICE = 4
ERR_WORKSPACE_TOO_SMALL = 5

# neptune_dtype
DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_FP8_E4M3 = 3

# every entry point the header declares (checked by the CPU test suite)
EXPORTED_SYMBOLS = (
    "neptune_hip_get_backend_info",
    "neptune_last_error",
    "neptune_device_count",
    "neptune_attn_fwd",
    "neptune_decode_workspace_bytes",
    "neptune_decode_splitk",
    "neptune_decode_splitk_noalloc",
    "neptune_decode_paged",
    "neptune_decode_paged_fp8",
    "neptune_kv_quantize_fp8",
    "neptune_selective_scan_fwd",
)


class BackendInfo(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("name", ctypes.c_char_p),
        ("gcn_arch", ctypes.c_char_p),
        ("hip_runtime_version", ctypes.c_int32),
    ]


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("heads_q", ctypes.c_int64),
        ("heads_kv", ctypes.c_int64),
        ("seq_q", ctypes.c_int64),
        ("seq_kv", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 3),
        ("k_stride", ctypes.c_int64 * 3),
        ("v_stride", ctypes.c_int64 * 3),
        ("o_stride", ctypes.c_int64 * 3),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("scale_log2", ctypes.c_float),
        ("pipeline_stages", ctypes.c_int16),
        ("k_dim_order", ctypes.c_int16),
    ]


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("heads_q", ctypes.c_int64),
        ("heads_kv", ctypes.c_int64),
        ("seq_kv", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("num_splits", ctypes.c_int64),
        ("scale_block", ctypes.c_int64),
        ("q_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("scale_log2", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class PagedKvDesc(ctypes.Structure):
    """include/neptune_hip.h: neptune_paged_kv_desc"""

    _fields_ = [
        ("num_pages", ctypes.c_int64),
        ("page_size", ctypes.c_int64),
        ("max_pages", ctypes.c_int64),
        ("k_stride", ctypes.c_int64 * 3),
        ("v_stride", ctypes.c_int64 * 3),
    ]


class ScanDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("dim", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("d_state", ctypes.c_int64),
        ("io_dtype", ctypes.c_int32),
        ("delta_softplus", ctypes.c_int32),
    ]


class NeptuneError(RuntimeError):
    status = -1


class NeptuneInvalidArgument(NeptuneError, ValueError):
    status = ERR_INVALID_ARGUMENT


class NeptuneUnsupported(NeptuneError, NotImplementedError):
    status = ERR_UNSUPPORTED


class NeptuneHipError(NeptuneError):
    status = ERR_HIP


class NeptuneNoDevice(NeptuneError):
    status = ERR_NO_DEVICE


class NeptuneWorkspaceTooSmall(NeptuneError, ValueError):
    status = ERR_WORKSPACE_TOO_SMALL


_STATUS_CLASSES = {
    cls.status: cls
    for cls in (
        NeptuneInvalidArgument,
        NeptuneUnsupported,
        NeptuneHipError,
        NeptuneNoDevice,
        NeptuneWorkspaceTooSmall,
    )
}


def _library_candidates(explicit) -> Iterator[Path]:
    """Files that may hold the backend, the caller's choice first: the
    explicit path, the LIBRARY_ENV variable, the library this package was
    built with, then a development build under the repository or the
    working directory (the reference's plugin search order,
    src/neptune_mlir/plugin.py:28-55)."""
    for given in (explicit, os.environ.get(LIBRARY_ENV)):
        if given:
            yield Path(given).expanduser()
    package = Path(__file__).resolve().parent
    for where in (package / "_native", package.parents[1] / "build", Path.cwd() / "build"):
        yield where / LIBRARY_FILE


def find_library_path(explicit: str | os.PathLike[str] | None = None) -> Path | None:
    """The first existing candidate of ``_library_candidates``, or None."""
    return next((c.resolve() for c in _library_candidates(explicit) if c.is_file()), None)


_LIB: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.neptune_hip_get_backend_info.argtypes = [ctypes.POINTER(BackendInfo)]
    lib.neptune_hip_get_backend_info.restype = i32
    lib.neptune_last_error.argtypes = []
    lib.neptune_last_error.restype = ctypes.c_char_p
    lib.neptune_device_count.argtypes = []
    lib.neptune_device_count.restype = i32
    lib.neptune_attn_fwd.argtypes = [ctypes.POINTER(AttnDesc), vp, vp, vp, vp, vp, vp]
    lib.neptune_attn_fwd.restype = i32
    lib.neptune_decode_workspace_bytes.argtypes = [
        ctypes.POINTER(DecodeDesc),
        ctypes.POINTER(ctypes.c_size_t),
    ]
    lib.neptune_decode_workspace_bytes.restype = i32
    lib.neptune_decode_splitk.argtypes = [
        ctypes.POINTER(DecodeDesc), vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp,
    ]
    lib.neptune_decode_splitk.restype = i32
    lib.neptune_decode_splitk_noalloc.argtypes = [
        ctypes.POINTER(DecodeDesc), vp, vp, vp, vp, vp, vp, vp, vp,
    ]
    lib.neptune_decode_splitk_noalloc.restype = i32
    lib.neptune_decode_paged.argtypes = [
        ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedKvDesc), vp, vp, vp, vp, vp, vp, vp, vp,
        ctypes.c_size_t, vp,
    ]
    lib.neptune_decode_paged.restype = i32
    lib.neptune_decode_paged_fp8.argtypes = [
        ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedKvDesc), vp, vp, vp, vp, vp, vp, vp, vp,
        vp, vp, ctypes.c_size_t, vp,
    ]
    lib.neptune_decode_paged_fp8.restype = i32
    lib.neptune_kv_quantize_fp8.argtypes = [i64, i64, i64, i64, i64, vp, vp, vp, vp]
    lib.neptune_kv_quantize_fp8.restype = i32
    lib.neptune_selective_scan_fwd.argtypes = [
        ctypes.POINTER(ScanDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
    ]
    lib.neptune_selective_scan_fwd.restype = i32


def load_library(explicit: str | os.PathLike[str] | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP backend; raise if it is not built."""
    global _LIB
    if _LIB is not None and explicit is None:
        return _LIB
    path = find_library_path(explicit)
    if path is None:
        raise RuntimeError(
            "libneptune_hip.so not found: build it (python -c 'import __graft_entry__ as g; "
            f"g.build()') or set {LIBRARY_ENV}"
        )
    lib = ctypes.CDLL(str(path))
    _declare(lib)
    info = BackendInfo()
    lib.neptune_hip_get_backend_info(ctypes.byref(info))
    if info.abi_version != ABI_VERSION:
        raise RuntimeError(
            f"{path}: ABI version {info.abi_version}, this package expects {ABI_VERSION}"
        )
    if explicit is None:
        _LIB = lib
    return lib


def check(status: int, lib: ctypes.CDLL | None = None) -> None:
    """Raise the exception class mapped to a non-zero neptune_status."""
    if status == OK:
        return
    lib = lib or load_library()
    msg = (lib.neptune_last_error() or b"").decode(errors="replace")
    cls = _STATUS_CLASSES.get(status, NeptuneError)
    raise cls(msg or f"neptune status {status}")


def backend_info(lib: ctypes.CDLL | None = None) -> dict:
    lib = lib or load_library()
    info = BackendInfo()
    check(lib.neptune_hip_get_backend_info(ctypes.byref(info)), lib)
    return {
        "abi_version": info.abi_version,
        "name": info.name.decode(),
        "gcn_arch": info.gcn_arch.decode(),
        "hip_runtime_version": info.hip_runtime_version,
    }
