"""neptune_mlir.backends.hip: the reference-side binding of libneptune_hip.so.

A maintainer adds this module to the reference as
src/neptune_mlir/backends/hip.py. `flash_attention_htile(q, k, v, out)` then
takes the place of the generated kernel that the reference's functional test
launches as `flash_attention_htile[(32, 32, 1)](q, k, v, out)`
(tests/test_translators.py:184-194; golden tests/golden/flash_attention_triton.py:4-5):
same arguments, caller-allocated `out`, work enqueued on torch's current
stream. The library is found as the reference finds its own plugin
(src/neptune_mlir/plugin.py:28-55): an explicit path, else the
NEPTUNE_HIP_LIB environment variable.

Errors follow the reference's translators (translators/common.py:187-197,
217-224): a request the backend does not cover raises NotImplementedError,
any other failure RuntimeError, with the library's message.
"""

import ctypes
import os

import torch

NEPTUNE_HIP_ENV = "NEPTUNE_HIP_LIB"

# neptune_dtype and neptune_status of include/neptune_hip.h
F32, F16, BF16 = 0, 1, 2
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


class AttnDesc(ctypes.Structure):
    """neptune_attn_desc (include/neptune_hip.h)."""
    _fields_ = [("batch", ctypes.c_int64), ("heads_q", ctypes.c_int64),
                ("heads_kv", ctypes.c_int64), ("seq_q", ctypes.c_int64),
                ("seq_kv", ctypes.c_int64), ("head_dim", ctypes.c_int64),
                ("q_stride", ctypes.c_int64 * 3), ("k_stride", ctypes.c_int64 * 3),
                ("v_stride", ctypes.c_int64 * 3), ("o_stride", ctypes.c_int64 * 3),
                ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32),
                ("scale_log2", ctypes.c_float), ("pipeline_stages", ctypes.c_int16),
                ("k_dim_order", ctypes.c_int16)]


_lib = None


def load(path=None):
    """Open the backend (an explicit path, else $NEPTUNE_HIP_LIB) and declare
    the entry point this module calls."""
    global _lib
    if path is None:
        path = os.environ.get(NEPTUNE_HIP_ENV)
        if not path:
            raise RuntimeError(f"set {NEPTUNE_HIP_ENV} to the path of libneptune_hip.so")
    lib = ctypes.CDLL(str(path))
    lib.neptune_attn_fwd.argtypes = [ctypes.POINTER(AttnDesc)] + [ctypes.c_void_p] * 6
    lib.neptune_attn_fwd.restype = ctypes.c_int32
    lib.neptune_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def _dtype(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise NotImplementedError(f"flash_attention_htile: no kernel for {t.dtype}") from None


def _check(q, k, v, out):
    """What the generated kernel assumes of its arguments, checked before any
    call: one device (the GPU whenever there is one), one dtype, agreeing
    [batch, heads, seq, head_dim] shapes, and contiguous storage (the zero
    strides the descriptor carries)."""
    ts = (q, k, v, out)
    if len({t.device for t in ts}) != 1:
        raise RuntimeError("flash_attention_htile: q, k, v and out must be on one device")
    if not q.is_cuda and torch.cuda.is_available():
        raise RuntimeError("flash_attention_htile: q, k, v and out must be GPU tensors")
    if any(t.dtype != q.dtype for t in ts):
        raise RuntimeError("flash_attention_htile: q, k, v and out must share one dtype")
    if (q.dim() != 4 or k.dim() != 4 or tuple(v.shape) != tuple(k.shape)
            or tuple(out.shape) != tuple(q.shape)
            or (k.shape[0], k.shape[3]) != (q.shape[0], q.shape[3])):
        raise RuntimeError(f"flash_attention_htile: shapes q {tuple(q.shape)} k {tuple(k.shape)} "
                           f"v {tuple(v.shape)} out {tuple(out.shape)} do not agree")
    if not all(t.is_contiguous() for t in ts):
        raise NotImplementedError("flash_attention_htile: contiguous tensors only")


def flash_attention_htile(q, k, v, out):
    """Same arguments and effect as the generated kernel: out <- attention(q,
    k, v) over contiguous [batch, heads, seq, head_dim] tensors, scaled by
    log2(e)/sqrt(head_dim) in the exp2 domain (the HTile constant)."""
    _check(q, k, v, out)
    lib = _lib if _lib is not None else load()
    d = AttnDesc()
    d.batch, d.heads_q, d.seq_q, d.head_dim = q.shape
    d.heads_kv, d.seq_kv = k.shape[1], k.shape[2]
    d.dtype = _dtype(q)
    # zero strides = contiguous; scale_log2 = 0 -> log2(e)/sqrt(D)
    stream = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else None
    st = lib.neptune_attn_fwd(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                              out.data_ptr(), None, stream)
    if st == OK:
        return
    msg = lib.neptune_last_error().decode()
    if st == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
