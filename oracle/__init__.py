"""ctypes wrapper of the CPU oracle (oracle/neptune_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as the product path. Arrays are numpy arrays holding the
storage bits: float32 for F32, float16 for F16, uint16 bit patterns for BF16
and uint8 codes for FP8_E4M3.

The descriptor structs are declared here independently of the product
package; tests/test_abi.py checks that both declarations agree with each
other field by field.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# NEPTUNE_ORACLE_LIB selects another build of the same source (the
# host-sanitizer build of oracle/Makefile's `sanitize` target)
LIB_PATH = Path(os.environ.get("NEPTUNE_ORACLE_LIB") or HERE / "libneptune_oracle.so")

F32, F16, BF16, FP8 = 0, 1, 2, 3
_NP_STORAGE = {F32: np.float32, F16: np.float16, BF16: np.uint16, FP8: np.uint8}


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


_LIB = None


def build() -> Path:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.neptune_cpu_f32_to_bf16.argtypes = [ctypes.c_float]
        L.neptune_cpu_f32_to_bf16.restype = ctypes.c_uint16
        L.neptune_cpu_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.neptune_cpu_bf16_to_f32.restype = ctypes.c_float
        L.neptune_cpu_f32_to_f16.argtypes = [ctypes.c_float]
        L.neptune_cpu_f32_to_f16.restype = ctypes.c_uint16
        L.neptune_cpu_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.neptune_cpu_f16_to_f32.restype = ctypes.c_float
        L.neptune_cpu_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.neptune_cpu_f32_to_e4m3.restype = ctypes.c_uint8
        L.neptune_cpu_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.neptune_cpu_e4m3_to_f32.restype = ctypes.c_float
        L.neptune_cpu_convert_f32.argtypes = [vp, vp, i64, i32]
        L.neptune_cpu_convert_f32.restype = None
        L.neptune_cpu_to_f32.argtypes = [vp, vp, i64, i32]
        L.neptune_cpu_to_f32.restype = None
        L.neptune_cpu_num_threads.argtypes = []
        L.neptune_cpu_num_threads.restype = i32
        L.neptune_cpu_attn_fwd.argtypes = [ctypes.POINTER(AttnDesc), vp, vp, vp, vp, vp]
        L.neptune_cpu_attn_fwd.restype = i32
        L.neptune_cpu_attn_exact.argtypes = [ctypes.POINTER(AttnDesc), vp, vp, vp, vp, vp]
        L.neptune_cpu_attn_exact.restype = i32
        L.neptune_cpu_decode_splitk.argtypes = [
            ctypes.POINTER(DecodeDesc), vp, vp, vp, vp, vp, vp, vp, vp,
        ]
        L.neptune_cpu_decode_splitk.restype = i32
        L.neptune_cpu_decode_paged.argtypes = [
            ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedKvDesc), vp, vp, vp, vp, vp, vp, vp,
        ]
        L.neptune_cpu_decode_paged.restype = i32
        L.neptune_cpu_decode_paged_fp8.argtypes = [
            ctypes.POINTER(DecodeDesc), ctypes.POINTER(PagedKvDesc), vp, vp, vp, vp, vp, vp, vp,
            vp, vp,
        ]
        L.neptune_cpu_decode_paged_fp8.restype = i32
        L.neptune_cpu_decode_layout.argtypes = [
            ctypes.POINTER(DecodeDesc), ctypes.POINTER(i64), ctypes.POINTER(i64),
        ]
        L.neptune_cpu_decode_layout.restype = i32
        L.neptune_cpu_kv_quantize_fp8.argtypes = [i64, i64, i64, i64, i64, vp, vp, vp]
        L.neptune_cpu_kv_quantize_fp8.restype = i32
        L.neptune_cpu_selective_scan_fwd.argtypes = [
            ctypes.POINTER(ScanDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
        ]
        L.neptune_cpu_selective_scan_fwd.restype = i32
        _LIB = L
    return _LIB


def num_threads() -> int:
    return int(lib().neptune_cpu_num_threads())


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(status: int, what: str) -> None:
    if status != 0:
        raise ValueError(f"oracle {what}: status {status}")


# ----------------------------------------------------------------- codecs


def encode(x: np.ndarray, dtype: int) -> np.ndarray:
    """float32 -> storage bits of dtype (RNE; E4M3 saturates)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=_NP_STORAGE[dtype])
    lib().neptune_cpu_convert_f32(_ptr(x), _ptr(out), x.size, dtype)
    return out


def decode(bits: np.ndarray, dtype: int) -> np.ndarray:
    """storage bits of dtype -> float32."""
    bits = np.ascontiguousarray(bits, dtype=_NP_STORAGE[dtype])
    out = np.empty(bits.shape, dtype=np.float32)
    lib().neptune_cpu_to_f32(_ptr(bits), _ptr(out), bits.size, dtype)
    return out


# -------------------------------------------------------------- attention


def _attn_desc(q, k, dtype, causal, scale_log2, k_dim_order=0) -> AttnDesc:
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], (k.shape[3] if k_dim_order else k.shape[2])
    d = AttnDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_q, d.seq_kv, d.head_dim = B, Hq, Hk, Sq, Sk, D
    d.dtype, d.causal, d.scale_log2 = dtype, 1 if causal else 0, scale_log2
    d.k_dim_order = k_dim_order
    return d


def attn_fwd(q, k, v, dtype: int, causal: bool = False, scale_log2: float = 0.0,
             k_dim_order: int = 0):
    """HTile-policy attention. Returns (o storage bits, lse float32).
    k_dim_order=1: k is given [B, Hk, D, Sk]."""
    q, k, v = (np.ascontiguousarray(t) for t in (q, k, v))
    d = _attn_desc(q, k, dtype, causal, scale_log2, k_dim_order)
    o = np.empty(q.shape, dtype=_NP_STORAGE[dtype])
    lse = np.empty(q.shape[:3], dtype=np.float32)
    _check(lib().neptune_cpu_attn_fwd(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(o),
                                      _ptr(lse)), "attn_fwd")
    return o, lse


def attn_exact(q, k, v, dtype: int, causal: bool = False, scale_log2: float = 0.0,
               k_dim_order: int = 0):
    """fp64 closed form. Returns (o float64, lse float64)."""
    q, k, v = (np.ascontiguousarray(t) for t in (q, k, v))
    d = _attn_desc(q, k, dtype, causal, scale_log2, k_dim_order)
    o = np.empty(q.shape, dtype=np.float64)
    lse = np.empty(q.shape[:3], dtype=np.float64)
    _check(lib().neptune_cpu_attn_exact(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v), _ptr(o),
                                        _ptr(lse)), "attn_exact")
    return o, lse


# ------------------------------------------------------------------ decode


def _decode_desc(q, k, kv_dtype, num_splits, scale_block, scale_log2) -> DecodeDesc:
    B, Hq, D = q.shape
    _, Hk, L, _ = k.shape
    d = DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = B, Hq, Hk, L, D
    d.num_splits, d.scale_block = num_splits, scale_block
    d.q_dtype, d.kv_dtype, d.scale_log2 = BF16, kv_dtype, scale_log2
    return d


def decode_layout(batch, heads_kv, seq_kv, num_splits=0):
    d = DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = batch, heads_kv, heads_kv, seq_kv, 128
    d.num_splits = num_splits
    s, c = ctypes.c_int64(), ctypes.c_int64()
    _check(lib().neptune_cpu_decode_layout(ctypes.byref(d), ctypes.byref(s), ctypes.byref(c)),
           "decode_layout")
    return s.value, c.value


def decode_splitk(q, k, v, kv_dtype: int = BF16, k_scale=None, v_scale=None,
                  num_splits: int = 0, scale_block: int = 64, scale_log2: float = 0.0):
    """Split-K decode. q [B,Hq,D] bf16 bits. Returns (o bits, lse, partials)."""
    q, k, v = (np.ascontiguousarray(t) for t in (q, k, v))
    if k_scale is not None:
        k_scale = np.ascontiguousarray(k_scale, dtype=np.float32)
        v_scale = np.ascontiguousarray(v_scale, dtype=np.float32)
    d = _decode_desc(q, k, kv_dtype, num_splits, scale_block, scale_log2)
    S, _ = decode_layout(q.shape[0], k.shape[1], k.shape[2], num_splits)
    o = np.empty(q.shape, dtype=np.uint16)
    lse = np.empty(q.shape[:2], dtype=np.float32)
    parts = np.empty(q.shape[:2] + (S, q.shape[2] + 2), dtype=np.float32)
    _check(lib().neptune_cpu_decode_splitk(ctypes.byref(d), _ptr(q), _ptr(k), _ptr(v),
                                           _ptr(k_scale), _ptr(v_scale), _ptr(o), _ptr(lse),
                                           _ptr(parts)), "decode_splitk")
    return o, lse, parts


def decode_paged(q, k_pool, v_pool, block_table, seq_lens, max_seq_len=None,
                 num_splits: int = 0, scale_log2: float = 0.0, k_scales=None, v_scales=None):
    """Split-K decode over a paged pool. q [B,Hq,D] bf16 bits; k_pool /
    v_pool viewed as [pages, Hk, page_size, D] (any element strides with D
    contiguous; read in place): bf16 bits (uint16), or E4M3 codes (uint8)
    with k_scales / v_scales float32 [pages, Hk], one scale per (page, kv
    head); block_table [B, max_pages] and seq_lens [B] int32. Returns
    (o bits, lse)."""
    q = np.ascontiguousarray(q)
    block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
    fp8 = k_pool.dtype == np.uint8
    esize = 1 if fp8 else 2
    for pool in (k_pool, v_pool):
        if (pool.dtype != k_pool.dtype or pool.dtype not in (np.uint16, np.uint8)
                or pool.ndim != 4 or pool.strides[3] != esize):
            raise ValueError("pools must be uint16 (bf16) or uint8 (E4M3) "
                             "[pages, Hk, page_size, D] with D contiguous")
    npages, Hk, ps, D = k_pool.shape
    if fp8:
        if k_scales is None or v_scales is None:
            raise ValueError("fp8 pools need k_scales and v_scales [pages, Hk]")
        k_scales = np.ascontiguousarray(k_scales, dtype=np.float32)
        v_scales = np.ascontiguousarray(v_scales, dtype=np.float32)
        if k_scales.shape != (npages, Hk) or v_scales.shape != (npages, Hk):
            raise ValueError("k_scales / v_scales must be [pages, Hk]")
    L = int(max_seq_len) if max_seq_len is not None else block_table.shape[1] * ps
    d = DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = q.shape[0], q.shape[1], Hk, L, D
    d.num_splits, d.scale_block = num_splits, (ps if fp8 else 64)
    d.q_dtype, d.kv_dtype, d.scale_log2 = BF16, (FP8 if fp8 else BF16), scale_log2
    pk = PagedKvDesc()
    pk.num_pages, pk.page_size, pk.max_pages = npages, ps, block_table.shape[1]
    pk.k_stride[:] = tuple(x // esize for x in k_pool.strides[:3])
    pk.v_stride[:] = tuple(x // esize for x in v_pool.strides[:3])
    o = np.empty(q.shape, dtype=np.uint16)
    lse = np.empty(q.shape[:2], dtype=np.float32)
    if fp8:
        st = lib().neptune_cpu_decode_paged_fp8(
            ctypes.byref(d), ctypes.byref(pk), _ptr(q), k_pool.ctypes.data, v_pool.ctypes.data,
            _ptr(k_scales), _ptr(v_scales), _ptr(block_table), _ptr(seq_lens), _ptr(o), _ptr(lse))
    else:
        st = lib().neptune_cpu_decode_paged(
            ctypes.byref(d), ctypes.byref(pk), _ptr(q), k_pool.ctypes.data, v_pool.ctypes.data,
            _ptr(block_table), _ptr(seq_lens), _ptr(o), _ptr(lse))
    _check(st, "decode_paged")
    return o, lse


def kv_quantize_fp8(src_bits: np.ndarray, scale_block: int = 64):
    """bf16 bits [B,Hk,L,D] -> (codes uint8, scales float32 [B,Hk,nblocks])."""
    src_bits = np.ascontiguousarray(src_bits, dtype=np.uint16)
    B, Hk, L, D = src_bits.shape
    nsb = -(-L // scale_block)
    codes = np.empty(src_bits.shape, dtype=np.uint8)
    scales = np.empty((B, Hk, nsb), dtype=np.float32)
    _check(lib().neptune_cpu_kv_quantize_fp8(B, Hk, L, D, scale_block, _ptr(src_bits),
                                             _ptr(codes), _ptr(scales)), "kv_quantize")
    return codes, scales


# -------------------------------------------------------------------- scan


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, softplus=True):
    """fp64 sequential scan. u/delta/z [b,d,L], B/C [b,n,L] bf16 bits; A [d,n],
    D, delta_bias [d] float32. Returns (y bf16 bits, y float64)."""
    u, delta, B, C = (np.ascontiguousarray(t, dtype=np.uint16) for t in (u, delta, B, C))
    z = None if z is None else np.ascontiguousarray(z, dtype=np.uint16)
    A = np.ascontiguousarray(A, dtype=np.float32)
    D = None if D is None else np.ascontiguousarray(D, dtype=np.float32)
    delta_bias = None if delta_bias is None else np.ascontiguousarray(delta_bias, dtype=np.float32)
    b, dm, L = u.shape
    d = ScanDesc(b, dm, L, A.shape[1], BF16, 1 if softplus else 0)
    y = np.empty(u.shape, dtype=np.uint16)
    y64 = np.empty(u.shape, dtype=np.float64)
    _check(lib().neptune_cpu_selective_scan_fwd(ctypes.byref(d), _ptr(u), _ptr(delta), _ptr(A),
                                                _ptr(B), _ptr(C), _ptr(D), _ptr(z),
                                                _ptr(delta_bias), _ptr(y), _ptr(y64)),
           "selective_scan")
    return y, y64
