"""CPU tests of the drop-in boundary (include/neptune_hip.h).

No kernel runs here: every check is one the library answers on the host
before any HIP call (symbol export, descriptor layout, the backend info
record, argument validation and its status codes, the no-device path).
The classes of failure mirror the reference's: invalid input and
unsupported requests (NotImplementedError, translators/common.py:187-197),
runtime failures (RuntimeError, common.py:217-224).
"""

import ctypes
import re
import subprocess
import threading
from pathlib import Path

import pytest

import oracle
from neptune_hip import _abi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "neptune_hip.h"

# Plausible-looking, 16-byte aligned device addresses. They are only ever
# passed to calls that must fail validation (or find no device) before any
# HIP work is enqueued; test_no_device_path runs only where no device exists.
FAKE = 0x10000


@pytest.fixture(scope="module")
def lib():
    return _abi.load_library()


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"NEPTUNE_API[^;{]*?\b(neptune_\w+)\s*\(", text, re.S)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 8
    assert sorted(_abi.EXPORTED_SYMBOLS) == names
    so = _abi.find_library_path()
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], check=True,
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (neptune_\w+)$", out, re.M))
    assert set(names) <= exported
    for n in names:
        assert hasattr(lib, n)


def test_library_does_not_link_the_oracle():
    so = _abi.find_library_path()
    out = subprocess.run(["nm", "-D", str(so)], check=True, capture_output=True,
                         text=True).stdout
    assert "neptune_cpu_" not in out
    deps = subprocess.run(["ldd", str(so)], capture_output=True, text=True).stdout
    assert "oracle" not in deps


def test_backend_info(lib):
    info = _abi.backend_info(lib)
    assert info["abi_version"] == _abi.ABI_VERSION == 1
    assert info["name"] == "NeptuneHTileHIP"
    assert info["gcn_arch"] == "gfx950"
    assert isinstance(info["hip_runtime_version"], int)
    assert lib.neptune_hip_get_backend_info(None) == _abi.ERR_INVALID_ARGUMENT
    assert b"NULL" in lib.neptune_last_error()


_LAYOUT_C = r"""
#include <stddef.h>
#include <stdio.h>
#include "neptune_hip.h"
#define F(T, f) printf(#T " " #f " %zu\n", offsetof(T, f));
#define S(T) printf(#T " sizeof %zu\n", sizeof(T));
int main(void) {
  F(neptune_attn_desc, batch) F(neptune_attn_desc, heads_q) F(neptune_attn_desc, heads_kv)
  F(neptune_attn_desc, seq_q) F(neptune_attn_desc, seq_kv) F(neptune_attn_desc, head_dim)
  F(neptune_attn_desc, q_stride) F(neptune_attn_desc, k_stride) F(neptune_attn_desc, v_stride)
  F(neptune_attn_desc, o_stride) F(neptune_attn_desc, dtype) F(neptune_attn_desc, causal)
  F(neptune_attn_desc, scale_log2) F(neptune_attn_desc, pipeline_stages)
  F(neptune_attn_desc, k_dim_order) S(neptune_attn_desc)
  F(neptune_decode_desc, batch) F(neptune_decode_desc, heads_q) F(neptune_decode_desc, heads_kv)
  F(neptune_decode_desc, seq_kv) F(neptune_decode_desc, head_dim)
  F(neptune_decode_desc, num_splits) F(neptune_decode_desc, scale_block)
  F(neptune_decode_desc, q_dtype) F(neptune_decode_desc, kv_dtype)
  F(neptune_decode_desc, scale_log2) F(neptune_decode_desc, reserved) S(neptune_decode_desc)
  F(neptune_paged_kv_desc, num_pages) F(neptune_paged_kv_desc, page_size)
  F(neptune_paged_kv_desc, max_pages) F(neptune_paged_kv_desc, k_stride)
  F(neptune_paged_kv_desc, v_stride) S(neptune_paged_kv_desc)
  F(neptune_scan_desc, batch) F(neptune_scan_desc, dim) F(neptune_scan_desc, seq_len)
  F(neptune_scan_desc, d_state) F(neptune_scan_desc, io_dtype)
  F(neptune_scan_desc, delta_softplus) S(neptune_scan_desc)
  F(neptune_backend_info, abi_version) F(neptune_backend_info, name)
  F(neptune_backend_info, gcn_arch) F(neptune_backend_info, hip_runtime_version)
  S(neptune_backend_info)
  return 0;
}
"""


def test_ctypes_descriptors_match_the_c_header(tmp_path):
    """Offsets and sizes the C compiler gives the header's structs equal
    the ctypes declarations of both the product package and the oracle."""
    src = tmp_path / "layout.c"
    src.write_text(_LAYOUT_C)
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    c = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        t, f, n = line.split()
        c[(t, f)] = int(n)
    pairs = [("neptune_attn_desc", _abi.AttnDesc, oracle.AttnDesc),
             ("neptune_decode_desc", _abi.DecodeDesc, oracle.DecodeDesc),
             ("neptune_scan_desc", _abi.ScanDesc, oracle.ScanDesc),
             ("neptune_paged_kv_desc", _abi.PagedKvDesc, oracle.PagedKvDesc),
             ("neptune_backend_info", _abi.BackendInfo, None)]
    for cname, prod, orc in pairs:
        for cls in (prod, orc):
            if cls is None:
                continue
            assert ctypes.sizeof(cls) == c[(cname, "sizeof")], (cname, cls)
            for fname, _ in cls._fields_:
                assert getattr(cls, fname).offset == c[(cname, fname)], (cname, fname)


def _attn_desc(**kw):
    d = _abi.AttnDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_q, d.seq_kv, d.head_dim = 1, 4, 2, 256, 256, 128
    d.dtype = _abi.DTYPE_BF16
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def _attn(lib, d, ptrs=(FAKE, FAKE, FAKE, FAKE)):
    return lib.neptune_attn_fwd(ctypes.byref(d) if d is not None else None, *ptrs, None, None)


@pytest.mark.parametrize("field,value,status", [
    ("batch", 0, _abi.ERR_INVALID_ARGUMENT),
    ("seq_q", -1, _abi.ERR_INVALID_ARGUMENT),
    ("head_dim", 0, _abi.ERR_INVALID_ARGUMENT),
    ("heads_kv", 3, _abi.ERR_INVALID_ARGUMENT),         # 4 % 3 != 0
    ("dtype", _abi.DTYPE_FP8_E4M3, _abi.ERR_UNSUPPORTED),
    ("dtype", 17, _abi.ERR_UNSUPPORTED),
    ("head_dim", 96, _abi.ERR_UNSUPPORTED),
    ("scale_log2", float("nan"), _abi.ERR_INVALID_ARGUMENT),
    ("scale_log2", -1.0, _abi.ERR_INVALID_ARGUMENT),
    ("pipeline_stages", 4, _abi.ERR_INVALID_ARGUMENT),
    ("pipeline_stages", -1, _abi.ERR_INVALID_ARGUMENT),
    ("k_dim_order", 2, _abi.ERR_INVALID_ARGUMENT),
])
def test_attn_validation(lib, field, value, status):
    assert _attn(lib, _attn_desc(**{field: value})) == status
    assert lib.neptune_last_error()


def test_attn_null_and_stride_errors(lib):
    assert _attn(lib, None) == _abi.ERR_INVALID_ARGUMENT
    assert _attn(lib, _attn_desc(), (FAKE, 0, FAKE, FAKE)) == _abi.ERR_INVALID_ARGUMENT
    d = _attn_desc()
    d.q_stride[:] = (0, 128, 1)  # mixed zero / positive
    assert _attn(lib, d) == _abi.ERR_INVALID_ARGUMENT
    d = _attn_desc()
    d.k_stride[:] = (256 * 128 * 2, 256 * 128, 132)  # not a multiple of 8 elements
    assert _attn(lib, d) == _abi.ERR_UNSUPPORTED
    assert _attn(lib, _attn_desc(), (FAKE + 2, FAKE, FAKE, FAKE)) == _abi.ERR_UNSUPPORTED
    assert b"aligned" in lib.neptune_last_error()


@pytest.mark.parametrize("kw,status", [
    (dict(pipeline_stages=3, head_dim=64), _abi.ERR_UNSUPPORTED),   # knob is head_dim-128 only
    (dict(pipeline_stages=1, dtype=_abi.DTYPE_F32), _abi.ERR_UNSUPPORTED),
    (dict(k_dim_order=1, head_dim=64), _abi.ERR_UNSUPPORTED),
    (dict(k_dim_order=1, seq_kv=100), _abi.ERR_UNSUPPORTED),         # contiguous K^T row of 100
    (dict(batch=8192, heads_q=2048, heads_kv=2048, seq_q=256), _abi.ERR_UNSUPPORTED),  # 2^33 work-items
    (dict(pipeline_stages=2, dtype=_abi.DTYPE_F32, head_dim=64), _abi.ERR_NO_DEVICE),
    (dict(pipeline_stages=3, k_dim_order=1), _abi.ERR_NO_DEVICE),
    (dict(pipeline_stages=1), _abi.ERR_NO_DEVICE),
])
def test_attn_knob_validation(lib, kw, status):
    """Knob combinations the kernels do not cover are rejected before any
    device call; valid ones get as far as the device check (only where no
    device exists: these descriptors carry placeholder pointers)."""
    if status == _abi.ERR_NO_DEVICE and lib.neptune_device_count() > 0:
        pytest.skip("a HIP device is visible; the no-device path is not reachable")
    assert _attn(lib, _attn_desc(**kw)) == status


def test_attn_k_dim_order_strides(lib):
    """With k_dim_order 1 the K strides are (batch, head, head_dim row): a
    row stride of 260 elements passes the 16-bit rules only if it is a
    multiple of 8."""
    d = _attn_desc(k_dim_order=1, seq_kv=256)
    d.k_stride[:] = (2 * 128 * 264, 128 * 264, 260)
    assert _attn(lib, d) == _abi.ERR_UNSUPPORTED
    if lib.neptune_device_count() == 0:
        d.k_stride[:] = (2 * 128 * 264, 128 * 264, 264)
        assert _attn(lib, d) == _abi.ERR_NO_DEVICE


def _dec_desc(**kw):
    d = _abi.DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = 2, 8, 2, 1000, 128
    d.num_splits, d.scale_block = 3, 64
    d.q_dtype, d.kv_dtype = _abi.DTYPE_BF16, _abi.DTYPE_BF16
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_decode_workspace_matches_layout(lib):
    d = _dec_desc()
    n = ctypes.c_size_t()
    assert lib.neptune_decode_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == _abi.OK
    splits, _ = oracle.decode_layout(2, 2, 1000, 3)
    rows = 2 * 8 * splits
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert n.value == align(rows * 128 * 4) + align(rows * 2 * 4)
    assert lib.neptune_decode_workspace_bytes(ctypes.byref(d), None) == _abi.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("B,Hk,L,splits", [(16, 8, 32768, 16), (2, 2, 1000, 3), (1, 1, 100000, 0),
                                           (4, 2, 50, 0), (3, 1, 4097, 0), (1, 1, 64, 7)])
def test_decode_split_rule_agrees_with_oracle(lib, B, Hk, L, splits):
    """The library's workspace size follows the split count the oracle
    computes for the same request."""
    d = _dec_desc(batch=B, heads_q=Hk, heads_kv=Hk, seq_kv=L, num_splits=splits)
    n = ctypes.c_size_t()
    assert lib.neptune_decode_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == _abi.OK
    s, c = oracle.decode_layout(B, Hk, L, splits)
    assert c % 64 == 0 and (s - 1) * c < L <= s * c
    rows = B * Hk * s
    assert n.value == (rows * 128 * 4 + 255) // 256 * 256 + (rows * 8 + 255) // 256 * 256


def _decode(lib, d, ws_bytes=1 << 30, kscale=None, ptrs=(FAKE, FAKE, FAKE)):
    return lib.neptune_decode_splitk(ctypes.byref(d), *ptrs, kscale, kscale, FAKE, None, FAKE,
                                     ws_bytes, None)


@pytest.mark.parametrize("kw,status", [
    ({"heads_q": 5}, _abi.ERR_INVALID_ARGUMENT),           # 5 % 2
    ({"seq_kv": 0}, _abi.ERR_INVALID_ARGUMENT),
    ({"num_splits": -1}, _abi.ERR_INVALID_ARGUMENT),
    ({"q_dtype": _abi.DTYPE_F16}, _abi.ERR_UNSUPPORTED),
    ({"kv_dtype": _abi.DTYPE_F32}, _abi.ERR_UNSUPPORTED),
    ({"head_dim": 64}, _abi.ERR_UNSUPPORTED),
    ({"heads_q": 64, "heads_kv": 2}, _abi.ERR_UNSUPPORTED),  # group 32 > 16
])
def test_decode_validation(lib, kw, status):
    assert _decode(lib, _dec_desc(**kw)) == status
    assert lib.neptune_last_error()


def test_decode_workspace_and_fp8_errors(lib):
    assert _decode(lib, _dec_desc(), ws_bytes=16) == _abi.ERR_WORKSPACE_TOO_SMALL
    assert b"need" in lib.neptune_last_error()
    fp8 = _dec_desc(kv_dtype=_abi.DTYPE_FP8_E4M3)
    assert _decode(lib, fp8) == _abi.ERR_INVALID_ARGUMENT            # scales missing
    assert _decode(lib, _dec_desc(kv_dtype=_abi.DTYPE_FP8_E4M3, scale_block=48),
                   kscale=FAKE) == _abi.ERR_UNSUPPORTED              # not a multiple of 32
    assert _decode(lib, _dec_desc(), ptrs=(FAKE, FAKE, 0)) == _abi.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("ws,ws_bytes,status", [
    (None, 1 << 30, _abi.ERR_INVALID_ARGUMENT),
    # any pointer value is a caller's workspace: its size is checked, and the
    # library's static scratch is reached only through the noalloc entry point
    ((1 << 64) - 1, 0, _abi.ERR_WORKSPACE_TOO_SMALL),
    ((1 << 64) - 16, 16, _abi.ERR_WORKSPACE_TOO_SMALL),
])
def test_decode_workspace_pointer_is_the_callers(lib, ws, ws_bytes, status):
    d = _dec_desc()
    assert lib.neptune_decode_splitk(ctypes.byref(d), FAKE, FAKE, FAKE, None, None, FAKE, None, ws,
                                     ws_bytes, None) == status
    assert lib.neptune_last_error()


def _pages(**kw):
    p = _abi.PagedKvDesc()
    p.num_pages, p.page_size, p.max_pages = 64, 64, 32
    p.k_stride[:] = (2 * 64 * 128, 64 * 128, 128)
    p.v_stride[:] = (2 * 64 * 128, 64 * 128, 128)
    for k, v in kw.items():
        if k in ("k_stride", "v_stride"):
            getattr(p, k)[:] = v
        else:
            setattr(p, k, v)
    return p


def _paged(lib, d, p, ws_bytes=1 << 30, ptrs=(FAKE,) * 5):
    return lib.neptune_decode_paged(ctypes.byref(d), ctypes.byref(p) if p is not None else None,
                                    *ptrs, FAKE, None, FAKE, ws_bytes, None)


@pytest.mark.parametrize("dkw,pkw,status", [
    ({}, {"page_size": 48}, _abi.ERR_UNSUPPORTED),                 # not a multiple of 32
    ({}, {"max_pages": 15}, _abi.ERR_INVALID_ARGUMENT),             # 15 * 64 < seq_kv 1000
    ({}, {"num_pages": 0}, _abi.ERR_INVALID_ARGUMENT),
    ({}, {"k_stride": (100, 64 * 128, 128)}, _abi.ERR_UNSUPPORTED),  # not a multiple of 8
    ({}, {"v_stride": (2 * 64 * 128, 64 * 128, 256)}, _abi.ERR_UNSUPPORTED),  # K/V token strides
    ({"kv_dtype": _abi.DTYPE_FP8_E4M3}, {}, _abi.ERR_UNSUPPORTED),
    ({"heads_q": 5}, {}, _abi.ERR_INVALID_ARGUMENT),
])
def test_paged_decode_validation(lib, dkw, pkw, status):
    assert _paged(lib, _dec_desc(**dkw), _pages(**pkw)) == status
    assert lib.neptune_last_error()


def test_paged_decode_null_arguments(lib):
    assert _paged(lib, _dec_desc(), None) == _abi.ERR_INVALID_ARGUMENT
    for i in range(5):
        ptrs = [FAKE] * 5
        ptrs[i] = None
        assert _paged(lib, _dec_desc(), _pages(), ptrs=tuple(ptrs)) == _abi.ERR_INVALID_ARGUMENT
    assert _paged(lib, _dec_desc(), _pages(), ws_bytes=16) == _abi.ERR_WORKSPACE_TOO_SMALL


def test_paged_decode_no_device_path(lib):
    if lib.neptune_device_count() > 0:
        pytest.skip("a HIP device is visible; the no-device path is not reachable")
    assert _paged(lib, _dec_desc(), _pages()) == _abi.ERR_NO_DEVICE


def _paged8(lib, d, p, ws_bytes=1 << 30, ptrs=(FAKE,) * 7):
    """neptune_decode_paged_fp8 with q, k, v, k_scales, v_scales, block_table,
    seq_lens = ptrs."""
    return lib.neptune_decode_paged_fp8(ctypes.byref(d),
                                        ctypes.byref(p) if p is not None else None,
                                        *ptrs, FAKE, None, FAKE, ws_bytes, None)


def _fp8_desc(**kw):
    kw.setdefault("kv_dtype", _abi.DTYPE_FP8_E4M3)
    kw.setdefault("scale_block", 0)
    return _dec_desc(**kw)


@pytest.mark.parametrize("dkw,pkw,status", [
    ({"scale_block": 32}, {}, _abi.ERR_UNSUPPORTED),               # one scale per page only
    ({"kv_dtype": _abi.DTYPE_BF16}, {}, _abi.ERR_INVALID_ARGUMENT),  # bf16 pools: decode_paged
    ({}, {"k_stride": (2 * 64 * 128, 64 * 128, 136)}, _abi.ERR_UNSUPPORTED),  # not 16 bytes
    ({}, {"page_size": 48}, _abi.ERR_UNSUPPORTED),
    ({}, {"max_pages": 15}, _abi.ERR_INVALID_ARGUMENT),
])
def test_paged_fp8_decode_validation(lib, dkw, pkw, status):
    assert _paged8(lib, _fp8_desc(**dkw), _pages(**pkw)) == status
    assert lib.neptune_last_error()


def test_paged_fp8_decode_null_arguments(lib):
    assert _paged8(lib, _fp8_desc(), None) == _abi.ERR_INVALID_ARGUMENT
    for i in range(7):
        ptrs = [FAKE] * 7
        ptrs[i] = None
        assert _paged8(lib, _fp8_desc(), _pages(), ptrs=tuple(ptrs)) == _abi.ERR_INVALID_ARGUMENT
    assert _paged8(lib, _fp8_desc(), _pages(), ws_bytes=16) == _abi.ERR_WORKSPACE_TOO_SMALL


def test_paged_fp8_decode_no_device_path(lib):
    if lib.neptune_device_count() > 0:
        pytest.skip("a HIP device is visible; the no-device path is not reachable")
    # scale_block 0 and scale_block == page_size are both accepted
    assert _paged8(lib, _fp8_desc(), _pages()) == _abi.ERR_NO_DEVICE
    assert _paged8(lib, _fp8_desc(scale_block=64), _pages()) == _abi.ERR_NO_DEVICE


def test_quantize_and_scan_validation(lib):
    q = lib.neptune_kv_quantize_fp8
    assert q(1, 1, 64, 128, 64, None, FAKE, FAKE, None) == _abi.ERR_INVALID_ARGUMENT
    assert q(1, 0, 64, 128, 64, FAKE, FAKE, FAKE, None) == _abi.ERR_INVALID_ARGUMENT
    d = _abi.ScanDesc(1, 64, 128, 16, _abi.DTYPE_BF16, 1)
    s = lib.neptune_selective_scan_fwd
    assert s(None, *([FAKE] * 9), None) == _abi.ERR_INVALID_ARGUMENT
    bad = _abi.ScanDesc(1, 64, 0, 16, _abi.DTYPE_BF16, 1)
    assert s(ctypes.byref(bad), *([FAKE] * 9), None) == _abi.ERR_INVALID_ARGUMENT
    f16 = _abi.ScanDesc(1, 64, 128, 16, _abi.DTYPE_F16, 1)
    assert s(ctypes.byref(f16), *([FAKE] * 9), None) == _abi.ERR_UNSUPPORTED
    n8 = _abi.ScanDesc(1, 64, 128, 8, _abi.DTYPE_BF16, 1)
    assert s(ctypes.byref(n8), *([FAKE] * 9), None) == _abi.ERR_UNSUPPORTED
    assert s(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE,
             None) == _abi.ERR_INVALID_ARGUMENT  # C missing
    # the output kernel's 32-bit offsets span 16 rows of a sequence: below 2^26 steps
    long_seq = _abi.ScanDesc(1, 16, 1 << 26, 16, _abi.DTYPE_BF16, 1)
    assert s(ctypes.byref(long_seq), *([FAKE] * 9), None) == _abi.ERR_UNSUPPORTED
    assert b"seq_len below 2^26" in lib.neptune_last_error()
    if lib.neptune_device_count() == 0:
        just_under = _abi.ScanDesc(1, 16, (1 << 26) - 2, 16, _abi.DTYPE_BF16, 1)
        apart = [FAKE + (i << 32) for i in range(9)]  # 4 GiB apart: no overlap
        assert s(ctypes.byref(just_under), *apart, None) == _abi.ERR_NO_DEVICE


def _scan_pointers(**moved):
    """Fake addresses of u, delta, A, B, C, D, z, delta_bias, y, 1 MiB apart
    (no overlap for the 1x64x128 desc below), with `moved` ones replaced."""
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias", "y")
    base = {n: FAKE + (i << 20) for i, n in enumerate(names)}
    base.update(moved)
    return [base[n] for n in names]


@pytest.mark.parametrize("moved, culprit", [
    ({"y": FAKE}, b"u"),                                   # y is u
    ({"y": FAKE + (1 << 20) + 16 * 1024 - 2}, b"delta"),   # y's first element is delta's last
    ({"y": FAKE + (3 << 20) - 16 * 1024 + 2}, b"B"),       # y's tail runs into B
    ({"y": FAKE + (5 << 20) + 200}, b"D"),                 # D inside y
    ({"z": FAKE + (8 << 20) + 4096}, b"z"),                # z inside y
    ({"delta_bias": FAKE + (8 << 20)}, b"delta_bias"),
])
def test_scan_rejects_y_overlapping_an_input(lib, moved, culprit):
    """y is written while later steps are read and holds per-chunk state, so
    a y that shares any byte with an input is INVALID_ARGUMENT, checked before
    any device work."""
    d = _abi.ScanDesc(1, 64, 128, 16, _abi.DTYPE_BF16, 1)  # u, delta, z, y 16 KiB; B, C 4 KiB
    s = lib.neptune_selective_scan_fwd
    assert s(ctypes.byref(d), *_scan_pointers(**moved), None) == _abi.ERR_INVALID_ARGUMENT
    assert lib.neptune_last_error() == b"selective_scan: y overlaps " + culprit


def test_scan_accepts_adjacent_and_null_optional_inputs(lib):
    """Ranges that touch but share no byte, and NULL D, z and delta_bias,
    pass the overlap check (NO_DEVICE on a host without a GPU)."""
    if lib.neptune_device_count() > 0:
        pytest.skip("a HIP device is visible: a valid request would launch on fake pointers")
    d = _abi.ScanDesc(1, 64, 128, 16, _abi.DTYPE_BF16, 1)
    s = lib.neptune_selective_scan_fwd
    ptr = _scan_pointers(y=FAKE + 16 * 1024)  # y starts where u ends
    assert s(ctypes.byref(d), *ptr, None) == _abi.ERR_NO_DEVICE
    ptr = _scan_pointers(y=FAKE + (3 << 20) - 16 * 1024)  # y ends where B starts
    assert s(ctypes.byref(d), *ptr, None) == _abi.ERR_NO_DEVICE
    ptr = _scan_pointers(D=None, z=None, delta_bias=None, y=FAKE + (5 << 20))
    assert s(ctypes.byref(d), *ptr, None) == _abi.ERR_NO_DEVICE


def test_no_device_path(lib):
    """A fully valid request on a host without a HIP device reports
    NO_DEVICE instead of crashing (never reached where a device exists)."""
    if lib.neptune_device_count() > 0:
        pytest.skip("a HIP device is visible; the no-device path is not reachable")
    assert _attn(lib, _attn_desc()) == _abi.ERR_NO_DEVICE
    assert b"no HIP device" in lib.neptune_last_error()
    with pytest.raises(_abi.NeptuneNoDevice):
        _abi.check(_abi.ERR_NO_DEVICE, lib)


def test_error_text_is_thread_local(lib):
    assert _attn(lib, _attn_desc(batch=0)) == _abi.ERR_INVALID_ARGUMENT
    mine = lib.neptune_last_error()
    other = {}

    def worker():
        other["before"] = lib.neptune_last_error()
        _abi.backend_info(lib)
        other["after"] = lib.neptune_last_error()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert other["before"] == b"" and other["after"] == b""
    assert lib.neptune_last_error() == mine


def test_status_to_exception_mapping(lib):
    assert _attn(lib, _attn_desc(head_dim=96)) == _abi.ERR_UNSUPPORTED
    with pytest.raises(NotImplementedError):
        _abi.check(_abi.ERR_UNSUPPORTED, lib)
    with pytest.raises(ValueError):
        _abi.check(_abi.ERR_INVALID_ARGUMENT, lib)
    with pytest.raises(_abi.NeptuneWorkspaceTooSmall):
        _abi.check(_abi.ERR_WORKSPACE_TOO_SMALL, lib)
    with pytest.raises(RuntimeError):
        _abi.check(_abi.ERR_HIP, lib)


def test_locator_order(tmp_path, monkeypatch):
    """Explicit path, then NEPTUNE_HIP_LIB, then the package's _native dir
    (the reference's plugin resolution order, src/neptune_mlir/plugin.py:28-55)."""
    fake = tmp_path / "libneptune_hip.so"
    fake.write_bytes(b"")
    monkeypatch.delenv(_abi.LIBRARY_ENV, raising=False)
    default = _abi.find_library_path()
    assert default is not None and default.parent.name == "_native"
    assert _abi.find_library_path(fake) == fake.resolve()
    monkeypatch.setenv(_abi.LIBRARY_ENV, str(fake))
    assert _abi.find_library_path() == fake.resolve()
    monkeypatch.setenv(_abi.LIBRARY_ENV, str(tmp_path / "missing.so"))
    assert _abi.find_library_path() == default


@pytest.mark.parametrize("field,stride", [
    ("k_stride", (1, 1, 34_100_000)),   # 63 rows x 68.2 MB per K row passes 2^32 bytes
    ("v_stride", (1, 1, 34_100_000)),
])
def test_attn_rejects_tiles_past_32_bit_offsets(lib, field, stride):
    """A 64-key K or V tile is addressed as a base plus 32-bit per-lane byte
    offsets; token strides that would wrap them are UNSUPPORTED, not
    silently read from the wrong rows."""
    d = _attn_desc()
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(d, name)[:] = (1 << 40, 1 << 32, 128)
    getattr(d, field)[:] = (1 << 40, 1 << 32, stride[2] // 8 * 8)
    assert _attn(lib, d) == _abi.ERR_UNSUPPORTED
    assert b"4 GiB" in lib.neptune_last_error()


def test_attn_rejects_long_head_dim_major_k(lib):
    """k_dim_order 1 spans 128 head_dim rows of seq_kv keys: seq_kv above
    about 16.9M tokens would wrap the 32-bit offsets."""
    L = 17_000_000
    d = _attn_desc(k_dim_order=1, seq_kv=L, seq_q=128)
    assert _attn(lib, d) == _abi.ERR_UNSUPPORTED
    assert b"4 GiB" in lib.neptune_last_error()
    if lib.neptune_device_count() == 0:
        ok = _attn_desc(k_dim_order=1, seq_kv=16_000_000, seq_q=128)
        assert _attn(lib, ok) == _abi.ERR_NO_DEVICE


def test_decode_rejects_splits_past_the_combine_lds(lib):
    """decode_combine keeps one fp32 weight per split in LDS: more than
    16384 splits is UNSUPPORTED at validation, before any launch."""
    L = 64 * 16385
    d = _dec_desc(batch=1, heads_q=1, heads_kv=1, seq_kv=L, num_splits=16385)
    assert _decode(lib, d) == _abi.ERR_UNSUPPORTED
    assert b"16384 splits" in lib.neptune_last_error()
    if lib.neptune_device_count() == 0:
        d = _dec_desc(batch=1, heads_q=1, heads_kv=1, seq_kv=L, num_splits=16384)
        assert _decode(lib, d) == _abi.ERR_NO_DEVICE
