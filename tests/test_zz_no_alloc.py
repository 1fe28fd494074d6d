"""The allocation-free decode entry point, neptune_decode_splitk_noalloc,
called through the C-ABI against neptune_decode_splitk with a caller-owned
workspace: the same kernels, so the outputs must agree bit for bit. Two
calls run back to back on one device, the second on a smaller input, so the
shared static scratch is reused with stale contents from the first."""

import ctypes

import pytest
import torch

from helpers import randn
from neptune_hip import _abi, ops

FAKE = 0x10000


def _desc(B, Hq, Hk, L, splits, fp8=False):
    d = _abi.DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = B, Hq, Hk, L, 128
    d.num_splits, d.scale_block = splits, 64
    d.q_dtype = _abi.DTYPE_BF16
    d.kv_dtype = _abi.DTYPE_FP8_E4M3 if fp8 else _abi.DTYPE_BF16
    return d


def test_noalloc_rejects_requests_past_its_scratch():
    """16 MiB of partials at most: 64 x 64 rows x 64 splits need 8.5x that.
    Rejected on the host before any HIP call."""
    lib = _abi.load_library()
    d = _desc(64, 64, 8, 64 * 4096, 64)
    st = lib.neptune_decode_splitk_noalloc(ctypes.byref(d), FAKE, FAKE, FAKE, None, None, FAKE,
                                           None, None)
    assert st == _abi.ERR_WORKSPACE_TOO_SMALL
    assert b"static scratch" in lib.neptune_last_error()
    d8 = _desc(2, 8, 2, 1000, 3, fp8=True)
    assert lib.neptune_decode_splitk_noalloc(ctypes.byref(d8), FAKE, FAKE, FAKE, None, None, FAKE,
                                             None, None) == _abi.ERR_INVALID_ARGUMENT
    if lib.neptune_device_count() == 0:
        d = _desc(2, 8, 2, 1000, 3)
        assert lib.neptune_decode_splitk_noalloc(ctypes.byref(d), FAKE, FAKE, FAKE, None, None,
                                                 FAKE, None, None) == _abi.ERR_NO_DEVICE


def _run_pair(lib, B, Hq, Hk, L, splits, fp8, seed):
    """(o, lse) from the workspace entry point and from the allocation-free
    one, on the same device inputs."""
    q = randn((B, Hq, 128), seed=seed).cuda()
    k = randn((B, Hk, L, 128), seed=seed + 1).cuda()
    v = randn((B, Hk, L, 128), seed=seed + 2).cuda()
    ks = vs = None
    if fp8:
        k, ks = ops.kv_quantize_fp8(k)
        v, vs = ops.kv_quantize_fp8(v)
    d = _desc(B, Hq, Hk, L, splits, fp8)
    n = ctypes.c_size_t()
    _abi.check(lib.neptune_decode_workspace_bytes(ctypes.byref(d), ctypes.byref(n)), lib)
    ws = torch.empty(n.value, dtype=torch.uint8, device="cuda")
    outs = []
    for noalloc in (False, True):
        o = torch.full((B, Hq, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        lse = torch.full((B, Hq), float("nan"), dtype=torch.float32, device="cuda")
        args = (ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                ks.data_ptr() if fp8 else None, vs.data_ptr() if fp8 else None, o.data_ptr(),
                lse.data_ptr())
        stream = torch.cuda.current_stream().cuda_stream
        if noalloc:
            st = lib.neptune_decode_splitk_noalloc(*args, stream)
        else:
            st = lib.neptune_decode_splitk(*args, ws.data_ptr(), n.value, stream)
        _abi.check(st, lib)
        outs.append((o, lse))
    torch.cuda.synchronize()
    return outs


@pytest.mark.gpu
@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_equals_workspace_decode_on_two_calls(fp8):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    lib = _abi.load_library()
    # first a config-3-like row count, then a smaller ragged request whose
    # partials cover only the front of the scratch left by the first
    for i, (B, Hq, Hk, L, splits) in enumerate([(8, 32, 8, 8192, 16), (3, 8, 2, 1000, 3)]):
        print(f"case: decode_noalloc fp8={fp8} call {i}: B={B} Hq={Hq} Hk={Hk} L={L} "
              f"splits={splits}", flush=True)
        (o_ws, lse_ws), (o_na, lse_na) = _run_pair(lib, B, Hq, Hk, L, splits, fp8, seed=40 + i)
        assert not torch.isnan(o_ws.float()).any()
        assert torch.equal(o_ws.view(torch.int16), o_na.view(torch.int16))
        assert torch.equal(lse_ws.view(torch.int32), lse_na.view(torch.int32))
