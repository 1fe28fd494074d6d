"""Concurrent host threads, each on its own stream, calling the library.

Apart from neptune_decode_splitk_noalloc (whose shared scratch makes
overlapping calls race, as its header states), every entry point keeps no
state between calls: buffers belong to the caller and the last-error text is
kept per thread. So four threads running decode, prefill and scan on their
own streams and inputs at once must produce exactly what the same calls
produce one after another. Each thread also makes its own kind of invalid
call between launches and checks that the error text it reads back is its
own.
"""

import ctypes
import threading

import pytest
import torch

from helpers import randn
from neptune_hip import _abi, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _inputs(t):
    """Thread t's inputs: a decode step, a causal prefill and a scan."""
    q = randn((2, 8, 128), seed=500 + t).cuda()
    k = randn((2, 2, 1500 + 100 * t, 128), seed=510 + t).cuda()
    v = randn((2, 2, 1500 + 100 * t, 128), seed=520 + t).cuda()
    pq, pk, pv = (randn((1, 2, 300 + 50 * t, 128), seed=530 + 10 * t + s, scale=0.5).cuda()
                  for s in range(3))
    L = 256 + 64 * t
    su, sdr, sz = (randn((1, 32, L), seed=560 + 10 * t + s).cuda() for s in range(3))
    sB, sC = (randn((1, 16, L), seed=590 + 10 * t + s).cuda() for s in range(2))
    sA = -torch.exp(randn((32, 16), seed=620 + t, dtype=torch.float32)).cuda()
    return (q, k, v), (pq, pk, pv), (su, sdr, sA, sB, sC, None, sz, None)


def _bad_call(lib, t):
    """A call that fails host-side validation, a different one per thread;
    returns (status, the message this thread then reads, the expected text)."""
    fake = 0x10000  # never dereferenced: each call fails before any launch
    if t in (0, 1):
        d = _abi.DecodeDesc()
        d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = 1, 8, 2, 256, 128
        d.num_splits = 1
        d.q_dtype = d.kv_dtype = _abi.DTYPE_BF16
        if t == 0:
            st = lib.neptune_decode_workspace_bytes(ctypes.byref(d), None)
            want = "bytes is NULL"
        else:
            st = lib.neptune_decode_splitk(ctypes.byref(d), fake, fake, fake, None, None, fake,
                                           None, fake, 0, None)
            want = "workspace 0 bytes"
    elif t == 2:
        a = _abi.AttnDesc()
        a.batch, a.heads_q, a.heads_kv, a.seq_q, a.seq_kv, a.head_dim = 1, 2, 2, 64, 64, 96
        a.dtype = _abi.DTYPE_BF16
        for i in range(3):
            a.q_stride[i] = a.k_stride[i] = a.v_stride[i] = a.o_stride[i] = 0
        st = lib.neptune_attn_fwd(ctypes.byref(a), fake, fake, fake, fake, None, None)
        want = "head_dim"
    else:
        sd = _abi.ScanDesc()
        sd.batch, sd.dim, sd.seq_len, sd.d_state = 1, 16, 64, 8
        sd.io_dtype = _abi.DTYPE_BF16
        st = lib.neptune_selective_scan_fwd(ctypes.byref(sd), fake, fake, fake, fake, fake, None,
                                            None, None, fake, None)
        want = "d_state 16"
    return st, (lib.neptune_last_error() or b"").decode(), want


def _work(inp):
    dec, pre, scan = inp
    o = ops.decode_splitk(*dec, num_splits=4)
    a = ops.attention(*pre, causal=True)
    y = ops.selective_scan(*scan)
    return o, a, y


def test_threads_on_own_streams_equal_sequential_calls():
    n = 4
    inputs = [_inputs(t) for t in range(n)]
    torch.cuda.synchronize()
    want = [_work(inp) for inp in inputs]
    torch.cuda.synchronize()

    got = [None] * n
    errors = [None] * n
    start = threading.Barrier(n)

    def run(t):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            start.wait()
            lib = _abi.load_library()
            msgs = []
            with torch.cuda.stream(stream):
                for _ in range(3):
                    res = _work(inputs[t])
                    # between launches, a failing call: the error text this
                    # thread reads back is its own, whatever the others do
                    for _ in range(20):
                        msgs.append(_bad_call(lib, t))
            stream.synchronize()
            got[t] = (res, msgs)
        except BaseException as e:  # reported by the main thread
            errors[t] = e

    threads = [threading.Thread(target=run, args=(t,)) for t in range(n)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert all(not th.is_alive() for th in threads), "a worker thread did not finish"
    for t in range(n):
        assert errors[t] is None, f"thread {t}: {errors[t]!r}"
        (o, a, y), msgs = got[t]
        wo, wa, wy = want[t]
        assert torch.equal(o.view(torch.int16), wo.view(torch.int16)), f"thread {t}: decode"
        assert torch.equal(a.view(torch.int16), wa.view(torch.int16)), f"thread {t}: prefill"
        assert torch.equal(y.view(torch.int16), wy.view(torch.int16)), f"thread {t}: scan"
        for st, msg, expect in msgs:
            assert st in (_abi.ERR_UNSUPPORTED, _abi.ERR_INVALID_ARGUMENT,
                          _abi.ERR_WORKSPACE_TOO_SMALL), (t, st, msg)
            assert expect in msg, f"thread {t} read another thread's error: {msg!r}"
