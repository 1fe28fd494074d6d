"""The hot-path entry points captured in a HIP graph and replayed.

A serving loop captures its decode step (or prefill) once and replays it.
Every entry point here only launches kernels: no memset, no allocation, no
synchronisation, and the one-time host set-up (the static scratch address of
the allocation-free entry point) happens on the first call, which runs
before the capture.
So each replay must equal an eager call on the same inputs bit for bit.
Each test replays three times, rewriting the inputs in place before each
replay and running eager work of another shape between replays, and checks
every replay against an eager call made after it.
"""

import ctypes

import pytest
import torch

from helpers import randn
from neptune_hip import _abi, ops

pytestmark = pytest.mark.gpu

REPLAYS = 3


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _log(msg):
    print(msg, flush=True)


def _capture(fn):
    """Run fn once on a side stream (first-call set-up), then capture it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    torch.cuda.synchronize()
    return graph, out


def _same(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b)


def _decode_inputs(B, Hq, Hk, L, seed, fp8):
    q = randn((B, Hq, 128), seed=seed).cuda()
    k = randn((B, Hk, L, 128), seed=seed + 1).cuda()
    v = randn((B, Hk, L, 128), seed=seed + 2).cuda()
    ks = vs = None
    if fp8:
        k, ks = ops.kv_quantize_fp8(k)
        v, vs = ops.kv_quantize_fp8(v)
    return q, k, v, ks, vs


@pytest.mark.parametrize("fp8", [False, True])
def test_graph_decode_replays_equal_eager(fp8):
    B, Hq, Hk, L, splits = 2, 16, 4, 3000, 5
    _log(f"graph decode fp8={fp8} B{B} Hq{Hq} Hk{Hk} L{L} splits{splits}")
    q, k, v, ks, vs = _decode_inputs(B, Hq, Hk, L, 11, fp8)
    ws = torch.empty(ops.decode_workspace_bytes(q, k, num_splits=splits, fp8=fp8),
                     dtype=torch.uint8, device="cuda")

    def step():
        return ops.decode_splitk(q, k, v, k_scale=ks, v_scale=vs, num_splits=splits,
                                 workspace=ws, return_lse=True)

    graph, (o_g, lse_g) = _capture(step)
    other = _decode_inputs(1, 8, 2, 777, 90, fp8)
    for r in range(REPLAYS):
        q.copy_(randn(q.shape, seed=100 + r).cuda())
        ops.decode_splitk(*other[:3], k_scale=other[3], v_scale=other[4], num_splits=3)
        graph.replay()
        o_e, lse_e = step()
        torch.cuda.synchronize()
        assert _same(o_g, o_e), f"replay {r}: output differs from the eager call"
        assert _same(lse_g, lse_e), f"replay {r}: lse differs from the eager call"


@pytest.mark.parametrize("fp8", [False, True])
def test_graph_noalloc_decode_replays_equal_workspace_entry(fp8):
    """The allocation-free entry point is the one graph-captured callers use:
    each replay equals neptune_decode_splitk with a workspace."""
    B, Hq, Hk, L, splits = 2, 16, 4, 2500, 4
    _log(f"graph noalloc decode fp8={fp8}")
    lib = _abi.load_library()
    q, k, v, ks, vs = _decode_inputs(B, Hq, Hk, L, 21, fp8)
    d = _abi.DecodeDesc()
    d.batch, d.heads_q, d.heads_kv, d.seq_kv, d.head_dim = B, Hq, Hk, L, 128
    d.num_splits, d.scale_block = splits, 64
    d.q_dtype = _abi.DTYPE_BF16
    d.kv_dtype = _abi.DTYPE_FP8_E4M3 if fp8 else _abi.DTYPE_BF16
    o = torch.empty((B, Hq, 128), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((B, Hq), dtype=torch.float32, device="cuda")
    sc = (ks.data_ptr(), vs.data_ptr()) if fp8 else (None, None)

    def step():
        stream = torch.cuda.current_stream().cuda_stream
        _abi.check(lib.neptune_decode_splitk_noalloc(
            ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(), *sc, o.data_ptr(),
            lse.data_ptr(), stream), lib)

    graph, _ = _capture(step)
    for r in range(REPLAYS):
        q.copy_(randn(q.shape, seed=200 + r).cuda())
        graph.replay()
        o_w, lse_w = ops.decode_splitk(q, k, v, k_scale=ks, v_scale=vs, num_splits=splits,
                                       return_lse=True)
        torch.cuda.synchronize()
        assert _same(o, o_w), f"replay {r}: output differs from the workspace entry point"
        assert _same(lse, lse_w), f"replay {r}: lse differs from the workspace entry point"


def test_graph_prefill_replays_equal_eager():
    B, H, S = 1, 4, 640
    _log(f"graph prefill causal bf16 B{B} H{H} S{S}")
    q, k, v = (randn((B, H, S, 128), seed=s, scale=0.5).cuda() for s in (31, 32, 33))
    out = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device="cuda")

    def step():
        return ops.attention(q, k, v, causal=True, out=out, lse=lse)

    graph, _ = _capture(step)
    other = [randn((1, 2, 200, 128), seed=s).cuda() for s in (40, 41, 42)]
    for r in range(REPLAYS):
        q.copy_(randn(q.shape, seed=300 + r, scale=0.5).cuda())
        ops.attention(*other, causal=False)
        graph.replay()
        torch.cuda.synchronize()
        o_g, lse_g = out.clone(), lse.clone()
        step()
        torch.cuda.synchronize()
        assert _same(o_g, out), f"replay {r}: output differs from the eager call"
        assert _same(lse_g, lse), f"replay {r}: lse differs from the eager call"


def test_graph_sequence_parallel_scan_replays_equal_eager():
    """Few channels and a long sequence: the captured step is the chunked
    path's three launches (state, carry, output), with y as their scratch."""
    b, d, L, n = 1, 32, 4096, 16
    _log(f"graph scan b{b} d{d} L{L} (sequence-parallel path)")
    u, dr, z = (randn((b, d, L), seed=s).cuda() for s in (51, 52, 53))
    Bm, Cm = (randn((b, n, L), seed=s).cuda() for s in (54, 55))
    A = -torch.exp(randn((d, n), seed=56, dtype=torch.float32)).cuda()
    D = randn((d,), seed=57, dtype=torch.float32).cuda()
    bias = randn((d,), seed=58, dtype=torch.float32).cuda()

    def step():
        return ops.selective_scan(u, dr, A, Bm, Cm, D, z, bias)

    graph, y_g = _capture(step)
    for r in range(REPLAYS):
        u.copy_(randn(u.shape, seed=400 + r).cuda())
        graph.replay()
        y_e = step()
        torch.cuda.synchronize()
        assert _same(y_g, y_e), f"replay {r}: y differs from the eager call"
