"""GPU parity of the Mamba-1 selective scan against the fp64 oracle.

|y| reaches ~150 for the config-4 distributions, where half a bf16 ulp
alone exceeds 2e-2, so the criterion is |a - b| <= 2e-2 * max(1, |ref|)
against the oracle's fp64 result rounded to bf16 (both sides are bf16).
"""

import ctypes

import numpy as np
import pytest
import torch

from helpers import bits, randn, steady_scan_table, to_f32
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def scan_inputs(b, d, L, n=16, seed=0, with_bias=True):
    u = randn((b, d, L), seed=seed)
    dr = randn((b, d, L), seed=seed + 1)
    z = randn((b, d, L), seed=seed + 2)
    Bm = randn((b, n, L), seed=seed + 3)
    Cm = randn((b, n, L), seed=seed + 4)
    A = -torch.exp(randn((d, n), seed=seed + 5, dtype=torch.float32))
    D = randn((d,), seed=seed + 6, dtype=torch.float32)
    bias = randn((d,), seed=seed + 7, dtype=torch.float32) if with_bias else None
    return u, dr, A, Bm, Cm, D, z, bias


def _check(y_gpu, ins, chan=None):
    u, dr, A, Bm, Cm, D, z, bias = ins
    if chan is not None:
        u, dr, z = u[:, chan], dr[:, chan], z[:, chan]
        A, D = A[chan], D[chan]
        bias = None if bias is None else bias[chan]
        y_gpu = y_gpu[:, chan]
    ref_bits, ref64 = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm),
                                            D.numpy(), bits(z),
                                            None if bias is None else bias.numpy())
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y_gpu).astype(np.float64)
    assert np.isfinite(got).all()
    bound = 2e-2 * np.maximum(1.0, np.abs(ref))
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], np.abs(got - ref).max())


@pytest.mark.parametrize("b,d,L,bias", [(2, 64, 300, True), (1, 40, 64, False), (2, 96, 1024, True)])
def test_scan_small_matches_oracle(ops, b, d, L, bias):
    _log(f"case: scan small b={b} d={d} L={L} bias={bias}")
    ins = scan_inputs(b, d, L, with_bias=bias)
    y = ops.selective_scan(*(t.cuda() if t is not None else None for t in ins))
    torch.cuda.synchronize()
    _check(y, ins)


def test_scan_pair_loads_equal_16bit_loads(ops):
    """B and C taken as 4-byte step pairs (aligned inputs) and as 16-bit
    values (B two bytes past a 4-byte boundary) give the same bits. The
    shape has 1024 channel blocks, so both launches take the single pass."""
    _log("case: scan pair loads against 16-bit loads b=4 d=4096 L=96")
    u, dr, A, Bm, Cm, D, z, bias = (t.cuda() for t in scan_inputs(4, 4096, 96))
    y_pairs = ops.selective_scan(u, dr, A, Bm, Cm, D, z, bias)
    buf = torch.empty(Bm.numel() + 1, dtype=Bm.dtype, device=Bm.device)
    b_odd = buf[1:].view(Bm.shape)
    b_odd.copy_(Bm)
    assert b_odd.data_ptr() % 4 == 2
    y_16 = ops.selective_scan(u, dr, A, b_odd, Cm, D, z, bias)
    torch.cuda.synchronize()
    assert torch.equal(y_pairs.view(torch.int16), y_16.view(torch.int16))


def test_scan_no_gate_no_D(ops):
    _log("case: scan without z and D")
    u, dr, A, Bm, Cm, D, z, bias = scan_inputs(1, 32, 256)
    y = ops.selective_scan(u.cuda(), dr.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), None, None,
                           bias.cuda())
    torch.cuda.synchronize()
    ref_bits, _ = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm), None,
                                        None, bias.numpy())
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y).astype(np.float64)
    assert (np.abs(got - ref) <= 2e-2 * np.maximum(1.0, np.abs(ref))).all()


def test_config4_full_shape(ops):
    """B=4 L=2048 d_inner=5120 d_state=16; sampled
    channels (every channel is an independent recurrence) against the oracle."""
    _log("case: config4 full shape")
    ins = scan_inputs(4, 5120, 2048, seed=100)
    y = ops.selective_scan(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    chan = torch.tensor([0, 1, 2, 777, 2048, 4095, 5000, 5119])
    _check(y.cpu(), ins, chan)


# config 4 (the single pass) and a few channels over a long sequence (the
# sequence-parallel path: 320 chunks, the wave-parallel carry)
FULL_SHAPES = [(4, 5120, 2048), (1, 64, 65536)]


@pytest.mark.parametrize("shape", FULL_SHAPES, ids=["config4", "b1d64L65536"])
def test_scan_full_size_linear_in_u(ops, shape):
    """Every channel: y(2u) = 2 y(u) bit for bit. u enters the
    recurrence, the skip term and nothing else, each time through products
    and sums that doubling commutes with exactly in fp32 and in the bf16
    rounding of y (no value here is near the subnormal range), so any
    channel, state or step whose mapping differs between the two calls, or
    an input read out of place, breaks the equality."""
    _log(f"case: scan linear in u, shape {shape}")
    u, dr, A, Bm, Cm, D, z, bias = scan_inputs(*shape, seed=300)
    dev = [t.cuda() if t is not None else None for t in (u, dr, A, Bm, Cm, D, z, bias)]
    y1 = ops.selective_scan(*dev)
    dev[0] = (2 * u).cuda()
    y2 = ops.selective_scan(*dev)
    torch.cuda.synchronize()
    y1, y2 = y1.cpu(), y2.cpu()
    assert torch.isfinite(y1.float()).all()
    diff = (bits(y2) != bits(2 * y1))
    assert not diff.any(), (np.argwhere(diff)[:5], int(diff.sum()))


@pytest.mark.parametrize("shape", FULL_SHAPES, ids=["config4", "b1d64L65536"])
@pytest.mark.parametrize("case", ["B zero", "C zero", "delta zero"])
def test_scan_full_size_skip_term_only(ops, case, shape):
    """Every channel, where the state term vanishes: with B = 0
    the state stays 0, with C = 0 it is not read, and with delta = 0 (no
    softplus, no bias) the state gains nothing. Then y = D u silu(z), within
    one bf16 ulp of that product in fp32 (the kernel forms D u as
    (D log2 e)(u ln2) and silu through the hardware reciprocal)."""
    _log(f"case: scan skip term only, {case}, shape {shape}")
    u, dr, A, Bm, Cm, D, z, bias = scan_inputs(*shape, seed=400)
    softplus = True
    if case == "B zero":
        Bm = torch.zeros_like(Bm)
    elif case == "C zero":
        Cm = torch.zeros_like(Cm)
    else:
        dr, bias, softplus = torch.zeros_like(dr), None, False
    y = ops.selective_scan(*(t.cuda() if t is not None else None
                             for t in (u, dr, A, Bm, Cm, D, z, bias)),
                           delta_softplus=softplus)
    torch.cuda.synchronize()
    zf = z.float()
    want = D.view(1, -1, 1) * u.float() * (zf * torch.sigmoid(zf))
    got = y.cpu().float()
    # one bf16 ulp of the result (8 significant bits), plus the smallest
    # normal step for results near 0
    ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(2.0 ** -120))) - 7)
    err = (got - want).abs()
    assert (err <= ulp).all(), (float(err.max()), int((err > ulp).sum()))


def _chunked(b, d, L):
    """Whether the library takes the sequence-parallel path for this shape
    (the rule of scan_chunking in scan.hip: fewer than 1024 work-groups of 16
    channels, an even length and at least two 64-step chunks)."""
    groups = -(-d // 16) * b
    return L % 2 == 0 and groups < 1024 and L >= 128


@pytest.mark.parametrize("b,d,L,bias,gate", [
    (1, 64, 65536, True, True),    # 4 channel blocks over a long sequence: 320 chunks
    (2, 20, 9000, True, True),     # 140 chunks: the wave carry's two full passes and a part
    (1, 16, 4096, False, True),    # one channel block, 64 chunks of 64 steps
    (2, 48, 1000, True, False),    # ragged channel block, chunks of 96, 64 and 72 steps
    (1, 8, 130, True, True),       # two chunks, the second 66 steps
])
def test_scan_sequence_parallel_matches_oracle(ops, b, d, L, bias, gate):
    """The chunked path (state pass, carry pass, output pass, with y as the
    scratch of the chunk carries) against the fp64 sequential oracle."""
    assert _chunked(b, d, L)
    _log(f"case: scan chunked b={b} d={d} L={L} bias={bias} gate={gate}")
    u, dr, A, Bm, Cm, D, z, bias_t = scan_inputs(b, d, L, seed=200 + L, with_bias=bias)
    y = ops.selective_scan(u.cuda(), dr.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), D.cuda(),
                           z.cuda() if gate else None,
                           bias_t.cuda() if bias_t is not None else None)
    torch.cuda.synchronize()
    ref_bits, _ = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm),
                                        D.numpy(), bits(z) if gate else None,
                                        None if bias_t is None else bias_t.numpy())
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y).astype(np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref) > 2e-2 * np.maximum(1.0, np.abs(ref))
    assert not bad.any(), (np.argwhere(bad)[:5], np.abs(got - ref).max())


@pytest.mark.parametrize("b,d,L", [(1, 32, 129), (4, 4096, 256), (2, 64, 126)])
def test_scan_single_pass_matches_oracle(ops, b, d, L):
    """Shapes the single pass keeps: an odd length, enough channel blocks to
    fill the GPU, and a sequence too short for two chunks."""
    assert not _chunked(b, d, L)
    _log(f"case: scan single pass b={b} d={d} L={L}")
    ins = scan_inputs(b, d, L, seed=300 + L)
    y = ops.selective_scan(*(t.cuda() for t in ins))
    torch.cuda.synchronize()
    _check(y, ins)


def test_scan_chunked_repeated_call_is_identical(ops):
    """y serves as the chunked path's scratch: a second call into the same
    buffer (holding the first call's outputs) gives bit-identical results."""
    _log("case: scan chunked repeat")
    ins = [t.cuda() for t in scan_inputs(1, 32, 2048, seed=9)]
    y1 = ops.selective_scan(*ins)
    y2 = ops.selective_scan(*ins)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("softplus", [True, False])
@pytest.mark.parametrize("b,d,L", [(2, 40, 301), (1, 32, 4096)])
def test_scan_softplus_branches(ops, b, d, L, softplus):
    """Softplus on: delta_raw + bias spread over [-30, 30], so both the
    threshold branch (delta = the input above 20) and the exp / log branch
    run. Softplus off: a positive delta_raw + bias feeds delta directly. The
    first shape takes the single pass, the second the chunked path (whose
    state pass computes delta on its own)."""
    assert _chunked(b, d, L) == (L == 4096)
    _log(f"case: scan softplus={softplus} b={b} d={d} L={L}")
    u, dr, A, Bm, Cm, D, z, bias = scan_inputs(b, d, L, seed=700 + L)
    g = torch.Generator().manual_seed(710 + L)
    if softplus:
        dr = (torch.rand((b, d, L), generator=g) * 60.0 - 30.0).to(torch.bfloat16)
    else:
        dr = (torch.rand((b, d, L), generator=g) * 0.5 + 0.01).to(torch.bfloat16)
        bias = torch.rand((d,), generator=g) * 0.1
    y = ops.selective_scan(u.cuda(), dr.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), D.cuda(),
                           z.cuda(), bias.cuda(), delta_softplus=softplus)
    torch.cuda.synchronize()
    ref_bits, _ = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm),
                                        D.numpy(), bits(z), bias.numpy(), softplus=softplus)
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y).astype(np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref) > 2e-2 * np.maximum(1.0, np.abs(ref))
    assert not bad.any(), (np.argwhere(bad)[:5], np.abs(got - ref).max())


@pytest.mark.parametrize("L", [(1 << 26) - 2, (1 << 26) - 1])
def test_scan_longest_sequence_closed_form(L):
    """seq_len just below the 2^26 limit, where a 16-channel block spans
    nearly 2^31 bytes of the kernels' 32-bit offsets: the even length takes
    the chunked path (about 1280 chunks), the odd one the single pass (one
    work-group walking the whole sequence). The inputs have a closed form:
    delta = 0.5 (softplus off), A = -1, B = C = 1, no D, no gate, and
    u[c, t] = ((5 t + c) mod 9) - 4, so y[c, t] = 16 x_t of the recurrence in
    helpers.steady_scan_table, which after 200 steps (e^-100 of the start left) is
    periodic in t with a phase set by the channel. y starts as NaN, so an
    output stored in the wrong place, or not stored, fails. The oracle is not
    run: 2^26 steps of 256 recurrences is too long for it."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import _abi
    d, n, warm = 16, 16, 200
    _log(f"case: scan closed form d={d} L={L} ({'chunked' if _chunked(1, d, L) else 'single pass'})")
    dev = "cuda"
    t = torch.arange(L, device=dev, dtype=torch.int32)
    u = torch.empty((1, d, L), dtype=torch.bfloat16, device=dev)
    for c in range(d):
        u[0, c] = ((5 * t + c) % 9 - 4).to(torch.bfloat16)
    dr = torch.full((1, d, L), 0.5, dtype=torch.bfloat16, device=dev)
    Bm = torch.ones((1, n, L), dtype=torch.bfloat16, device=dev)
    Cm = torch.ones((1, n, L), dtype=torch.bfloat16, device=dev)
    A = torch.full((d, n), -1.0, dtype=torch.float32, device=dev)
    y = torch.full((1, d, L), float("nan"), dtype=torch.bfloat16, device=dev)
    lib = _abi.load_library()
    desc = _abi.ScanDesc(1, d, L, n, _abi.DTYPE_BF16, 0)
    _abi.check(lib.neptune_selective_scan_fwd(
        ctypes.byref(desc), u.data_ptr(), dr.data_ptr(), A.data_ptr(), Bm.data_ptr(), Cm.data_ptr(), None, None,
        None, y.data_ptr(), torch.cuda.current_stream().cuda_stream), lib)
    torch.cuda.synchronize()
    del u, dr, Bm, Cm
    head, period = steady_scan_table(d, warm)
    phase = (t[warm:] - warm) % 9
    for c in range(d):
        got = y[0, c].float()
        want = torch.empty(L, dtype=torch.float32, device=dev)
        want[:warm] = torch.from_numpy(head[c]).float().to(dev)
        want[warm:] = torch.from_numpy(period[c]).float().to(dev)[phase.long()]
        assert bool(torch.isfinite(got).all()), f"channel {c}: an output was not stored"
        err = (got - want).abs()
        bad = err > 2e-2 * want.abs().clamp(min=1.0)
        assert not bool(bad.any()), (c, int(bad.nonzero()[0]), float(err.max()))
