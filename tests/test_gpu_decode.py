"""GPU parity of split-K GQA decode (bf16 and fp8-E4M3 KV) and of the fp8
KV quantiser, against the CPU oracle on the same inputs.

Decode outputs of N(0,1) data are ~0.03 in magnitude, so besides the
contract's max-abs bounds (2e-2 bf16, 6e-2 fp8) each case also holds every
sequence to max|a-b| <= 2e-2 * max|ref| against the oracle on the same K/V
(bf16 values or fp8 codes) and, for fp8 KV end to end against the oracle on
the bf16 K/V, to 6e-2 * max|ref|.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_BF16_REL, TOL_FP8_ABS, TOL_FP8_REL, TOL_LSE_ABS,
                     assert_rel_rows, bits, from_bf16_bits, max_abs, periodic_attention,
                     periodic_k0, periodic_k127, periodic_vper, randn, to_f32)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def _check_bf16(got, lse, q, k, v, splits):
    ref_o, ref_lse, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16,
                                             num_splits=splits)
    ref = oracle.decode(ref_o, oracle.BF16)
    err = max_abs(to_f32(got), ref)
    assert err <= TOL_BF16_ABS
    assert_rel_rows(to_f32(got), ref, TOL_BF16_REL, "bf16 decode vs oracle")
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS


@pytest.mark.parametrize("B,Hq,Hk,L,splits", [
    (2, 8, 2, 1000, 3),     # ragged tail, GQA 4
    (1, 4, 4, 256, 1),      # MHA, one split
    (3, 16, 1, 4097, 0),    # MQA 16, library-chosen splits
    (2, 32, 8, 2048, 16),   # config-3 head layout, short cache
])
def test_decode_bf16_matches_oracle(ops, B, Hq, Hk, L, splits):
    _log(f"case: decode bf16 B={B} Hq={Hq} Hk={Hk} L={L} splits={splits}")
    q = randn((B, Hq, 128), seed=1)
    k = randn((B, Hk, L, 128), seed=2)
    v = randn((B, Hk, L, 128), seed=3)
    o, lse = ops.decode_splitk(q.cuda(), k.cuda(), v.cuda(), num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    _check_bf16(o, lse, q, k, v, splits)


def test_decode_split_invariance(ops):
    """splits = 1 and splits = 16 agree (the combine is exact up to rounding)."""
    _log("case: decode split invariance")
    q = randn((2, 8, 128), seed=4).cuda()
    k = randn((2, 2, 4096, 128), seed=5).cuda()
    v = randn((2, 2, 4096, 128), seed=6).cuda()
    o1 = ops.decode_splitk(q, k, v, num_splits=1)
    o16 = ops.decode_splitk(q, k, v, num_splits=16)
    torch.cuda.synchronize()
    assert max_abs(to_f32(o1), to_f32(o16)) <= 2e-3


def test_decode_gqa_equals_repeated_mha(ops):
    _log("case: decode gqa == repeated mha")
    q = randn((2, 8, 128), seed=7).cuda()
    k = randn((2, 2, 640, 128), seed=8).cuda()
    v = randn((2, 2, 640, 128), seed=9).cuda()
    o_gqa = ops.decode_splitk(q, k, v, num_splits=2)
    o_mha = ops.decode_splitk(q, k.repeat_interleave(4, dim=1).contiguous(),
                              v.repeat_interleave(4, dim=1).contiguous(), num_splits=2)
    torch.cuda.synchronize()
    assert torch.equal(o_gqa, o_mha)


def test_config3_full_shape(ops):
    """B=16 Hq=32 Hkv=8 L=32768 D=128, 16 splits, N(0,1).
    Sampled (batch, kv head) groups against the oracle."""
    _log("case: config3 full shape")
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((16, 32, 128), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    o, lse = ops.decode_splitk(q, k, v, num_splits=16, return_lse=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    for b, hk in ((0, 0), (15, 7), (9, 3)):
        qs = q[b:b + 1, 4 * hk:4 * hk + 4].cpu()
        _check_bf16(o[b:b + 1, 4 * hk:4 * hk + 4], lse[b:b + 1, 4 * hk:4 * hk + 4], qs,
                    k[b:b + 1, hk:hk + 1].cpu(), v[b:b + 1, hk:hk + 1].cpu(), 16)


@pytest.mark.parametrize("L,sb", [(1000, 64), (4096, 64), (512, 128)])
def test_kv_quantize_bit_exact(ops, L, sb):
    _log(f"case: kv quantize L={L} sb={sb}")
    kv = randn((2, 3, L, 128), seed=11)
    kv[0, 1, :sb] = 0  # an all-zero block: scale 0, codes 0
    codes, scales = ops.kv_quantize_fp8(kv.cuda(), scale_block=sb)
    torch.cuda.synchronize()
    ref_codes, ref_scales = oracle.kv_quantize_fp8(bits(kv), sb)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


def test_kv_quantize_every_bf16_value(ops):
    """Every finite bf16 value of magnitude <= 448, both signs (ties, the
    E4M3 subnormal range and signed zeros included), quantised with a block
    scale of exactly 1 (each 64 x 128 block opens with 448): the codes must
    equal the oracle's encoder bit for bit."""
    _log("case: kv quantize exhaustive bf16")
    pos = np.arange(0x0000, 0x43E1, dtype=np.uint16)
    vals = np.concatenate([pos, pos | 0x8000])
    per = 64 * 128 - 1
    nblk = -(-vals.size // per)
    flat = np.zeros(nblk * (per + 1), dtype=np.uint16)
    for i in range(nblk):
        chunk = vals[i * per:(i + 1) * per]
        flat[i * (per + 1)] = 0x43E0
        flat[i * (per + 1) + 1:i * (per + 1) + 1 + chunk.size] = chunk
    src = flat.reshape(1, 1, nblk * 64, 128)
    kv = from_bf16_bits(src)
    codes, scales = ops.kv_quantize_fp8(kv.cuda(), scale_block=64)
    torch.cuda.synchronize()
    ref_codes, ref_scales = oracle.kv_quantize_fp8(src, 64)
    assert (ref_scales == 1.0).all()
    got = codes.cpu().numpy()
    bad = np.flatnonzero(got != ref_codes)
    assert bad.size == 0, [(hex(src.ravel()[i]), hex(got.ravel()[i]), hex(ref_codes.ravel()[i]))
                           for i in bad[:8]]
    assert np.array_equal(scales.cpu().numpy(), ref_scales)


def test_kv_quantize_general_path(ops):
    """head_dim 100 (not a multiple of 8) takes the element-wise kernel."""
    _log("case: kv quantize head_dim 100")
    kv = randn((1, 2, 300, 100), seed=13)
    codes, scales = ops.kv_quantize_fp8(kv.cuda(), scale_block=64)
    torch.cuda.synchronize()
    ref_codes, ref_scales = oracle.kv_quantize_fp8(bits(kv), 64)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy(), ref_scales)


@pytest.mark.parametrize("B,Hq,Hk,L,splits", [(2, 8, 2, 1000, 3), (2, 32, 8, 2048, 16)])
def test_decode_fp8_matches_oracle(ops, B, Hq, Hk, L, splits):
    _log(f"case: decode fp8 B={B} Hq={Hq} Hk={Hk} L={L} splits={splits}")
    q = randn((B, Hq, 128), seed=12)
    k = randn((B, Hk, L, 128), seed=13)
    v = randn((B, Hk, L, 128), seed=14)
    kc, ks = ops.kv_quantize_fp8(k.cuda())
    vc, vs = ops.kv_quantize_fp8(v.cuda())
    o, lse = ops.decode_splitk(q.cuda(), kc, vc, k_scale=ks, v_scale=vs, num_splits=splits,
                               return_lse=True)
    torch.cuda.synchronize()
    got = to_f32(o)
    # kernel error alone: oracle on the same codes and scales
    ref_o, ref_lse, _ = oracle.decode_splitk(bits(q), kc.cpu().numpy(), vc.cpu().numpy(),
                                             oracle.FP8, ks.cpu().numpy(), vs.cpu().numpy(),
                                             num_splits=splits)
    ref = oracle.decode(ref_o, oracle.BF16)
    assert max_abs(got, ref) <= TOL_FP8_ABS
    assert_rel_rows(got, ref, TOL_BF16_REL, "fp8 decode vs oracle on the same codes")
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS
    # end to end against bf16 KV (quantisation error included)
    ref_bf, _, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16, num_splits=splits)
    ref_bf = oracle.decode(ref_bf, oracle.BF16)
    assert max_abs(got, ref_bf) <= TOL_FP8_ABS
    assert_rel_rows(got, ref_bf, TOL_FP8_REL, "fp8 decode vs oracle on bf16 KV")


def test_config5_full_shape(ops):
    """config 3 with E4M3 KV and per-(b, kv head, 64-token)
    scales; sampled groups against the oracle on the same codes."""
    _log("case: config5 full shape")
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((16, 32, 128), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    kc, ks = ops.kv_quantize_fp8(k)
    del k
    v = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    vc, vs = ops.kv_quantize_fp8(v)
    del v
    o = ops.decode_splitk(q, kc, vc, k_scale=ks, v_scale=vs, num_splits=16)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    for b, hk in ((0, 0), (15, 7)):
        sl = (slice(b, b + 1), slice(hk, hk + 1))
        ref_o, _, _ = oracle.decode_splitk(
            bits(q[b:b + 1, 4 * hk:4 * hk + 4]), kc[sl].cpu().numpy(), vc[sl].cpu().numpy(),
            oracle.FP8, ks[sl].cpu().numpy(), vs[sl].cpu().numpy(), num_splits=16)
        ref = oracle.decode(ref_o, oracle.BF16)
        got = to_f32(o[b:b + 1, 4 * hk:4 * hk + 4])
        assert max_abs(got, ref) <= TOL_FP8_ABS
        assert_rel_rows(got, ref, TOL_BF16_REL, f"config5 (b, hk) = {(b, hk)} vs same codes")


@pytest.mark.parametrize("fp8", [False, True], ids=["config3", "config5"])
def test_full_shape_linear_in_v(ops, fp8):
    """Configs 3 and 5 at full size, every (batch, query head): O(2V) = 2 O(V)
    bit for bit and the same LSE. The split maxima, sums and combine weights
    do not depend on V, and doubling V doubles every product and partial sum
    exactly. With fp8 KV the quantiser keeps the codes of 2V and doubles
    their scales (amax / 448 commutes with doubling), checked first."""
    _log(f"case: decode linear in V, fp8={fp8}")
    g = torch.Generator(device="cuda").manual_seed(31)
    q = torch.randn((16, 32, 128), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((16, 8, 32768, 128), device="cuda", generator=g).to(torch.bfloat16)
    if fp8:
        kc, ks = ops.kv_quantize_fp8(k)
        vc, vs = ops.kv_quantize_fp8(v)
        vc2, vs2 = ops.kv_quantize_fp8(2 * v)
        del k, v
        assert torch.equal(vc2, vc)
        assert torch.equal(vs2, 2 * vs)
        o1, lse1 = ops.decode_splitk(q, kc, vc, k_scale=ks, v_scale=vs, num_splits=16,
                                     return_lse=True)
        o2, lse2 = ops.decode_splitk(q, kc, vc2, k_scale=ks, v_scale=vs2, num_splits=16,
                                     return_lse=True)
    else:
        o1, lse1 = ops.decode_splitk(q, k, v, num_splits=16, return_lse=True)
        o2, lse2 = ops.decode_splitk(q, k, 2 * v, num_splits=16, return_lse=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o1).all())
    assert torch.equal(lse1, lse2)
    assert torch.equal(o2, 2 * o1)


def test_workspace_too_small(ops):
    from neptune_hip import NeptuneWorkspaceTooSmall
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 1, 256, 128), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(NeptuneWorkspaceTooSmall):
        ops.decode_splitk(q, k, k, workspace=ws)


def test_strided_workspace_raises(ops):
    """The library writes the workspace's numel * element_size bytes from its
    first element, so a strided view is refused before any launch."""
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 1, 256, 128), dtype=torch.bfloat16, device="cuda")
    n = ops.decode_workspace_bytes(q, k)
    ws = torch.empty(2 * n, dtype=torch.uint8, device="cuda")[::2]
    with pytest.raises(ValueError):
        ops.decode_splitk(q, k, k, workspace=ws)



SEG_STEP = 4.0  # V's step per 2^24 tokens (4 GiB of 256-byte rows)


def _periodic_kv_rows(t0, t1, dev):
    """K and V rows [t1 - t0, 128] bf16 of tokens t0 .. t1 - 1 for the
    closed-form decode tests: K's head_dim rows 0 and 127 and V periodic in
    the token index (helpers.periodic_*), V stepped by SEG_STEP every 2^24
    tokens, K's other rows a period-11 pattern the queries do not see."""
    D = 128
    dcol = torch.arange(D, device=dev, dtype=torch.int32)
    j = torch.arange(t0, t1, device=dev, dtype=torch.int32)
    jm = j % 35
    krows = (jm[:, None] + dcol[None, :]) % 11 - 5
    krows[:, 0] = periodic_k0(jm)
    krows[:, D - 1] = periodic_k127(jm)
    vrows = periodic_vper(jm[:, None], dcol[None, :]) + int(SEG_STEP) * (j >> 24)[:, None]
    return krows.to(torch.bfloat16), vrows.to(torch.bfloat16)


def _periodic_queries(q0, dev):
    q = torch.zeros((1, len(q0), 128), dtype=torch.bfloat16, device=dev)
    q[0, :, 0] = torch.tensor(q0, dtype=torch.bfloat16)
    q[0, :, 127] = torch.tensor(q0, dtype=torch.bfloat16)
    return q


def _check_periodic(o, lse, q0, L):
    want_o, want_lse = periodic_attention(q0, L, 1.0 / np.sqrt(128), seg_shift=SEG_STEP)
    got_o, got_lse = to_f32(o)[0], to_f32(lse)[0]
    assert np.isfinite(got_o).all()
    err = np.abs(got_o - want_o)
    assert (err <= TOL_BF16_ABS * np.maximum(1.0, np.abs(want_o))).all(), err.max()
    assert max_abs(got_lse, want_lse) <= TOL_LSE_ABS, (got_lse, want_lse)


def test_decode_16gib_head_closed_form(ops):
    """One KV head of 2^26 + 37 tokens (16 GiB each for K and V, past every
    32-bit byte offset) read by a GQA group of four query heads over 1024
    splits. Query head h is q0[h] (e_0 + e_127); K's head_dim rows 0 and 127
    and V are periodic in the token index with period 35 (coprime to the
    32-token step), V steps up every 2^24 tokens (every 4 GiB), K's other
    rows carry a pattern q does not see, so O and the LSE have the closed
    form of helpers.periodic_attention (P's bf16 rounding included; each
    split's own running max changes that rounding by a relative 2^-8 at
    most). A token read from the wrong place changes the pairing of scores
    and values, and one read 4 GiB low loses a step; either fails. The
    oracle is not run over 67M tokens."""
    L, D, q0 = (1 << 26) + 37, 128, [2.0, 4.0, 6.0, 8.0]
    _log(f"case: decode bf16 closed form L={L} Hq=4 Hkv=1 splits=1024")
    dev = "cuda"
    k = torch.empty((1, 1, L, D), dtype=torch.bfloat16, device=dev)
    v = torch.empty((1, 1, L, D), dtype=torch.bfloat16, device=dev)
    step = 1 << 21
    for t0 in range(0, L, step):
        t1 = min(t0 + step, L)
        k[0, 0, t0:t1], v[0, 0, t0:t1] = _periodic_kv_rows(t0, t1, dev)
    o, lse = ops.decode_splitk(_periodic_queries(q0, dev), k, v, num_splits=1024, return_lse=True)
    torch.cuda.synchronize()
    _check_periodic(o, lse, q0, L)


def test_decode_max_splits_closed_form(ops):
    """The largest split count the library accepts, 16384: the combine then
    holds one fp32 weight per split in 64 KiB of LDS. One KV head of
    16384 x 64 tokens (the periodic K and V of the test above, 256 MiB each)
    in 16384 one-block splits, read by a GQA group of four query heads,
    against the closed form; the same call with 16 splits agrees with it."""
    L, q0 = 16384 * 64, [2.0, 4.0, 6.0, 8.0]
    _log(f"case: decode bf16 closed form L={L} Hq=4 Hkv=1 splits=16384")
    dev = "cuda"
    kr, vr = _periodic_kv_rows(0, L, dev)
    k, v = kr.view(1, 1, L, 128), vr.view(1, 1, L, 128)
    q = _periodic_queries(q0, dev)
    for splits in (16384, 16):
        o, lse = ops.decode_splitk(q, k, v, num_splits=splits, return_lse=True)
        torch.cuda.synchronize()
        _check_periodic(o, lse, q0, L)


def test_decode_paged_16gib_pool_closed_form(ops):
    """The same 2^26 + 37 tokens in a pool of 64-token pages (16 GiB for K,
    16 for V), logical page i stored at page (i + 12345) mod pages: page
    bases lie past every 32-bit byte offset, the block table is not the
    identity, and the last page is partly filled. A page base that wrapped at
    4 GiB would read the pages 2^24 tokens earlier, a step lower in V."""
    L, D, q0, P = (1 << 26) + 37, 128, [2.0, 4.0, 6.0, 8.0], 64
    npages = -(-L // P)
    _log(f"case: decode paged bf16 closed form L={L} pages={npages} rotated")
    dev = "cuda"
    perm = (torch.arange(npages, device=dev) + 12345) % npages
    kp = torch.zeros((npages, 1, P, D), dtype=torch.bfloat16, device=dev)
    vp = torch.zeros((npages, 1, P, D), dtype=torch.bfloat16, device=dev)
    step = 1 << 15  # pages per fill
    for p0 in range(0, npages, step):
        p1 = min(p0 + step, npages)
        t1 = min(p1 * P, L)
        kr, vr = _periodic_kv_rows(p0 * P, t1, dev)
        pad = p1 * P - t1
        if pad:
            kr = torch.cat([kr, torch.zeros((pad, D), dtype=kr.dtype, device=dev)])
            vr = torch.cat([vr, torch.zeros((pad, D), dtype=vr.dtype, device=dev)])
        kp[perm[p0:p1]] = kr.view(p1 - p0, 1, P, D)
        vp[perm[p0:p1]] = vr.view(p1 - p0, 1, P, D)
    table = perm.to(torch.int32)[None]
    lens = torch.tensor([L], dtype=torch.int32, device=dev)
    o, lse = ops.decode_paged(_periodic_queries(q0, dev), kp, vp, table, lens, num_splits=1024,
                              return_lse=True)
    torch.cuda.synchronize()
    _check_periodic(o, lse, q0, L)
