"""GPU parity of split-K GQA decode (bf16 and fp8-E4M3 KV) and of the fp8
KV quantiser, against the CPU oracle on the same inputs.

Decode outputs of N(0,1) data are ~0.03 in magnitude, so besides the
contract's max-abs bounds (2e-2 bf16, 6e-2 fp8) each case also checks
max|a-b| <= 2e-2 * max|ref| (bf16) / 6e-2 * max|ref| (fp8 vs the oracle on
the same codes).
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_FP8_ABS, TOL_LSE_ABS, bits, from_bf16_bits, max_abs,
                     randn, to_f32)

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
    assert err <= 2e-2 * np.abs(ref).max()
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
    assert max_abs(got, ref) <= 6e-2 * np.abs(ref).max()
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS
    # end to end against bf16 KV (quantisation error included)
    ref_bf, _, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16, num_splits=splits)
    assert max_abs(got, oracle.decode(ref_bf, oracle.BF16)) <= TOL_FP8_ABS


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
        assert max_abs(got, ref) <= 6e-2 * np.abs(ref).max()


def test_workspace_too_small(ops):
    from neptune_hip import NeptuneWorkspaceTooSmall
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 1, 256, 128), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(NeptuneWorkspaceTooSmall):
        ops.decode_splitk(q, k, k, workspace=ws)
