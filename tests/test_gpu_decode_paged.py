"""GPU parity of split-K decode over a paged KV cache (neptune_decode_paged).

* With every sequence at the full length, paged decode over a shuffled page
  pool equals contiguous decode of the same tokens bit for bit (same kernel
  arithmetic, only the addressing differs), for both pool layouts
  ([pages, Hkv, page, D] and [pages, page, Hkv, D] seen through a view).
* Ragged lengths: each sequence against the oracle on its own tokens, and
  the whole batch against the oracle's paged twin (same split layout).
* A zero-length sequence gives O = 0 and lse = -inf; block-table entries
  outside the pool are clamped by the kernel exactly as by the twin.
* fp8 pools (neptune_decode_paged_fp8, one scale per page and kv head):
  bit for bit equal to the contiguous fp8 decode whose scale block is the
  page, for both pool layouts; ragged, empty and out-of-pool cases against
  the oracle's fp8 paged twin.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_BF16_REL, TOL_FP8_ABS, TOL_LSE_ABS, assert_rel_rows, bits,
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


def paginate(kv, ps, seed, token_major=False, spare=3):
    """Scatter contiguous [B, Hk, L, D] into a shuffled page pool. Returns the
    pool view [pages, Hk, ps, D] and the block table [B, L / ps]."""
    B, Hk, L, D = kv.shape
    per = -(-L // ps)
    npages = B * per + spare
    g = torch.Generator().manual_seed(seed)
    ids = torch.randperm(npages, generator=g)[: B * per].view(B, per).to(torch.int32)
    if token_major:
        pool = torch.zeros((npages, ps, Hk, D), dtype=kv.dtype)
    else:
        pool = torch.zeros((npages, Hk, ps, D), dtype=kv.dtype)
    for b in range(B):
        for j in range(per):
            blk = kv[b, :, j * ps:(j + 1) * ps]
            n = blk.shape[1]
            if token_major:
                pool[ids[b, j], :n] = blk.transpose(0, 1)
            else:
                pool[ids[b, j], :, :n] = blk
    pool = pool.cuda()
    view = pool.permute(0, 2, 1, 3) if token_major else pool
    return view, ids.cuda()


@pytest.mark.parametrize("token_major", [False, True])
def test_paged_equals_contiguous_bitwise(ops, token_major):
    _log(f"case: paged == contiguous, token_major={token_major}")
    B, Hq, Hk, L, D, ps, splits = 2, 8, 2, 1024, 128, 64, 5
    q = randn((B, Hq, D), seed=20).cuda()
    k, v = randn((B, Hk, L, D), seed=21), randn((B, Hk, L, D), seed=22)
    kp, table = paginate(k, ps, seed=23, token_major=token_major)
    vp, _ = paginate(v, ps, seed=23, token_major=token_major)
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    o_ref, lse_ref = ops.decode_splitk(q, k.cuda(), v.cuda(), num_splits=splits, return_lse=True)
    o, lse = ops.decode_paged(q, kp, vp, table, lens, max_seq_len=L, num_splits=splits,
                              return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse, lse_ref)


@pytest.mark.parametrize("token_major", [False, True])
def test_paged_equals_contiguous_config3_full_size(ops, token_major):
    """Config 3 at full size (B=16 Hq=32 Hkv=8 L=32768 D=128, 16 splits) in
    64-token pages, shuffled over the pool on the device: every (batch,
    query head) bit-identical to the contiguous kernel, output and LSE."""
    _log(f"case: paged == contiguous at config 3, token_major={token_major}")
    B, Hq, Hk, L, D, ps = 16, 32, 8, 32768, 128, 64
    per = L // ps
    g = torch.Generator(device="cuda").manual_seed(41)
    q = torch.randn((B, Hq, D), device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn((B, Hk, L, D), device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn((B, Hk, L, D), device="cuda", generator=g).to(torch.bfloat16)
    ids = torch.randperm(B * per, device="cuda", generator=g)
    table = ids.view(B, per).to(torch.int32)

    def pool_of(kv):
        blocks = kv.view(B, Hk, per, ps, D).permute(0, 2, 1, 3, 4)  # [B, per, Hk, ps, D]
        if token_major:
            blocks = blocks.transpose(2, 3)                          # [B, per, ps, Hk, D]
        pool = torch.empty((B * per,) + tuple(blocks.shape[2:]), dtype=kv.dtype, device="cuda")
        pool[ids] = blocks.reshape((B * per,) + tuple(blocks.shape[2:]))
        return pool.permute(0, 2, 1, 3) if token_major else pool

    kp, vp = pool_of(k), pool_of(v)
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    o_ref, lse_ref = ops.decode_splitk(q, k, v, num_splits=16, return_lse=True)
    o, lse = ops.decode_paged(q, kp, vp, table, lens, max_seq_len=L, num_splits=16,
                              return_lse=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o_ref).all())
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse, lse_ref)


def test_paged_ragged_lengths_match_oracle(ops):
    _log("case: paged ragged lengths")
    B, Hq, Hk, L, D, ps = 3, 8, 2, 1000, 128, 128
    lens = [1000, 37, 513]
    q = randn((B, Hq, D), seed=30)
    k, v = randn((B, Hk, L, D), seed=31), randn((B, Hk, L, D), seed=32)
    kp, table = paginate(k, ps, seed=33)
    vp, _ = paginate(v, ps, seed=33)
    o, lse = ops.decode_paged(q.cuda(), kp, vp, table,
                              torch.tensor(lens, dtype=torch.int32, device="cuda"),
                              max_seq_len=L, num_splits=4, return_lse=True)
    torch.cuda.synchronize()
    to, tl = oracle.decode_paged(bits(q), bits(kp), bits(vp), table.cpu().numpy(),
                                 np.array(lens, np.int32), max_seq_len=L, num_splits=4)
    ref_all = oracle.decode(to, oracle.BF16)
    assert np.abs(to_f32(o) - ref_all).max() <= TOL_BF16_ABS
    assert_rel_rows(to_f32(o), ref_all, TOL_BF16_REL, "paged ragged vs twin")
    assert np.abs(to_f32(lse) - tl).max() <= TOL_LSE_ABS
    for b, n in enumerate(lens):
        ro, rl, _ = oracle.decode_splitk(bits(q[b:b + 1]), bits(k[b:b + 1, :, :n]),
                                         bits(v[b:b + 1, :, :n]), oracle.BF16, num_splits=1)
        ref = oracle.decode(ro, oracle.BF16)[0]
        got = to_f32(o[b])
        err = np.abs(got - ref).max()
        assert err <= TOL_BF16_ABS and err <= 2e-2 * np.abs(ref).max(), (b, err)
        assert np.abs(to_f32(lse[b]) - rl[0]).max() <= TOL_LSE_ABS


def test_paged_empty_sequence_and_bad_table(ops):
    _log("case: paged empty sequence, out-of-range table entries")
    B, Hq, Hk, L, D, ps = 2, 4, 1, 256, 128, 64
    q = randn((B, Hq, D), seed=40).cuda()
    k, v = randn((B, Hk, L, D), seed=41), randn((B, Hk, L, D), seed=42)
    kp, table = paginate(k, ps, seed=43)
    vp, _ = paginate(v, ps, seed=43)
    lens = torch.tensor([0, L], dtype=torch.int32, device="cuda")
    o, lse = ops.decode_paged(q, kp, vp, table, lens, max_seq_len=L, return_lse=True)
    torch.cuda.synchronize()
    assert (to_f32(o[0]) == 0).all() and torch.isinf(lse[0]).all() and (lse[0] < 0).all()
    assert torch.isfinite(o[1].float()).all()
    bad = table.clone()
    bad[1, 0], bad[1, 1] = -5, 10 ** 6
    o2 = ops.decode_paged(q, kp, vp, bad, lens, max_seq_len=L)
    torch.cuda.synchronize()
    assert torch.isfinite(o2.float()).all()
    to, _ = oracle.decode_paged(bits(q), bits(kp), bits(vp), bad.cpu().numpy(),
                                lens.cpu().numpy(), max_seq_len=L)
    ref2 = oracle.decode(to, oracle.BF16)
    assert np.abs(to_f32(o2) - ref2).max() <= TOL_BF16_ABS
    assert_rel_rows(to_f32(o2), ref2, TOL_BF16_REL, "paged bad table vs twin")


def page_scales(scales, table, npages, seed):
    """Per-(page, kv head) scales [npages, Hk] from per-block scales
    [B, Hk, per]: block j of sequence b lives in page table[b, j]; pages no
    sequence uses get unrelated scales, so a misread shows."""
    B, Hk, per = scales.shape
    g = torch.Generator().manual_seed(seed)
    pool = (torch.rand((npages, Hk), generator=g) * 1.5 + 0.5).cuda()
    for b in range(B):
        pool[table[b].long()] = scales[b].t()
    return pool.contiguous()


def fp8_pools(ops, k, v, ps, seed, token_major=False):
    kc, ks = ops.kv_quantize_fp8(k.cuda(), scale_block=ps)
    vc, vs = ops.kv_quantize_fp8(v.cuda(), scale_block=ps)
    kp, table = paginate(kc.cpu(), ps, seed=seed, token_major=token_major)
    vp, _ = paginate(vc.cpu(), ps, seed=seed, token_major=token_major)
    kps = page_scales(ks, table, kp.shape[0], seed + 1)
    vps = page_scales(vs, table, kp.shape[0], seed + 2)
    return (kc, ks, vc, vs), (kp, vp, kps, vps, table)


@pytest.mark.parametrize("token_major", [False, True])
def test_paged_fp8_equals_contiguous_bitwise(ops, token_major):
    _log(f"case: paged fp8 == contiguous fp8, token_major={token_major}")
    B, Hq, Hk, L, D, ps, splits = 2, 8, 2, 1024, 128, 64, 5
    q = randn((B, Hq, D), seed=50).cuda()
    k, v = randn((B, Hk, L, D), seed=51), randn((B, Hk, L, D), seed=52)
    (kc, ks, vc, vs), (kp, vp, kps, vps, table) = fp8_pools(ops, k, v, ps, 53, token_major)
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    o_ref, lse_ref = ops.decode_splitk(q, kc, vc, k_scale=ks, v_scale=vs, num_splits=splits,
                                       scale_block=ps, return_lse=True)
    o, lse = ops.decode_paged(q, kp, vp, table, lens, max_seq_len=L, num_splits=splits,
                              return_lse=True, k_scales=kps, v_scales=vps)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse, lse_ref)
    to, tl = oracle.decode_paged(bits(q), kp.cpu().numpy(), vp.cpu().numpy(),
                                 table.cpu().numpy(), lens.cpu().numpy(), max_seq_len=L,
                                 num_splits=splits, k_scales=kps.cpu().numpy(),
                                 v_scales=vps.cpu().numpy())
    ref = oracle.decode(to, oracle.BF16)
    assert np.abs(to_f32(o) - ref).max() <= TOL_FP8_ABS
    assert_rel_rows(to_f32(o), ref, TOL_BF16_REL, "paged fp8 vs twin")
    assert np.abs(to_f32(lse) - tl).max() <= TOL_LSE_ABS


@pytest.mark.parametrize("ps", [32, 128, 256])
def test_paged_fp8_ragged_empty_and_bad_table(ops, ps):
    _log(f"case: paged fp8 ragged/empty/bad table, page={ps}")
    B, Hq, Hk, L, D = 4, 16, 2, 1000, 128
    lens = torch.tensor([1000, 0, 37, 513], dtype=torch.int32, device="cuda")
    q = randn((B, Hq, D), seed=60).cuda()
    k, v = randn((B, Hk, L, D), seed=61), randn((B, Hk, L, D), seed=62)
    _, (kp, vp, kps, vps, table) = fp8_pools(ops, k, v, ps, 63, token_major=(ps == 128))
    bad = table.clone()
    bad[3, 0], bad[0, 1] = -9, 10 ** 6
    for tab in (table, bad):
        o, lse = ops.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=3,
                                  return_lse=True, k_scales=kps, v_scales=vps)
        torch.cuda.synchronize()
        to, tl = oracle.decode_paged(bits(q), kp.cpu().numpy(), vp.cpu().numpy(),
                                     tab.cpu().numpy(), lens.cpu().numpy(), max_seq_len=L,
                                     num_splits=3, k_scales=kps.cpu().numpy(),
                                     v_scales=vps.cpu().numpy())
        ref = oracle.decode(to, oracle.BF16)
        assert np.abs(to_f32(o) - ref).max() <= TOL_FP8_ABS
        assert_rel_rows(to_f32(o), ref, TOL_BF16_REL, f"paged fp8 ragged page={ps} vs twin")
        assert (to_f32(o[1]) == 0).all() and torch.isinf(lse[1]).all() and (lse[1] < 0).all()
        fin = np.isfinite(tl)
        assert np.array_equal(fin, torch.isfinite(lse).cpu().numpy())
        assert np.abs(to_f32(lse)[fin] - tl[fin]).max() <= TOL_LSE_ABS
