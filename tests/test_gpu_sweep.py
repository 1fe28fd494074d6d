"""Seeded random-shape sweeps of every GPU entry point against the oracle.

Each case draws its shape, layout and options from a fixed seed (so a
failure names a reproducible case), prints them before the GPU call and
checks the result against the CPU oracle at the contract's tolerances:

* prefill (neptune_attn_fwd): batch, heads, GQA group, ragged Sq and Sk
  (including Sq > Sk under the causal mask, where early rows see no key),
  head_dim 64 / 128, bf16 / f16, the pipeline_stages and k_dim_order
  knobs, and strided views of larger buffers;
* split-K decode (neptune_decode_splitk): bf16 and fp8 KV, GQA groups 1-16,
  ragged L, explicit and library-chosen split counts, fp8 scale blocks of
  32, 64 and 128 tokens;
* paged decode (neptune_decode_paged, neptune_decode_paged_fp8): page sizes
  32-256, both pool layouts, bf16 and fp8 pools, ragged lengths including
  empty sequences;
* selective scan (neptune_selective_scan_fwd): batch 1-3, ragged channel
  counts, lengths 1-1500 (odd ones take the single pass, even ones of two
  64-step chunks or more the chunked path when the channels leave the GPU
  unfilled), with or without z, D and delta_bias, softplus on or off; and
  eight long few-channel cases (lengths 2048-24000, 1-47 channels), whose
  chains of more than 64 chunks take the wave-parallel carry.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_BF16_REL, TOL_FP8_ABS, TOL_LSE_ABS, assert_rel_rows,
                     bits, max_abs, oracle_dtype, randn, to_f32)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def _lse_close(got, ref):
    """Equal -inf pattern (rows that see no key), finite values within tolerance."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.isfinite(got[fin]).all()
    if fin.any():
        assert np.abs(got[fin] - ref[fin]).max() <= TOL_LSE_ABS


def _prefill_case(i):
    rng = np.random.default_rng(1000 + i)
    D = int(rng.choice([64, 128, 128]))
    B = int(rng.integers(1, 3))
    Hk = int(rng.choice([1, 2, 4]))
    Hq = Hk * int(rng.choice([1, 2, 4]))
    Sq = int(rng.integers(1, 700))
    Sk = int(rng.integers(1, 900))
    causal = bool(rng.integers(0, 2))
    dtype = torch.bfloat16 if rng.integers(0, 2) else torch.float16
    stages = int(rng.choice([0, 1, 2, 3])) if D == 128 else 0
    kd = int(D == 128 and Sk % 8 == 0 and rng.integers(0, 2))
    strided = bool(rng.integers(0, 2))
    return dict(B=B, Hq=Hq, Hk=Hk, Sq=Sq, Sk=Sk, D=D, causal=causal, dtype=dtype,
                stages=stages, kd=kd, strided=strided, seed=1000 + i)


@pytest.mark.parametrize("i", range(200))
def test_prefill_sweep(ops, i):
    c = _prefill_case(i)
    _log(f"case: prefill sweep {c}")
    B, Hq, Hk, Sq, Sk, D = c["B"], c["Hq"], c["Hk"], c["Sq"], c["Sk"], c["D"]
    q = randn((B, Hq, Sq, D), seed=c["seed"], dtype=c["dtype"])
    k = randn((B, Hk, Sk, D), seed=c["seed"] + 1, dtype=c["dtype"])
    v = randn((B, Hk, Sk, D), seed=c["seed"] + 2, dtype=c["dtype"])
    ro, rl = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle_dtype(q), c["causal"])
    ref = oracle.decode(ro, oracle_dtype(q))
    kk = k.transpose(2, 3) if c["kd"] else k
    if c["strided"]:
        # every tensor a view into a larger buffer (padded head_dim rows / seq)
        def pad(t, last_pad):
            buf = torch.zeros(t.shape[:-1] + (t.shape[-1] + last_pad,), dtype=t.dtype)
            buf[..., :t.shape[-1]] = t
            return buf.cuda()[..., :t.shape[-1]]
        qd, vd = pad(q, 8), pad(v, 16)
        if c["kd"]:
            kbuf = torch.zeros(kk.shape[:-1] + (kk.shape[-1] + 8,), dtype=kk.dtype)
            kbuf[..., :kk.shape[-1]] = kk
            kdv = kbuf.cuda()[..., :kk.shape[-1]]
        else:
            kdv = pad(kk, 24)
    else:
        qd, kdv, vd = q.cuda(), kk.contiguous().cuda(), v.cuda()
    o, lse = ops.attention(qd, kdv, vd, causal=c["causal"], return_lse=True,
                           pipeline_stages=c["stages"], k_dim_order=c["kd"])
    torch.cuda.synchronize()
    assert max_abs(to_f32(o), ref) <= TOL_BF16_ABS
    _lse_close(to_f32(lse), rl)


def _decode_case(i):
    rng = np.random.default_rng(2000 + i)
    B = int(rng.integers(1, 5))
    Hk = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8, 16]))
    L = int(rng.integers(1, 3000))
    splits = int(rng.choice([0, 1, 3, 7]))
    fp8 = bool(rng.integers(0, 2))
    sb = int(rng.choice([32, 64, 128]))
    return dict(B=B, Hq=Hk * group, Hk=Hk, L=L, splits=splits, fp8=fp8, sb=sb, seed=2000 + i)


@pytest.mark.parametrize("i", range(120))
def test_decode_sweep(ops, i):
    c = _decode_case(i)
    _log(f"case: decode sweep {c}")
    B, Hq, Hk, L = c["B"], c["Hq"], c["Hk"], c["L"]
    q = randn((B, Hq, 128), seed=c["seed"])
    k = randn((B, Hk, L, 128), seed=c["seed"] + 1)
    v = randn((B, Hk, L, 128), seed=c["seed"] + 2)
    if c["fp8"]:
        kc, ks = ops.kv_quantize_fp8(k.cuda(), scale_block=c["sb"])
        vc, vs = ops.kv_quantize_fp8(v.cuda(), scale_block=c["sb"])
        o, lse = ops.decode_splitk(q.cuda(), kc, vc, k_scale=ks, v_scale=vs,
                                   num_splits=c["splits"], scale_block=c["sb"], return_lse=True)
        torch.cuda.synchronize()
        ro, rl, _ = oracle.decode_splitk(bits(q), kc.cpu().numpy(), vc.cpu().numpy(), oracle.FP8,
                                         ks.cpu().numpy(), vs.cpu().numpy(),
                                         num_splits=c["splits"], scale_block=c["sb"])
        tol = TOL_FP8_ABS
    else:
        o, lse = ops.decode_splitk(q.cuda(), k.cuda(), v.cuda(), num_splits=c["splits"],
                                   return_lse=True)
        torch.cuda.synchronize()
        ro, rl, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16,
                                         num_splits=c["splits"])
        tol = TOL_BF16_ABS
    ref = oracle.decode(ro, oracle.BF16)
    assert max_abs(to_f32(o), ref) <= tol
    # the oracle reads the same values (bf16 or fp8 codes): kernel error alone
    assert_rel_rows(to_f32(o), ref, TOL_BF16_REL, "decode sweep vs oracle")
    assert max_abs(to_f32(lse), rl) <= TOL_LSE_ABS


def _paginate(kv, ps, rng, token_major):
    B, Hk, L, D = kv.shape
    per = -(-L // ps)
    npages = B * per + 2
    ids = torch.from_numpy(rng.permutation(npages)[: B * per].reshape(B, per).astype(np.int32))
    shape = (npages, ps, Hk, D) if token_major else (npages, Hk, ps, D)
    pool = torch.zeros(shape, dtype=kv.dtype)
    for b in range(B):
        for j in range(per):
            blk = kv[b, :, j * ps:(j + 1) * ps]
            if token_major:
                pool[ids[b, j], :blk.shape[1]] = blk.transpose(0, 1)
            else:
                pool[ids[b, j], :, :blk.shape[1]] = blk
    view = pool.cuda()
    return (view.permute(0, 2, 1, 3) if token_major else view), ids.cuda()


@pytest.mark.parametrize("i", range(80))
def test_paged_decode_sweep(ops, i):
    rng = np.random.default_rng(3000 + i)
    B = int(rng.integers(1, 4))
    Hk = int(rng.choice([1, 2, 4]))
    Hq = Hk * int(rng.choice([1, 4, 8]))
    ps = int(rng.choice([32, 64, 128, 256]))
    L = int(rng.integers(ps, 2500))
    lens = [int(x) for x in rng.integers(0, L + 1, size=B)]
    token_major = bool(rng.integers(0, 2))
    splits = int(rng.choice([0, 2, 5]))
    fp8 = bool(rng.integers(0, 2))
    _log(f"case: paged sweep B={B} Hq={Hq} Hk={Hk} page={ps} L={L} lens={lens} "
         f"token_major={token_major} splits={splits} fp8={fp8}")
    q = randn((B, Hq, 128), seed=3000 + i)
    k = randn((B, Hk, L, 128), seed=3100 + i)
    v = randn((B, Hk, L, 128), seed=3200 + i)
    scales = {}
    if fp8:
        # one scale per page: quantise with the page as the scale block and
        # carry block j of sequence b to page table[b, j]
        k, ks = (t.cpu() for t in ops.kv_quantize_fp8(k.cuda(), scale_block=ps))
        v, vs = (t.cpu() for t in ops.kv_quantize_fp8(v.cuda(), scale_block=ps))
    kp, table = _paginate(k, ps, np.random.default_rng(3300 + i), token_major)
    vp, _ = _paginate(v, ps, np.random.default_rng(3300 + i), token_major)
    if fp8:
        for name, sc in (("k_scales", ks), ("v_scales", vs)):
            pool = torch.ones((kp.shape[0], Hk), dtype=torch.float32)
            tab = table.cpu().long()
            for b in range(B):
                pool[tab[b]] = sc[b].t()
            scales[name] = pool.cuda()
    sl = torch.tensor(lens, dtype=torch.int32)
    o, lse = ops.decode_paged(q.cuda(), kp, vp, table, sl.cuda(), max_seq_len=L,
                              num_splits=splits, return_lse=True, **scales)
    torch.cuda.synchronize()
    pool_np = (lambda t: t.cpu().numpy()) if fp8 else bits
    ro, rl = oracle.decode_paged(bits(q), pool_np(kp), pool_np(vp), table.cpu().numpy(),
                                 sl.numpy(), max_seq_len=L, num_splits=splits,
                                 **{n: t.cpu().numpy() for n, t in scales.items()})
    ref = oracle.decode(ro, oracle.BF16)
    assert max_abs(to_f32(o), ref) <= (TOL_FP8_ABS if fp8 else TOL_BF16_ABS)
    # the twin reads the same values (bf16 or fp8 codes): kernel error alone
    assert_rel_rows(to_f32(o), ref, TOL_BF16_REL, "paged sweep vs twin")
    _lse_close(to_f32(lse), rl)


def _scan_case(i):
    rng = np.random.default_rng(4000 + i)
    return dict(b=int(rng.integers(1, 4)), d=int(rng.integers(1, 200)),
                L=int(rng.integers(1, 1500)), gate=bool(rng.integers(0, 2)),
                with_d=bool(rng.integers(0, 2)), bias=bool(rng.integers(0, 2)),
                softplus=bool(rng.integers(0, 4)), seed=4000 + i)


def _scan_long_case(i):
    """Few channels over long even sequences: the chunked path with chains of
    more than 64 chunks (the wave-parallel carry)."""
    rng = np.random.default_rng(9000 + i)
    L = int(rng.integers(1024, 12000)) * 2
    return dict(b=int(rng.integers(1, 3)), d=int(rng.integers(1, 48)), L=L,
                gate=bool(rng.integers(0, 2)), with_d=bool(rng.integers(0, 2)),
                bias=bool(rng.integers(0, 2)), softplus=bool(rng.integers(0, 4)), seed=9000 + i)


@pytest.mark.parametrize("i", range(60))
def test_scan_sweep(ops, i):
    _scan_sweep_case(ops, _scan_case(i))


@pytest.mark.parametrize("i", range(8))
def test_scan_sweep_long(ops, i):
    _scan_sweep_case(ops, _scan_long_case(i))


def _scan_sweep_case(ops, c):
    _log(f"case: scan sweep {c}")
    b, d, L, n = c["b"], c["d"], c["L"], 16
    u, z = randn((b, d, L), seed=c["seed"]), randn((b, d, L), seed=c["seed"] + 1)
    Bm, Cm = randn((b, n, L), seed=c["seed"] + 2), randn((b, n, L), seed=c["seed"] + 3)
    A = -torch.exp(randn((d, n), seed=c["seed"] + 4, dtype=torch.float32))
    D = randn((d,), seed=c["seed"] + 5, dtype=torch.float32) if c["with_d"] else None
    g = torch.Generator().manual_seed(c["seed"] + 6)
    if c["softplus"]:
        dr = randn((b, d, L), seed=c["seed"] + 7)
        bias = randn((d,), seed=c["seed"] + 8, dtype=torch.float32) if c["bias"] else None
    else:  # delta = delta_raw + bias directly: keep it positive
        dr = (torch.rand((b, d, L), generator=g) * 0.5 + 0.01).to(torch.bfloat16)
        bias = torch.rand((d,), generator=g) * 0.1 if c["bias"] else None
    y = ops.selective_scan(u.cuda(), dr.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(),
                           None if D is None else D.cuda(), z.cuda() if c["gate"] else None,
                           None if bias is None else bias.cuda(),
                           delta_softplus=c["softplus"])
    torch.cuda.synchronize()
    ref_bits, _ = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm),
                                        None if D is None else D.numpy(),
                                        bits(z) if c["gate"] else None,
                                        None if bias is None else bias.numpy(),
                                        softplus=c["softplus"])
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y).astype(np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref) > 2e-2 * np.maximum(1.0, np.abs(ref))
    assert not bad.any(), (np.argwhere(bad)[:5], np.abs(got - ref).max())
