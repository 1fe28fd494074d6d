"""Pins the CPU oracle (oracle/neptune_oracle.c) before it is trusted as the
checker of the HIP kernels.

The reference holds no numeric golden vectors (its goldens are emitted
source text, tests/golden/*.py), so each oracle function is pinned by an
independent computation: numpy float64 brute force written here from the
textbook definitions, torch/numpy codecs, closed forms and invariants, and
fixtures committed under tests/golden/. Each check is chosen so that a
plausible slip (wrong scale, missing mask, dropped rescale, wrong rounding
mode, transposed operand) fails it; test_planted_* show that for a few.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from helpers import (bits, periodic_attention, periodic_k0, periodic_k127, periodic_vper, randn,
                     steady_scan_table)

LN2 = math.log(2.0)
LOG2E = 1.0 / LN2


# --------------------------------------------------------------- codecs


def test_bf16_codec_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-45, 3.4e38, 1.0 + 2.0 ** -8,
                  1.0 + 3 * 2.0 ** -8], dtype=np.float32),
    ]).astype(np.float32)
    got = oracle.encode(x, oracle.BF16)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    back = oracle.decode(got, oracle.BF16)
    assert np.array_equal(back, torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_f16_codec_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 2.0 ** rng.integers(-30, 20, 20000),
        np.array([65504.0, 65519.0, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  6.1e-5, -0.0], dtype=np.float32),
    ]).astype(np.float32)
    got = oracle.encode(x, oracle.F16)
    assert np.array_equal(got.view(np.uint16), x.astype(np.float16).view(np.uint16))
    assert np.array_equal(oracle.decode(got, oracle.F16), got.astype(np.float32))


def _e4m3_spec_value(c: int) -> float:
    """OCP 8-bit FP spec v1.0, E4M3: S.EEEE.MMM, bias 7, S.1111.111 = NaN."""
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return float("nan")
    v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return -v if s else v


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.decode(codes, oracle.FP8)
    spec = np.array([_e4m3_spec_value(c) for c in range(256)], dtype=np.float32)
    via_torch = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(spec)
    assert np.array_equal(nan, np.isnan(got)) and np.array_equal(nan, np.isnan(via_torch))
    assert np.array_equal(got[~nan], spec[~nan])
    assert np.array_equal(got[~nan], via_torch[~nan])
    assert spec[0x7E] == 448.0 and spec[0x01] == 2.0 ** -9


def test_e4m3_encode_round_trip_and_ties():
    finite = np.array([c for c in range(256) if not math.isnan(_e4m3_spec_value(c))], dtype=np.uint8)
    vals = oracle.decode(finite, oracle.FP8)
    assert np.array_equal(oracle.encode(vals, oracle.FP8), finite)
    # midpoints between neighbours round to the even code
    pos = np.array(sorted(set(float(v) for v in vals if v >= 0)), dtype=np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    enc = oracle.encode(mids, oracle.FP8).astype(np.int64)
    lo = oracle.encode(pos[:-1].astype(np.float32), oracle.FP8).astype(np.int64)
    want = np.where(lo % 2 == 0, lo, lo + 1)
    assert np.array_equal(enc, want)


def test_e4m3_encode_matches_torch_in_range_and_saturates():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(50000) * 100).astype(np.float32)
    x = np.clip(x, -448, 448)
    got = oracle.encode(x, oracle.FP8)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)
    sat = oracle.encode(np.array([449.0, 464.0, 1e9, np.inf, -500.0], np.float32), oracle.FP8)
    assert list(sat) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE]


# ------------------------------------------------------------ attention


def brute_attention(q, k, v, causal, scale):
    """Textbook softmax attention in float64 (numpy), with GQA and a
    bottom-right-aligned causal mask."""
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    o = np.zeros((B, Hq, Sq, D))
    lse = np.zeros((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            kk, vv = k[b, h // (Hq // Hk)], v[b, h // (Hq // Hk)]
            s = (q[b, h] @ kk.T) * scale
            if causal:
                i = np.arange(Sq)[:, None]
                j = np.arange(Sk)[None, :]
                s = np.where(j > i + (Sk - Sq), -np.inf, s)
            mx = s.max(axis=1, keepdims=True)
            p = np.exp(s - mx)
            o[b, h] = (p @ vv) / p.sum(axis=1, keepdims=True)
            lse[b, h] = mx[:, 0] + np.log(p.sum(axis=1))
    return o, lse


def _f64(t):
    return t.double().numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape_q,shape_k", [((1, 2, 9, 16), (1, 2, 9, 16)),
                                             ((2, 4, 70, 32), (2, 2, 70, 32)),
                                             ((1, 2, 5, 8), (1, 1, 13, 8))])
def test_attn_exact_matches_brute_force(causal, shape_q, shape_k):
    q = randn(shape_q, 1, torch.float32)
    k = randn(shape_k, 2, torch.float32)
    v = randn(shape_k, 3, torch.float32)
    o, lse = oracle.attn_exact(bits(q), bits(k), bits(v), oracle.F32, causal)
    scale = float(np.float32(LOG2E / math.sqrt(shape_q[3]))) * LN2
    bo, blse = brute_attention(_f64(q), _f64(k), _f64(v), causal, scale)
    assert np.abs(o - bo).max() < 1e-12
    assert np.abs(lse - blse).max() < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_attn_fwd_fp32_policy_close_to_exact(causal):
    """Config 1 shape: the HTile recurrence in fp32 (no 16-bit rounding of P)
    is within 1e-5 relative of the fp64 closed form."""
    q, k, v = (randn((1, 1, 128, 64), s, torch.float32) for s in (0, 1, 2))
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.F32, causal)
    eo, else_ = oracle.attn_exact(bits(q), bits(k), bits(v), oracle.F32, causal)
    assert np.abs(o - eo).max() <= 1e-5 * np.abs(eo).max()
    assert np.abs(lse - else_).max() <= 1e-5 * np.abs(else_).max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attn_fwd_16bit_policy(dtype):
    """bf16/f16 policy: close to exact, and P really is rounded (the result
    differs from the fp32 recurrence run on the same values)."""
    dt = oracle.BF16 if dtype == torch.bfloat16 else oracle.F16
    q, k, v = (randn((2, 2, 200, 128), 5 + s, dtype, 0.5) for s in range(3))
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), dt, True)
    eo, else_ = oracle.attn_exact(bits(q), bits(k), bits(v), dt, True)
    got = oracle.decode(o, dt)
    assert np.abs(got - eo).max() <= 2e-2
    assert np.abs(lse - else_).max() <= 1e-4
    o32, _ = oracle.attn_fwd(*(bits(t.float()) for t in (q, k, v)), oracle.F32, True)
    assert np.abs(got - o32).max() > 0


def test_attn_causal_first_row_is_v0_and_q_zero_is_prefix_mean():
    v = randn((1, 2, 100, 64), 7, torch.bfloat16)
    k = randn((1, 2, 100, 64), 8, torch.bfloat16)
    q = randn((1, 2, 100, 64), 9, torch.bfloat16)
    o, _ = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.BF16, True)
    assert np.array_equal(o[:, :, 0, :], bits(v)[:, :, 0, :])
    o0, lse0 = oracle.attn_fwd(bits(torch.zeros_like(q)), bits(k), bits(v), oracle.BF16, True)
    prefix = _f64(v).cumsum(axis=2) / np.arange(1, 101)[None, None, :, None]
    assert np.abs(oracle.decode(o0, oracle.BF16) - prefix).max() <= 1e-2
    # Q = 0: all scores 0, lse = ln(number of visible keys)
    assert np.abs(lse0 - np.log(np.arange(1, 101))[None, None, :]).max() < 1e-5


def test_attn_shift_and_permutation_invariance():
    q, k, v = (randn((1, 1, 64, 32), 10 + s, torch.float32) for s in range(3))
    c = randn((32,), 13, torch.float32)
    base, _ = oracle.attn_exact(bits(q), bits(k), bits(v), oracle.F32, False)
    # adding c to every key adds q_i.c to every score of row i: no change
    kk = (k.double() + c.double()).float()
    shifted, _ = oracle.attn_exact(bits(q), bits(kk), bits(v), oracle.F32, False)
    assert np.abs(shifted - base).max() < 1e-5
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(0))
    permuted, _ = oracle.attn_exact(bits(q), bits(k[:, :, perm]), bits(v[:, :, perm]),
                                    oracle.F32, False)
    assert np.abs(permuted - base).max() < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_attn_k_dim_order_is_layout_only(causal):
    """K given [B, Hk, D, Sk] with k_dim_order 1 is the same operand as
    K [B, Hk, Sk, D]: the HTile policy and the fp64 closed form give
    identical results, and a strided K^T view (padded rows) is read in
    place."""
    B, Hq, Hk, Sq, Sk, D = 2, 4, 2, 40, 72, 16
    q = bits(randn((B, Hq, Sq, D), seed=61))
    k = bits(randn((B, Hk, Sk, D), seed=62))
    v = bits(randn((B, Hk, Sk, D), seed=63))
    kt = np.ascontiguousarray(k.transpose(0, 1, 3, 2))
    o0, l0 = oracle.attn_fwd(q, k, v, oracle.BF16, causal=causal)
    o1, l1 = oracle.attn_fwd(q, kt, v, oracle.BF16, causal=causal, k_dim_order=1)
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1)
    e0, _ = oracle.attn_exact(q, k, v, oracle.BF16, causal=causal)
    e1, _ = oracle.attn_exact(q, kt, v, oracle.BF16, causal=causal, k_dim_order=1)
    assert np.array_equal(e0, e1)
    # the same K^T buffer read in the other order is a different operand
    o2, _ = oracle.attn_fwd(q, kt.reshape(B, Hk, Sk, D), v, oracle.BF16, causal=causal)
    assert not np.array_equal(o0, o2)


def test_attn_gqa_equals_repeated_mha():
    q = randn((1, 8, 40, 64), 20, torch.bfloat16)
    k = randn((1, 2, 40, 64), 21, torch.bfloat16)
    v = randn((1, 2, 40, 64), 22, torch.bfloat16)
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.BF16, True)
    o2, lse2 = oracle.attn_fwd(bits(q), bits(k.repeat_interleave(4, 1)),
                               bits(v.repeat_interleave(4, 1)), oracle.BF16, True)
    assert np.array_equal(o, o2) and np.array_equal(lse, lse2)


def test_planted_scale_error_is_caught():
    """A wrong score scale (1/D instead of 1/sqrt(D)) fails the brute-force pin."""
    q, k, v = (randn((1, 1, 16, 16), 30 + s, torch.float32) for s in range(3))
    wrong = float(np.float32(LOG2E / 16.0))
    o, _ = oracle.attn_exact(bits(q), bits(k), bits(v), oracle.F32, False, scale_log2=wrong)
    bo, _ = brute_attention(_f64(q), _f64(k), _f64(v), False, 1.0 / 4.0)
    assert np.abs(o - bo).max() > 1e-3


# --------------------------------------------------------------- decode


def test_decode_layout_rules():
    assert oracle.decode_layout(16, 8, 32768, 16) == (16, 2048)
    assert oracle.decode_layout(2, 2, 1000, 3) == (3, 384)      # 334 -> 6 blocks of 64
    s, c = oracle.decode_layout(1, 1, 100000, 0)                 # library choice
    assert c % 64 == 0 and s * c >= 100000 and (s - 1) * c < 100000
    assert s <= -(-100000 // 256)
    assert oracle.decode_layout(4, 2, 50, 0) == (1, 64)


@pytest.mark.parametrize("B,Hq,Hk,L,splits", [(2, 8, 2, 1000, 3), (1, 4, 1, 300, 0),
                                              (2, 4, 4, 700, 5)])
def test_decode_matches_exact(B, Hq, Hk, L, splits):
    q = randn((B, Hq, 128), 40)
    k = randn((B, Hk, L, 128), 41)
    v = randn((B, Hk, L, 128), 42)
    o, lse, parts = oracle.decode_splitk(bits(q), bits(k), bits(v), num_splits=splits)
    eo, else_ = oracle.attn_exact(bits(q)[:, :, None, :], bits(k), bits(v), oracle.BF16)
    got = oracle.decode(o, oracle.BF16)
    ref = eo[:, :, 0, :]
    assert np.abs(got - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.abs(lse - else_[:, :, 0]).max() <= 1e-4
    # partials: per split (o~, m, l); recombined in float64 they give o and
    # each split's lse equals the exact lse over that split's keys alone
    S, chunk = oracle.decode_layout(B, Hk, L, splits)
    m, l, ot = parts[..., 128], parts[..., 129], parts[..., :128]
    M = m.max(axis=2, keepdims=True)
    w = np.exp2(m - M)
    comb = (w[..., None] * ot).sum(axis=2) / (w * l).sum(axis=2)[..., None]
    assert np.abs(comb - ref).max() <= 2e-2 * np.abs(ref).max()
    for s in range(S):
        k0, k1 = s * chunk, min(L, (s + 1) * chunk)
        _, slse = oracle.attn_exact(bits(q)[:, :, None, :], bits(k)[:, :, k0:k1],
                                    bits(v)[:, :, k0:k1], oracle.BF16)
        assert np.abs((m[:, :, s] + np.log2(l[:, :, s])) * LN2 - slse[:, :, 0]).max() <= 1e-4


def test_decode_split_invariance_and_gqa():
    q = randn((2, 8, 128), 50)
    k = randn((2, 2, 2048, 128), 51)
    v = randn((2, 2, 2048, 128), 52)
    o1, _, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), num_splits=1)
    o16, _, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), num_splits=16)
    assert np.abs(oracle.decode(o1, oracle.BF16) - oracle.decode(o16, oracle.BF16)).max() <= 2e-3
    om, _, _ = oracle.decode_splitk(bits(q), bits(k.repeat_interleave(4, 1)),
                                    bits(v.repeat_interleave(4, 1)), num_splits=16)
    assert np.array_equal(o16, om)


def _paginate(kv, ps, rng, token_major=False, spare=3):
    """Scatter bits [B, Hk, L, D] into a shuffled pool; returns the pool as a
    [pages, Hk, ps, D] view and the block table."""
    B, Hk, L, D = kv.shape
    per = -(-L // ps)
    npages = B * per + spare
    ids = rng.permutation(npages)[: B * per].reshape(B, per).astype(np.int32)
    pool = np.zeros((npages, ps, Hk, D) if token_major else (npages, Hk, ps, D), kv.dtype)
    for b in range(B):
        for j in range(per):
            blk = kv[b, :, j * ps:(j + 1) * ps]
            if token_major:
                pool[ids[b, j], :blk.shape[1]] = blk.transpose(1, 0, 2)
            else:
                pool[ids[b, j], :, :blk.shape[1]] = blk
    return (pool.transpose(0, 2, 1, 3) if token_major else pool), ids


@pytest.mark.parametrize("token_major", [False, True])
def test_decode_paged_equals_contiguous(token_major):
    """At full lengths the paged twin reads the same tokens in the same split
    layout as the contiguous decode: bit-identical output and lse."""
    rng = np.random.default_rng(5)
    B, Hq, Hk, L, D, ps = 2, 8, 2, 640, 32, 64
    q = bits(randn((B, Hq, D), seed=50))
    k, v = bits(randn((B, Hk, L, D), seed=51)), bits(randn((B, Hk, L, D), seed=52))
    kp, tab = _paginate(k, ps, np.random.default_rng(7), token_major)
    vp, _ = _paginate(v, ps, np.random.default_rng(7), token_major)
    lens = np.full(B, L, np.int32)
    o0, l0, _ = oracle.decode_splitk(q, k, v, oracle.BF16, num_splits=3)
    o1, l1 = oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=3)
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1)
    # a table that points one page elsewhere changes the result
    bad = tab.copy()
    bad[0, 1] = tab[1, 1]
    o2, _ = oracle.decode_paged(q, kp, vp, bad, lens, max_seq_len=L, num_splits=3)
    assert not np.array_equal(o0, o2)


def test_decode_paged_ragged_empty_and_clamped():
    B, Hq, Hk, L, D, ps = 3, 4, 2, 256, 32, 64
    q = bits(randn((B, Hq, D), seed=53))
    k, v = bits(randn((B, Hk, L, D), seed=54)), bits(randn((B, Hk, L, D), seed=55))
    kp, tab = _paginate(k, ps, np.random.default_rng(8))
    vp, _ = _paginate(v, ps, np.random.default_rng(8))
    lens = np.array([200, 0, 37], np.int32)
    o, lse = oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=2)
    for b, n in ((0, 200), (2, 37)):
        ex, exl = oracle.attn_exact(q[b][None, :, None], k[b][None, :, :n], v[b][None, :, :n],
                                    oracle.BF16)
        got = oracle.decode(o[b], oracle.BF16)
        assert np.abs(got - ex[0, :, 0]).max() <= 1e-2 * np.abs(ex).max()
        assert np.abs(lse[b] - exl[0, :, 0]).max() <= 1e-3
    assert (oracle.decode(o[1], oracle.BF16) == 0).all() and np.isneginf(lse[1]).all()
    # entries outside the pool read the nearest page of the pool, as the kernel does
    bad = tab.copy()
    bad[2, 0] = -7
    o2, _ = oracle.decode_paged(q, kp, vp, bad, lens, max_seq_len=L, num_splits=2)
    fix = tab.copy()
    fix[2, 0] = 0
    o3, _ = oracle.decode_paged(q, kp, vp, fix, lens, max_seq_len=L, num_splits=2)
    assert np.array_equal(o2, o3)


def _page_scales(scales, ids, npages, rng):
    """Per-(page, kv head) scales [npages, Hk] from per-block scales
    [B, Hk, per] (block j of sequence b lives in page ids[b, j]); pages no
    sequence uses get unrelated scales, so a misread shows."""
    B, Hk, per = scales.shape
    pool = rng.uniform(0.5, 2.0, size=(npages, Hk)).astype(np.float32)
    for b in range(B):
        for j in range(per):
            pool[ids[b, j]] = scales[b, :, j]
    return pool


@pytest.mark.parametrize("token_major", [False, True])
def test_decode_paged_fp8_equals_contiguous(token_major):
    """fp8 pools with one scale per (page, kv head) read the same codes and
    scales, in the same split layout, as the contiguous fp8 decode whose
    scale block is the page: bit-identical output and lse. A scale moved to
    another page changes the result."""
    B, Hq, Hk, L, D, ps = 2, 8, 2, 640, 32, 64
    q = bits(randn((B, Hq, D), seed=70))
    kc, ks = oracle.kv_quantize_fp8(bits(randn((B, Hk, L, D), seed=71)), scale_block=ps)
    vc, vs = oracle.kv_quantize_fp8(bits(randn((B, Hk, L, D), seed=72)), scale_block=ps)
    kp, tab = _paginate(kc, ps, np.random.default_rng(9), token_major)
    vp, _ = _paginate(vc, ps, np.random.default_rng(9), token_major)
    npages = kp.shape[0]
    kps = _page_scales(ks, tab, npages, np.random.default_rng(10))
    vps = _page_scales(vs, tab, npages, np.random.default_rng(11))
    lens = np.full(B, L, np.int32)
    d = oracle.decode_splitk(q, kc, vc, oracle.FP8, ks, vs, num_splits=3, scale_block=ps)
    o1, l1 = oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=3,
                                 k_scales=kps, v_scales=vps)
    assert np.array_equal(d[0], o1) and np.array_equal(d[1], l1)
    moved = kps.copy()
    moved[tab[1, 2]] *= 1.5
    o2, _ = oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=3,
                                k_scales=moved, v_scales=vps)
    assert not np.array_equal(o1, o2)


def test_decode_paged_fp8_ragged_empty_and_clamped():
    B, Hq, Hk, L, D, ps = 3, 4, 2, 256, 32, 64
    q = bits(randn((B, Hq, D), seed=73))
    kc, ks = oracle.kv_quantize_fp8(bits(randn((B, Hk, L, D), seed=74)), scale_block=ps)
    vc, vs = oracle.kv_quantize_fp8(bits(randn((B, Hk, L, D), seed=75)), scale_block=ps)
    kp, tab = _paginate(kc, ps, np.random.default_rng(12))
    vp, _ = _paginate(vc, ps, np.random.default_rng(12))
    kps = _page_scales(ks, tab, kp.shape[0], np.random.default_rng(13))
    vps = _page_scales(vs, tab, kp.shape[0], np.random.default_rng(14))
    lens = np.array([200, 0, 37], np.int32)
    o, lse = oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L, num_splits=2,
                                 k_scales=kps, v_scales=vps)
    kd = oracle.decode(kc, oracle.FP8) * np.repeat(ks, ps, axis=2)[..., None]
    vd = oracle.decode(vc, oracle.FP8) * np.repeat(vs, ps, axis=2)[..., None]
    qf = oracle.decode(q, oracle.BF16)
    for b, n in ((0, 200), (2, 37)):
        ex, exl = oracle.attn_exact(qf[b][None, :, None], kd[b][None, :, :n].astype(np.float32),
                                    vd[b][None, :, :n].astype(np.float32), oracle.F32)
        got = oracle.decode(o[b], oracle.BF16)
        assert np.abs(got - ex[0, :, 0]).max() <= 2e-2 * np.abs(ex).max()
        assert np.abs(lse[b] - exl[0, :, 0]).max() <= 1e-4
    assert (oracle.decode(o[1], oracle.BF16) == 0).all() and np.isneginf(lse[1]).all()
    # entries outside the pool read the nearest page of the pool, scale included
    bad = tab.copy()
    bad[2, 0] = kp.shape[0] + 5
    o2, _ = oracle.decode_paged(q, kp, vp, bad, lens, max_seq_len=L, num_splits=2,
                                k_scales=kps, v_scales=vps)
    fix = tab.copy()
    fix[2, 0] = kp.shape[0] - 1
    o3, _ = oracle.decode_paged(q, kp, vp, fix, lens, max_seq_len=L, num_splits=2,
                                k_scales=kps, v_scales=vps)
    assert np.array_equal(o2, o3)
    with pytest.raises(ValueError):
        oracle.decode_paged(q, kp, vp, tab, lens, max_seq_len=L)


def test_decode_fp8_equals_dequantised_exact():
    q = randn((2, 8, 128), 60)
    k = randn((2, 2, 640, 128), 61)
    v = randn((2, 2, 640, 128), 62)
    kc, ks = oracle.kv_quantize_fp8(bits(k))
    vc, vs = oracle.kv_quantize_fp8(bits(v))
    o, lse, _ = oracle.decode_splitk(bits(q), kc, vc, oracle.FP8, ks, vs, num_splits=3)
    kd = oracle.decode(kc, oracle.FP8) * np.repeat(ks, 64, axis=2)[..., None]
    vd = oracle.decode(vc, oracle.FP8) * np.repeat(vs, 64, axis=2)[..., None]
    qf = oracle.decode(bits(q), oracle.BF16)[:, :, None, :]
    eo, else_ = oracle.attn_exact(qf, kd.astype(np.float32), vd.astype(np.float32), oracle.F32)
    got = oracle.decode(o, oracle.BF16)
    assert np.abs(got - eo[:, :, 0]).max() <= 2e-2 * np.abs(eo).max()
    assert np.abs(lse - else_[:, :, 0]).max() <= 1e-4


# ------------------------------------------------------------- quantiser


def test_kv_quantize_scales_and_codes():
    kv = randn((2, 2, 200, 128), 70)
    kv[1, 0, 64:128] = 0
    src = bits(kv)
    codes, scales = oracle.kv_quantize_fp8(src, 64)
    x = oracle.decode(src, oracle.BF16)
    for b in range(2):
        for h in range(2):
            for blk in range(4):
                seg = x[b, h, 64 * blk:64 * (blk + 1)]
                amax = np.float32(np.abs(seg).max())
                if amax == 0:
                    assert scales[b, h, blk] == 0 and not codes[b, h, 64 * blk:64 * (blk + 1)].any()
                    continue
                assert scales[b, h, blk] == np.float32(amax / np.float32(448.0))
                inv = np.float32(448.0) / amax
                y = (seg * inv).astype(np.float32)
                want = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
                assert np.array_equal(codes[b, h, 64 * blk:64 * (blk + 1)], want)
                assert (np.abs(codes[b, h, 64 * blk:64 * (blk + 1)]) & 0x7F).max() == 0x7E


# ----------------------------------------------------------------- scan


def brute_scan(u, dr, A, Bm, Cm, D, z, bias, softplus=True):
    """Mamba-1 selective scan from its definition, float64 numpy."""
    b, d, L = u.shape
    y = np.zeros((b, d, L))
    for bb in range(b):
        for c in range(d):
            x = np.zeros(A.shape[1])
            for t in range(L):
                r = dr[bb, c, t] + (bias[c] if bias is not None else 0.0)
                dl = (r if r > 20 else math.log1p(math.exp(r))) if softplus else r
                x = np.exp(dl * A[c]) * x + dl * Bm[bb, :, t] * u[bb, c, t]
                acc = float(Cm[bb, :, t] @ x) + (D[c] * u[bb, c, t] if D is not None else 0.0)
                if z is not None:
                    zz = z[bb, c, t]
                    acc *= zz / (1 + math.exp(-zz))
                y[bb, c, t] = acc
    return y


def _scan_in(b, d, L, n, seed):
    u, dr, z = (randn((b, d, L), seed + i) for i in range(3))
    Bm, Cm = randn((b, n, L), seed + 3), randn((b, n, L), seed + 4)
    A = -torch.exp(randn((d, n), seed + 5, torch.float32))
    D, bias = randn((d,), seed + 6, torch.float32), randn((d,), seed + 7, torch.float32)
    return u, dr, A, Bm, Cm, D, z, bias


@pytest.mark.parametrize("n,z_on", [(16, True), (4, False)])
def test_scan_matches_brute_force(n, z_on):
    u, dr, A, Bm, Cm, D, z, bias = _scan_in(2, 3, 37, n, 80)
    if not z_on:
        z = None
    _, y64 = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm), D.numpy(),
                                   None if z is None else bits(z), bias.numpy())
    ref = brute_scan(_f64(u), _f64(dr), _f64(A), _f64(Bm), _f64(Cm), _f64(D),
                     None if z is None else _f64(z), _f64(bias))
    assert np.abs(y64 - ref).max() <= 1e-9 * max(1.0, np.abs(ref).max())


def test_scan_closed_forms():
    u, dr, A, Bm, Cm, D, z, bias = _scan_in(1, 4, 20, 16, 90)
    uf, zf, Df = _f64(u), _f64(z), _f64(D)
    gate = zf / (1 + np.exp(-zf))
    skip = Df[None, :, None] * uf * gate
    # delta -> 0 (softplus(-60) ~ 1e-26): the state never moves
    tiny = torch.full_like(dr, -60.0)
    _, y = oracle.selective_scan(bits(u), bits(tiny), A.numpy(), bits(Bm), bits(Cm), D.numpy(),
                                 bits(z), None)
    assert np.abs(y - skip).max() < 1e-12
    for zero in ("B", "C"):
        Bz = torch.zeros_like(Bm) if zero == "B" else Bm
        Cz = torch.zeros_like(Cm) if zero == "C" else Cm
        _, y = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bz), bits(Cz),
                                     D.numpy(), bits(z), bias.numpy())
        assert np.abs(y - skip).max() < 1e-12
    # L = 1: y = (sum_n C_n delta B_n u + D u) silu(z)
    _, y1 = oracle.selective_scan(bits(u[..., :1]), bits(dr[..., :1]), A.numpy(),
                                  bits(Bm[..., :1]), bits(Cm[..., :1]), D.numpy(),
                                  bits(z[..., :1]), bias.numpy())
    r = _f64(dr)[0, :, 0] + _f64(bias)
    dl = np.log1p(np.exp(r))
    bc = float(_f64(Bm)[0, :, 0] @ _f64(Cm)[0, :, 0])
    want = (bc * dl * uf[0, :, 0] + Df * uf[0, :, 0]) * gate[0, :, 0]
    assert np.abs(y1[0, :, 0] - want).max() < 1e-12


def test_scan_closed_form_table_matches_oracle():
    """The expected outputs of the longest-sequence GPU test come from
    helpers.steady_scan_table; here they are held to the oracle on the same
    inputs over 300 steps, past the 200 after which the test uses the
    period."""
    d, L, n, warm = 3, 300, 16, 200
    t = np.arange(L)
    u = torch.tensor(np.stack([((5 * t + c) % 9) - 4 for c in range(d)])[None],
                     dtype=torch.bfloat16)
    dr = torch.full((1, d, L), 0.5, dtype=torch.bfloat16)
    ones = torch.ones((1, n, L), dtype=torch.bfloat16)
    A = np.full((d, n), -1.0, dtype=np.float32)
    _, y = oracle.selective_scan(bits(u), bits(dr), A, bits(ones), bits(ones), softplus=False)
    head, period = steady_scan_table(d, warm)
    want = np.concatenate([head, period[:, (t[warm:] - warm) % 9]], axis=1)
    assert np.abs(y[0] - want).max() < 1e-9 * np.abs(want).max()


def test_periodic_attention_closed_form_matches_oracle():
    """The expected outputs of the longest-sequence prefill and decode GPU
    tests come from helpers.periodic_attention; here they are held to the
    oracle's HTile attention on the same construction over 1000 keys (28
    full periods and a partial one), and its residue and segment counting to
    a direct sum over the keys."""
    S, D, q0 = 1000, 128, [2.0, 8.0]
    c = np.arange(S) % 35
    K = np.zeros((S, D))
    K[:, 0], K[:, D - 1] = periodic_k0(c), periodic_k127(c)
    K[:, 1:D - 1] = (c[:, None] + np.arange(1, D - 1)[None, :]) % 11 - 5
    V = periodic_vper(c[:, None], np.arange(D)[None, :])
    Q = np.zeros((len(q0), D))
    Q[:, 0] = Q[:, D - 1] = q0
    q, k, v = (torch.tensor(a[None, None], dtype=torch.bfloat16) for a in (Q, K, V))
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.BF16, False, 0.0)
    want_o, want_lse = periodic_attention(q0, S, 1.0 / math.sqrt(D))
    got = oracle.decode(o, oracle.BF16)[0, 0]
    assert np.abs(got - want_o).max() <= 2.0 ** -8 * np.abs(want_o).max()
    assert np.abs(lse[0, 0] - want_lse).max() < 1e-5
    # the residue and segment sums against the sums over every key, with a
    # step of 4 in V every 64 keys standing in for every 2^24
    sc = np.float32(1.0 / math.sqrt(D) * 1.4426950408889634)
    s = (np.float32(q0[1]) * (periodic_k0(c) + periodic_k127(c))).astype(np.float32)
    p = np.exp2((s * sc - np.float32(s.max() * sc)).astype(np.float32).astype(np.float64))
    p16 = torch.tensor(p, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    Vseg = V + 4.0 * (np.arange(S) >> 6)[:, None]
    seg_o, _ = periodic_attention(q0[1:], S, 1.0 / math.sqrt(D), seg_shift=4.0, seg_bits=6)
    assert np.abs(p16 @ Vseg / p.sum() - seg_o[0]).max() < 1e-12


def test_scan_linear_in_u():
    u, dr, A, Bm, Cm, D, z, bias = _scan_in(1, 3, 50, 16, 95)
    args = (A.numpy(), bits(Bm), bits(Cm), D.numpy(), bits(z), bias.numpy())
    _, y = oracle.selective_scan(bits(u), bits(dr), *args)
    _, y2 = oracle.selective_scan(bits(u * 2), bits(dr), *args)   # exact in bf16
    assert np.abs(y2 - 2 * y).max() <= 1e-12 * max(1.0, np.abs(y).max())


def test_planted_scan_sign_error_is_caught():
    """Feeding +exp instead of -exp for A (a sign slip) diverges from the
    brute force by far more than the tolerance."""
    u, dr, A, Bm, Cm, D, z, bias = _scan_in(1, 2, 30, 16, 99)
    _, y = oracle.selective_scan(bits(u), bits(dr), (-A).numpy(), bits(Bm), bits(Cm), D.numpy(),
                                 bits(z), bias.numpy())
    ref = brute_scan(_f64(u), _f64(dr), _f64(A), _f64(Bm), _f64(Cm), _f64(D), _f64(z),
                     _f64(bias))
    assert np.abs(y - ref).max() > 1.0
