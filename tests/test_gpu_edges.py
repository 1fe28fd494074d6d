"""GPU parity at the edges of each path, against the CPU oracle.

- Decode with caches shorter than one 32-token step, one token past a step,
  and more splits than steps: the layout then leaves whole splits empty,
  and the combine must weigh them zero.
- The head_dim-128 prefill kernel with one query row, one key, and more
  queries than keys under the causal mask. The early rows then see no key
  at all and must give O = 0 and LSE = -inf.
- The selective scan at sequence lengths 1, 2 and 3 and one step either side
  of its 32-step chunk, over a channel count that leaves a partial channel
  block.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_FP8_ABS, TOL_LSE_ABS, bits, max_abs, oracle_dtype,
                     periodic_attention, periodic_k0, periodic_k127, periodic_vper, randn,
                     to_f32)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("L", [1, 31, 32, 33, 100])
@pytest.mark.parametrize("splits", [1, 16])
def test_decode_short_caches(ops, L, splits):
    _log(f"case: decode bf16 short cache L={L} splits={splits}")
    B, Hq, Hk = 2, 8, 2
    q = randn((B, Hq, 128), seed=70)
    k = randn((B, Hk, L, 128), seed=71)
    v = randn((B, Hk, L, 128), seed=72)
    o, lse = ops.decode_splitk(q.cuda(), k.cuda(), v.cuda(), num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16,
                                             num_splits=splits)
    ref = oracle.decode(ref_o, oracle.BF16)
    got = to_f32(o)
    assert np.isfinite(got).all()
    assert max_abs(got, ref) <= TOL_BF16_ABS
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS
    if L == 1:
        # one key: the softmax weight is exactly 1, so O is that key's V row
        # (rounded to bf16 twice at most)
        want = np.repeat(to_f32(v)[:, :, 0, :], Hq // Hk, axis=1)
        assert max_abs(got, want) <= 1e-2 * np.abs(want).max()


@pytest.mark.parametrize("L", [1, 33, 100])
def test_decode_fp8_short_caches(ops, L):
    _log(f"case: decode fp8 short cache L={L} splits=16")
    B, Hq, Hk, splits = 2, 8, 2, 16
    q = randn((B, Hq, 128), seed=73)
    k = randn((B, Hk, L, 128), seed=74)
    v = randn((B, Hk, L, 128), seed=75)
    kc, ks = ops.kv_quantize_fp8(k.cuda())
    vc, vs = ops.kv_quantize_fp8(v.cuda())
    o, lse = ops.decode_splitk(q.cuda(), kc, vc, k_scale=ks, v_scale=vs, num_splits=splits,
                               return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse, _ = oracle.decode_splitk(bits(q), kc.cpu().numpy(), vc.cpu().numpy(),
                                             oracle.FP8, ks.cpu().numpy(), vs.cpu().numpy(),
                                             num_splits=splits)
    ref = oracle.decode(ref_o, oracle.BF16)
    got = to_f32(o)
    assert np.isfinite(got).all()
    assert max_abs(got, ref) <= TOL_FP8_ABS
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS


def _oracle_attn(q, k, v, causal):
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle_dtype(q), causal, 0.0)
    return oracle.decode(o, oracle_dtype(q)), lse


@pytest.mark.parametrize("Sq,Sk,causal", [
    (1, 1, False), (1, 1, True),       # one query, one key: O = V
    (1, 1000, False),                  # one query row over a ragged key range
    (1, 1000, True),                   # the last row of a causal block (sees every key)
    (300, 100, True),                  # rows 0..199 see no key: O = 0, LSE = -inf
    (129, 129, True),                  # one row past a 128-row block
])
def test_prefill_d128_edges(ops, Sq, Sk, causal):
    _log(f"case: prefill d128 bf16 Sq={Sq} Sk={Sk} causal={causal}")
    q = randn((1, 4, Sq, 128), seed=80, scale=0.5)
    k = randn((1, 2, Sk, 128), seed=81, scale=0.5)
    v = randn((1, 2, Sk, 128), seed=82, scale=0.5)
    out, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(q, k, v, causal)
    got, got_lse = to_f32(out), to_f32(lse)
    assert np.isfinite(got).all()
    assert max_abs(got, ref_o) <= TOL_BF16_ABS
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(ref_lse))
    fin = np.isfinite(ref_lse)
    assert max_abs(got_lse[fin], ref_lse[fin]) <= TOL_LSE_ABS
    if causal and Sq > Sk:
        dark = Sq - Sk  # bottom-right alignment: row r sees keys 0 .. r - (Sq - Sk)
        assert (got[:, :, :dark] == 0).all() and np.isneginf(got_lse[:, :, :dark]).all()


@pytest.mark.parametrize("L", [1, 2, 3, 31, 33])
def test_scan_short_sequences(ops, L):
    _log(f"case: scan short sequence L={L}")
    b, d, n = 2, 17, 16
    u, dr, z = (randn((b, d, L), seed=s) for s in (90, 91, 92))
    Bm, Cm = (randn((b, n, L), seed=s) for s in (93, 94))
    A = -torch.exp(randn((d, n), seed=95, dtype=torch.float32))
    D = randn((d,), seed=96, dtype=torch.float32)
    bias = randn((d,), seed=97, dtype=torch.float32)
    y = ops.selective_scan(u.cuda(), dr.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), D.cuda(),
                           z.cuda(), bias.cuda())
    torch.cuda.synchronize()
    ref_bits, _ = oracle.selective_scan(bits(u), bits(dr), A.numpy(), bits(Bm), bits(Cm),
                                        D.numpy(), bits(z), bias.numpy())
    ref = oracle.decode(ref_bits, oracle.BF16).astype(np.float64)
    got = to_f32(y).astype(np.float64)
    assert np.isfinite(got).all()
    assert (np.abs(got - ref) <= 2e-2 * np.maximum(1.0, np.abs(ref))).all()


def test_prefill_longest_kt_keys_closed_form(ops):
    """K stored [B, H, D, S] (k_dim_order = 1) at the longest seq_kv the
    head_dim-128 kernel accepts there: 127 S 2 + 256 < 2^32 bytes of per-lane
    offset, S = 16,909,312 (a multiple of 8). The last head_dim row of a K^T
    tile then sits nearly 4 GiB past the tile's base. Four query rows
    q = 2 (r + 1) (e_0 + e_127) score key j by K's rows 0 and 127 (periods 5
    and 7 in j; the other rows carry other patterns that q does not see), and
    V is periodic in j with period 35 plus a step of 32 at key 2^24 (V's
    first 4 GiB end there), so O and the LSE have the closed form of
    helpers.periodic_attention. A K row or key read from the wrong place
    changes the pairing of scores and values, and a V row read 4 GiB low
    loses the step; either fails. The oracle is not run over 16.9M keys."""
    S, D, rows = 16_909_312, 128, 4
    assert 127 * S * 2 + 256 < 1 << 32 <= 127 * (S + 8) * 2 + 256
    _log(f"case: prefill d128 k_dim_order=1 closed form Sk={S}")
    dev = "cuda"
    jm = torch.arange(S, device=dev, dtype=torch.int32) % 35
    kt = torch.empty((1, 1, D, S), dtype=torch.bfloat16, device=dev)
    kt[0, 0, 0] = periodic_k0(jm).to(torch.bfloat16)
    kt[0, 0, D - 1] = periodic_k127(jm).to(torch.bfloat16)
    for d in range(1, D - 1):
        kt[0, 0, d] = ((jm + d) % 11 - 5).to(torch.bfloat16)
    v = torch.empty((1, 1, S, D), dtype=torch.bfloat16, device=dev)
    dcol = torch.arange(D, device=dev, dtype=torch.int32)
    step = 1 << 21
    for s0 in range(0, S, step):
        seg = 32 * (torch.arange(s0, min(s0 + step, S), device=dev, dtype=torch.int32) >> 24)
        v[0, 0, s0:s0 + step] = (periodic_vper(jm[s0:s0 + step, None], dcol[None, :]) +
                                 seg[:, None]).to(torch.bfloat16)
    del jm
    q0 = [2.0 * (r + 1) for r in range(rows)]
    q = torch.zeros((1, 1, rows, D), dtype=torch.bfloat16, device=dev)
    q[0, 0, :, 0] = torch.tensor(q0, dtype=torch.bfloat16)
    q[0, 0, :, D - 1] = torch.tensor(q0, dtype=torch.bfloat16)
    out, lse = ops.attention(q, kt, v, return_lse=True, k_dim_order=1)
    torch.cuda.synchronize()
    want_o, want_lse = periodic_attention(q0, S, 1.0 / np.sqrt(D), seg_shift=32.0)
    got_o, got_lse = to_f32(out)[0, 0], to_f32(lse)[0, 0]
    assert np.isfinite(got_o).all()
    # |O| reaches 5 here, and both the bf16 rounding of P (where v_exp_f32's
    # last bit can flip it) and that of O are relative: 2e-2 of max(1, |O|),
    # against changes of order 1 from a misplaced row or key
    err = np.abs(got_o - want_o)
    assert (err <= TOL_BF16_ABS * np.maximum(1.0, np.abs(want_o))).all(), err.max()
    assert max_abs(got_lse, want_lse) <= TOL_LSE_ABS, (got_lse, want_lse)
