"""GPU parity of the lazy softmax rescale under scores that climb block by block.

Random inputs keep every key block's scores near the running max, so the
kernels' rescale paths run on the first block only. Here the keys are
built so that, against q of all ones, the log2-domain scores step through:
  blocks 0-3    around 0
  block 4       +12: the block max passes m + 8, so m moves and O, l rescale
  blocks 5-7    back to 0
  block 8       +242: 2^(s - m) against the old m overflows fp32 to inf
  blocks 9-11   +239
  block 12      +248 on every other key: p = 2^6 each, so a lane's sum
                passes 2^8 while no p does (the max is formed, m stays)
  blocks 13-    +239
Prefill (head_dim 128, bf16 and f16, causal and not) and split-K decode
(bf16 and fp8 KV, splits that start inside the ramp) are checked against the
CPU oracle, which takes the plain running max.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL_BF16_ABS, TOL_FP8_ABS, TOL_LSE_ABS, bits, max_abs, oracle_dtype, to_f32

pytestmark = pytest.mark.gpu

D = 128
LOG2_PER_UNIT = D * 1.4426950408889634 / D ** 0.5  # log2 score of q = 1, k = 1 per element


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def ramp_targets(L):
    """log2-domain score of each key against q = 1 (see the module text)."""
    j = torch.arange(L)
    blk = j // 64
    t = torch.zeros(L)
    t[blk == 4] = 12.0
    t[blk >= 8] = 239.0
    t[blk == 8] = 242.0
    t[(blk == 12) & (j % 2 == 0)] = 248.0
    return t


def ramp_kv(B, H, L, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    base = (ramp_targets(L) / LOG2_PER_UNIT).view(1, 1, L, 1)
    k = base + 0.05 * torch.randn((B, H, L, D), generator=g)
    v = torch.randn((B, H, L, D), generator=g)
    return k.to(dtype), v.to(dtype)


def ramp_q(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.02 * torch.randn(shape, generator=g)).to(dtype)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_climbing_scores(ops, causal, dtype):
    _log(f"case: prefill climbing scores causal={causal} dtype={dtype}")
    B, H, S = 1, 2, 1024
    q = ramp_q((B, H, S, D), 1, dtype)
    k, v = ramp_kv(B, H, S, 2, dtype)
    o, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ro, rl = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle_dtype(q), causal)
    ref = oracle.decode(ro, oracle_dtype(q))
    got = to_f32(o)
    assert np.isfinite(got).all()
    assert max_abs(got, ref) <= TOL_BF16_ABS * max(1.0, np.abs(ref).max())
    assert max_abs(to_f32(lse), rl) <= TOL_LSE_ABS


@pytest.mark.parametrize("splits", [1, 3])
def test_decode_bf16_climbing_scores(ops, splits):
    _log(f"case: decode bf16 climbing scores splits={splits}")
    B, Hq, Hk, L = 2, 8, 2, 1024
    q = ramp_q((B, Hq, D), 3, torch.bfloat16)
    k, v = ramp_kv(B, Hk, L, 4, torch.bfloat16)
    o, lse = ops.decode_splitk(q.cuda(), k.cuda(), v.cuda(), num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    ro, rl, _ = oracle.decode_splitk(bits(q), bits(k), bits(v), oracle.BF16, num_splits=splits)
    ref = oracle.decode(ro, oracle.BF16)
    got = to_f32(o)
    assert np.isfinite(got).all()
    assert max_abs(got, ref) <= TOL_BF16_ABS * max(1.0, np.abs(ref).max())
    assert max_abs(to_f32(lse), rl) <= TOL_LSE_ABS


@pytest.mark.parametrize("splits", [1, 3])
def test_decode_fp8_climbing_scores(ops, splits):
    _log(f"case: decode fp8 climbing scores splits={splits}")
    B, Hq, Hk, L = 2, 8, 2, 1024
    q = ramp_q((B, Hq, D), 5, torch.bfloat16)
    k, v = ramp_kv(B, Hk, L, 6, torch.bfloat16)
    kc, ks = ops.kv_quantize_fp8(k.cuda())
    vc, vs = ops.kv_quantize_fp8(v.cuda())
    o, lse = ops.decode_splitk(q.cuda(), kc, vc, k_scale=ks, v_scale=vs, num_splits=splits,
                               return_lse=True)
    torch.cuda.synchronize()
    ro, rl, _ = oracle.decode_splitk(bits(q), kc.cpu().numpy(), vc.cpu().numpy(), oracle.FP8,
                                     ks.cpu().numpy(), vs.cpu().numpy(), num_splits=splits)
    ref = oracle.decode(ro, oracle.BF16)
    got = to_f32(o)
    assert np.isfinite(got).all()
    assert max_abs(got, ref) <= TOL_FP8_ABS * max(1.0, np.abs(ref).max())
    assert max_abs(to_f32(lse), rl) <= TOL_LSE_ABS
