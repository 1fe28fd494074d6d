"""GPU parity of the prefill kernel's knobs: pipeline_stages and k_dim_order.

* pipeline_stages only changes how far ahead the K/V tiles are staged in
  LDS, not the arithmetic: stages 1 and 3 equal the default (2) bit for bit,
  across ragged, causal and GQA shapes.
* k_dim_order = 1 takes K as [B, Hkv, D, Skv] (the order of a
  dimension_order = [1, 0] tile load) and forms the MFMA operand with
  transpose reads. It is checked against the CPU oracle on the same K^T
  buffer (which the oracle reads in that order, and which it shows equal to
  the [S, D] form), for every stage count, contiguous and as a strided view.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL_BF16_ABS, TOL_LSE_ABS, bits, max_abs, oracle_dtype, randn, to_f32

pytestmark = pytest.mark.gpu

SHAPES = [  # B, Hq, Hkv, Sq, Sk
    (1, 4, 4, 300, 300),
    (2, 8, 2, 128, 1000),
    (1, 2, 1, 77, 200),
    (1, 2, 2, 40, 40),
    (1, 8, 8, 1024, 1024),
]


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def _inputs(shape, dtype, seed):
    B, Hq, Hk, Sq, Sk = shape
    q = randn((B, Hq, Sq, 128), seed=seed, dtype=dtype)
    k = randn((B, Hk, Sk, 128), seed=seed + 1, dtype=dtype)
    v = randn((B, Hk, Sk, 128), seed=seed + 2, dtype=dtype)
    return q, k, v


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stages_are_bitwise_equal(ops, shape, causal, dtype):
    _log(f"case: stages 1/2/3 shape={shape} causal={causal} dtype={dtype}")
    q, k, v = (t.cuda() for t in _inputs(shape, dtype, seed=70))
    ref, ref_lse = ops.attention(q, k, v, causal=causal, return_lse=True)
    for stages in (1, 3):
        o, lse = ops.attention(q, k, v, causal=causal, return_lse=True, pipeline_stages=stages)
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16)), stages
        assert torch.equal(lse, ref_lse), stages


@pytest.mark.parametrize("shape", [s for s in SHAPES if s[4] % 8 == 0])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k_dim_order_matches_oracle(ops, shape, causal, dtype):
    _log(f"case: k_dim_order=1 shape={shape} causal={causal} dtype={dtype}")
    q, k, v = _inputs(shape, dtype, seed=80)
    kt = k.transpose(2, 3).contiguous()
    ro, rl = oracle.attn_fwd(bits(q), bits(kt), bits(v), oracle_dtype(q), causal, k_dim_order=1)
    ref = oracle.decode(ro, oracle_dtype(q))
    qc, ktc, vc = q.cuda(), kt.cuda(), v.cuda()
    outs = []
    for stages in (2, 1, 3):
        o, lse = ops.attention(qc, ktc, vc, causal=causal, return_lse=True,
                               pipeline_stages=stages, k_dim_order=1)
        torch.cuda.synchronize()
        got = to_f32(o)
        assert max_abs(got, ref) <= TOL_BF16_ABS, stages
        assert max_abs(to_f32(lse), rl) <= TOL_LSE_ABS, stages
        outs.append(o)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


def test_k_dim_order_strided_view(ops):
    """K^T rows padded to a longer stride (a view into a larger buffer)."""
    _log("case: k_dim_order=1 strided view")
    B, Hq, Hk, S = 2, 4, 2, 520
    q, k, v = _inputs((B, Hq, Hk, S, S), torch.bfloat16, seed=90)
    buf = torch.zeros((B, Hk, 128, S + 24), dtype=torch.bfloat16)
    buf[..., :S] = k.transpose(2, 3)
    kt_view = buf.cuda()[..., :S]
    assert kt_view.stride(2) == S + 24
    o = ops.attention(q.cuda(), kt_view, v.cuda(), causal=True, k_dim_order=1)
    o_ref = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=True)
    torch.cuda.synchronize()
    ro, _ = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.BF16, True)
    assert max_abs(to_f32(o), oracle.decode(ro, oracle.BF16)) <= TOL_BF16_ABS
    assert max_abs(to_f32(o), to_f32(o_ref)) <= TOL_BF16_ABS
