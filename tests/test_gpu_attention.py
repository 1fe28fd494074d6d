"""GPU parity of the HTile attention tile program (neptune_attn_fwd).

Every HIP result is compared with the CPU oracle (oracle/neptune_oracle.c,
HTile policy) on the same seeded inputs; the fp16 case at the reference's
own shape is also checked the way the reference checks its generated
kernels (tests/test_translators.py:106-143: fp32 torch reference,
rtol=0, atol=1e-3).
"""

import math

import numpy as np
import pytest
import torch

import oracle
from helpers import (TOL_BF16_ABS, TOL_F32_REL, TOL_LSE_ABS, bits, max_abs,
                     oracle_dtype, randn, to_f32)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def _oracle_attn(q, k, v, causal, scale_log2=0.0):
    o, lse = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle_dtype(q), causal, scale_log2)
    return oracle.decode(o, oracle_dtype(q)), lse


def test_config1_fp32_matches_oracle(ops):
    """fp32, B=1 H=1 S=128 D=64, non-causal, N(0,1)."""
    _log("case: config1 fp32 [1,1,128,64]")
    q, k, v = (randn((1, 1, 128, 64), seed=s, dtype=torch.float32) for s in (0, 1, 2))
    out, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(q, k, v, causal=False)
    got = to_f32(out)
    assert np.isfinite(got).all()
    assert max_abs(got, ref_o) <= TOL_F32_REL * np.abs(ref_o).max()
    exact, exact_lse = oracle.attn_exact(bits(q), bits(k), bits(v), oracle.F32)
    assert max_abs(got, exact) <= TOL_F32_REL * np.abs(exact).max()
    assert max_abs(to_f32(lse), exact_lse) <= 1e-5 * np.abs(exact_lse).max()


@pytest.mark.parametrize("B,Hq,Hk,Sq,Sk,D,causal", [
    (2, 4, 2, 100, 100, 32, True),    # GQA, a partial 16-row block, causal
    (1, 2, 1, 70, 300, 128, False),   # queries shorter than keys, ragged key block
    (1, 2, 2, 33, 33, 64, True),      # a row block holding one valid row
    (1, 1, 1, 200, 150, 64, True),    # more queries than keys: early rows see no key
])
def test_fp32_shapes_match_oracle(ops, B, Hq, Hk, Sq, Sk, D, causal):
    """The fp32 path (16 lanes per query row, each over every 16th key, merged
    at the end) at 1e-5 relative of the oracle, LSE included; rows with no
    visible key give O = 0 and LSE = -inf."""
    _log(f"case: fp32 B={B} Hq={Hq} Hk={Hk} Sq={Sq} Sk={Sk} D={D} causal={causal}")
    q = randn((B, Hq, Sq, D), seed=11, dtype=torch.float32)
    k = randn((B, Hk, Sk, D), seed=12, dtype=torch.float32)
    v = randn((B, Hk, Sk, D), seed=13, dtype=torch.float32)
    out, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(q, k, v, causal)
    got = to_f32(out)
    assert np.isfinite(got).all()
    assert max_abs(got, ref_o) <= TOL_F32_REL * np.abs(ref_o).max()
    got_lse = to_f32(lse)
    assert np.array_equal(np.isneginf(got_lse), np.isneginf(ref_lse))
    fin = np.isfinite(ref_lse)
    assert max_abs(got_lse[fin], ref_lse[fin]) <= 1e-5 * np.abs(ref_lse[fin]).max()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 64])
def test_prefill_small_matches_oracle(ops, causal, dtype, head_dim):
    _log(f"case: prefill small causal={causal} dtype={dtype} D={head_dim}")
    shape = (2, 3, 384, head_dim)
    q, k, v = (randn(shape, seed=10 + s, dtype=dtype, scale=0.5) for s in range(3))
    out, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(q, k, v, causal)
    assert max_abs(to_f32(out), ref_o) <= TOL_BF16_ABS
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_gqa_ragged(ops, causal):
    """Grouped KV heads, sequence not a multiple of the 128/64 tiles, Sq < Sk."""
    _log(f"case: prefill gqa ragged causal={causal}")
    q = randn((2, 8, 300, 128), seed=20, scale=0.5)
    k = randn((2, 2, 333, 128), seed=21, scale=0.5)
    v = randn((2, 2, 333, 128), seed=22, scale=0.5)
    out, lse = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(q, k, v, causal)
    assert max_abs(to_f32(out), ref_o) <= TOL_BF16_ABS
    assert max_abs(to_f32(lse), ref_lse) <= TOL_LSE_ABS


def test_prefill_strided_views(ops):
    """[B, S, H, D] storage read through transposed views (non-contiguous)."""
    _log("case: prefill strided views")
    base = [randn((2, 256, 4, 128), seed=30 + s, scale=0.5) for s in range(3)]
    q, k, v = (t.cuda().transpose(1, 2) for t in base)
    out, lse = ops.attention(q, k, v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = _oracle_attn(*(t.transpose(1, 2).contiguous() for t in base), causal=True)
    assert max_abs(to_f32(out), ref_o) <= TOL_BF16_ABS


def test_prefill_custom_scale(ops):
    _log("case: prefill custom scale")
    q, k, v = (randn((1, 2, 256, 128), seed=40 + s, scale=0.5) for s in range(3))
    out = ops.attention(q.cuda(), k.cuda(), v.cuda(), scale=0.3)
    torch.cuda.synchronize()
    ref_o, _ = _oracle_attn(q, k, v, False, scale_log2=float(np.float32(0.3 * math.log2(math.e))))
    assert max_abs(to_f32(out), ref_o) <= TOL_BF16_ABS


def test_reference_htile_shape_fp16(ops):
    """The reference's functional test: fp16 (1, 32, 4096, 128) non-causal,
    N(0,1) inputs, fp32 torch reference computed in 128-row blocks,
    assert_close(rtol=0, atol=1e-3) (tests/test_translators.py:106-143)."""
    _log("case: reference htile shape fp16 [1,32,4096,128]")
    g = torch.Generator(device="cuda").manual_seed(0)
    shape = (1, 32, 4096, 128)
    q = torch.randn(shape, dtype=torch.float16, device="cuda", generator=g)
    k = torch.randn(shape, dtype=torch.float16, device="cuda", generator=g)
    v = torch.randn(shape, dtype=torch.float16, device="cuda", generator=g)
    out = ops.attention(q, k, v)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and tuple(out.shape) == shape
    assert bool(torch.isfinite(out).all())
    ref = torch.empty(shape, dtype=torch.float32, device="cuda")
    k_t = k.transpose(-1, -2).float().contiguous()
    v_f = v.float()
    for r0 in range(0, shape[2], 128):
        scores = torch.matmul(q[:, :, r0:r0 + 128, :].float(), k_t)
        probs = torch.softmax(scores * (1.0 / math.sqrt(shape[3])), dim=-1)
        ref[:, :, r0:r0 + 128, :] = torch.matmul(probs, v_f)
    torch.testing.assert_close(out.float(), ref, rtol=0, atol=1e-3)


def test_config2_full_shape(ops):
    """BASELINE config 2 at full size: causal bf16 B=4 H=32 S=4096 D=128,
    Q,K,V ~ 0.5 N(0,1). Sampled heads against the oracle; every head's
    first row is exactly V[0] (causal row 0 sees only key 0, p = 1)."""
    _log("case: config2 full shape [4,32,4096,128] causal bf16")
    shape = (4, 32, 4096, 128)
    g = torch.Generator(device="cuda").manual_seed(2)
    q, k, v = (torch.randn(shape, device="cuda", generator=g).mul_(0.5).to(torch.bfloat16)
               for _ in range(3))
    out, lse = ops.attention(q, k, v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    assert torch.equal(out[:, :, 0, :], v[:, :, 0, :])
    for b, h in ((0, 0), (3, 31), (1, 17)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        ref_o, ref_lse = _oracle_attn(q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), True)
        assert max_abs(to_f32(out[sl]), ref_o) <= TOL_BF16_ABS, (b, h)
        assert max_abs(to_f32(lse[sl]), ref_lse) <= TOL_LSE_ABS, (b, h)


def test_config2_full_shape_linear_in_v(ops):
    """Config 2 at full size, every head and row: O(2V) = 2 O(V) bit for bit
    and the same LSE. The scores, maxima, rescale decisions and P do not
    depend on V; doubling V doubles every P.V product and fp32 partial sum
    exactly, and commutes with the division by l and the bf16 rounding, so
    any output row whose work differs between the two calls breaks it."""
    _log("case: config2 linear in V")
    shape = (4, 32, 4096, 128)
    g = torch.Generator(device="cuda").manual_seed(21)
    q, k, v = (torch.randn(shape, device="cuda", generator=g).mul_(0.5).to(torch.bfloat16)
               for _ in range(3))
    o1, lse1 = ops.attention(q, k, v, causal=True, return_lse=True)
    o2, lse2 = ops.attention(q, k, 2 * v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o1).all())
    assert torch.equal(lse1, lse2)
    assert torch.equal(o2, 2 * o1)


def test_q_zero_gives_prefix_mean(ops):
    """Q = 0: uniform weights, so row i is the mean of V[0..i] (causal)."""
    _log("case: q zero prefix mean")
    v = randn((1, 2, 256, 128), seed=50, scale=1.0)
    k = randn((1, 2, 256, 128), seed=51, scale=1.0)
    q = torch.zeros_like(v)
    out = ops.attention(q.cuda(), k.cuda(), v.cuda(), causal=True)
    torch.cuda.synchronize()
    vf = v.double()
    prefix = vf.cumsum(dim=2) / torch.arange(1, 257, dtype=torch.float64).view(1, 1, -1, 1)
    assert max_abs(to_f32(out), prefix.numpy()) <= TOL_BF16_ABS


def test_host_lse_raises(ops):
    """A caller's lse in host memory is refused before any launch."""
    q = torch.zeros((1, 1, 64, 128), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty((1, 1, 64), dtype=torch.float32)
    with pytest.raises(ValueError):
        ops.attention(q, q, q, lse=lse)


def test_unsupported_head_dim_raises(ops):
    from neptune_hip import NeptuneUnsupported
    q = torch.zeros((1, 1, 64, 96), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NeptuneUnsupported):
        ops.attention(q, q, q)
