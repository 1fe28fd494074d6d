"""HTile front end on the GPU: tile programs bound to neptune_attn_fwd and
launched as kernel[grid](q, k, v, out).

The first case is the reference's own functional test through this front
end (tests/test_translators.py:106-143 in Evan-Zhao/mlir-toy): f16
[1, 32, 4096, 128], grid (32, 32, 1), an fp32 torch reference computed in
128-row blocks, atol 1e-3. The others cover the post-pass program form,
bf16 and fp32 against the oracle, a grid / trip count that covers only
part of the tensors, and a program over a [B, H, D, S] k memref with its
pipeline_stages bound to the kernel.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL_BF16_ABS, TOL_F32_REL, bits, randn, to_f32
from htile_gen import program

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def htile():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import htile as _htile
    return _htile


def _log(msg):
    print(msg, flush=True)


def _torch_reference(q, k, v, rows=128):
    """softmax(q k^T / sqrt(D)) v in fp32, 128 query rows at a time."""
    ref = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    kt = k.float().transpose(-1, -2).contiguous()
    vf = v.float()
    scale = 1.0 / math.sqrt(q.shape[-1])
    for r0 in range(0, q.shape[2], rows):
        s = torch.matmul(q[:, :, r0:r0 + rows].float(), kt) * scale
        ref[:, :, r0:r0 + rows] = torch.matmul(torch.softmax(s, dim=-1), vf)
    return ref


def test_reference_functional_case(htile):
    _log("case: htile f16 [1,32,4096,128] grid (32,32,1)")
    kern = htile.translate_source(program()).flash_attention_htile
    shape = (1, 32, 4096, 128)
    q, k, v = (randn(shape, seed=s, dtype=torch.float16, device="cuda") for s in (0, 1, 2))
    out = torch.empty(shape, dtype=torch.float16, device="cuda")
    kern[(32, 32, 1)](q, k, v, out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    ref = _torch_reference(q, k, v)
    torch.testing.assert_close(out.float(), ref, rtol=0, atol=1e-3)


@pytest.mark.parametrize("form", ["pre", "post"])
def test_bf16_program_matches_oracle(htile, form):
    _log(f"case: htile bf16 form={form}")
    shape = (2, 4, 512, 64)
    kern = htile.translate_source(program(B=2, H=4, S=512, D=64, dtype="bf16", form=form,
                                          canonical=form == "post")).flash_attention_htile
    q, k, v = (randn(shape, seed=s, dtype=torch.bfloat16) for s in (3, 4, 5))
    out = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
    kern[kern.program.grid](q.cuda(), k.cuda(), v.cuda(), out)
    torch.cuda.synchronize()
    ref_o, _ = oracle.attn_fwd(bits(q), bits(k), bits(v), oracle.BF16, causal=False)
    ref = oracle.decode(ref_o, oracle.BF16)
    assert np.abs(to_f32(out) - ref).max() <= TOL_BF16_ABS


def test_fp32_program_config1(htile):
    _log("case: htile fp32 [1,1,128,64]")
    shape = (1, 1, 128, 64)
    kern = htile.translate_source(program(B=1, H=1, S=128, D=64, dtype="f32",
                                          bm=64, bn=32)).flash_attention_htile
    q, k, v = (randn(shape, seed=s, dtype=torch.float32) for s in (6, 7, 8))
    out = torch.empty(shape, dtype=torch.float32, device="cuda")
    kern[kern.program.grid](q.cuda(), k.cuda(), v.cuda(), out)
    torch.cuda.synchronize()
    ref64, _ = oracle.attn_exact(q.numpy(), k.numpy(), v.numpy(), oracle.F32, causal=False)
    err = np.abs(to_f32(out) - ref64).max() / np.abs(ref64).max()
    assert err <= TOL_F32_REL


def test_partial_grid_and_trip_count(htile):
    _log("case: htile partial grid (2,3,1), 4 key blocks")
    shape = (1, 4, 512, 64)
    kern = htile.translate_source(program(B=1, H=4, S=512, D=64, dtype="bf16", grid=(2, 3, 1),
                                          trip=4)).flash_attention_htile
    q, k, v = (randn(shape, seed=s, dtype=torch.bfloat16) for s in (9, 10, 11))
    out = torch.full(shape, 7.0, dtype=torch.bfloat16, device="cuda")
    kern[(2, 3, 1)](q.cuda(), k.cuda(), v.cuda(), out)
    torch.cuda.synchronize()
    got = to_f32(out)
    # rows [0, 256) of heads 0..2 attend to keys [0, 256); the rest is untouched
    ref_o, _ = oracle.attn_fwd(bits(q[:, :3, :256]), bits(k[:, :3, :256]), bits(v[:, :3, :256]),
                               oracle.BF16, causal=False)
    assert np.abs(got[:, :3, :256] - oracle.decode(ref_o, oracle.BF16)).max() <= TOL_BF16_ABS
    assert (got[:, :3, 256:] == 7.0).all() and (got[:, 3:] == 7.0).all()


@pytest.mark.parametrize("stages", [1, 3])
def test_transposed_k_program_and_stages(htile, stages):
    """A program over a [B, H, D, S] k memref (its K tile read in stored
    order) runs on the kernel's k_dim_order 1 path, with the loop's
    htile.pipeline_stages bound to the kernel; a partial trip count reads
    only the first keys of the transposed memref."""
    _log(f"case: htile K^T memref, stages={stages}")
    B, H, S, D = 1, 4, 512, 128
    kern = htile.translate_source(program(B=B, H=H, S=S, D=D, dtype="bf16", k_mem="ds",
                                          stages=stages, trip=6)).flash_attention_htile
    assert kern.program.k_dim_order == 1 and kern.program.pipeline_stages == stages
    q, k, v = (randn((B, H, S, D), seed=s, dtype=torch.bfloat16) for s in (12, 13, 14))
    out = torch.empty((B, H, S, D), dtype=torch.bfloat16, device="cuda")
    kern[kern.program.grid](q.cuda(), k.transpose(2, 3).contiguous().cuda(), v.cuda(), out)
    torch.cuda.synchronize()
    keys = 6 * 64
    ref_o, _ = oracle.attn_fwd(bits(q), bits(k[:, :, :keys]), bits(v[:, :, :keys]), oracle.BF16,
                               causal=False)
    assert np.abs(to_f32(out) - oracle.decode(ref_o, oracle.BF16)).max() <= TOL_BF16_ABS
