"""CPU tests of the torch front's argument checks (neptune_hip.ops).

The C-ABI sees pointers, not buffer sizes, so a mis-shaped tensor that got
past the Python front would be read out of bounds on the device. Every
shape, dtype and layout check runs before the device check, so these tests
drive them with meta tensors (no storage, no GPU) and expect ValueError,
the class the reference raises for bad input.
"""

import pytest
import torch

from neptune_hip import ops

bf16, f32, u8, i32 = torch.bfloat16, torch.float32, torch.uint8, torch.int32


def meta(shape, dtype=bf16):
    return torch.empty(shape, dtype=dtype, device="meta")


def _decode_args(B=2, Hq=8, Hk=2, L=256, D=128, fp8=False, sb=64):
    q = meta((B, Hq, D))
    k = meta((B, Hk, L, D), u8 if fp8 else bf16)
    v = meta((B, Hk, L, D), u8 if fp8 else bf16)
    sc = dict(k_scale=meta((B, Hk, -(-L // sb)), f32), v_scale=meta((B, Hk, -(-L // sb)), f32),
              scale_block=sb) if fp8 else {}
    return q, k, v, sc


def test_valid_decode_arguments_reach_the_device_check():
    q, k, v, sc = _decode_args(fp8=True)
    with pytest.raises(ValueError, match="device tensors"):
        ops.decode_splitk(q, k, v, **sc)


@pytest.mark.parametrize("change,match", [
    (dict(k=meta((3, 2, 256, 128)), v=meta((3, 2, 256, 128))), "batch or head_dim"),
    (dict(k=meta((2, 2, 256, 64)), v=meta((2, 2, 256, 64))), "batch or head_dim"),
    (dict(v=meta((2, 2, 255, 128))), "k and v must match"),
    (dict(k=meta((2, 2, 256, 128))[..., ::1].transpose(2, 3).transpose(2, 3)), None),
])
def test_decode_shape_mismatch(change, match):
    q, k, v, _ = _decode_args()
    args = dict(q=q, k=k, v=v)
    args.update(change)
    if match is None:  # a valid view: reaches the device check
        with pytest.raises(ValueError, match="device tensors"):
            ops.decode_splitk(**args)
        return
    with pytest.raises(ValueError, match=match):
        ops.decode_splitk(**args)


@pytest.mark.parametrize("which,bad,match", [
    ("k_scale", meta((2, 2, 2), f32), "k_scale"),       # scale_block 128's count, 64 given
    ("v_scale", meta((2, 2, 4), bf16), "v_scale"),      # wrong dtype
    ("k_scale", meta((2, 4, 2), f32).transpose(1, 2), "k_scale"),  # not contiguous
    ("v_scale", None, "v_scale"),                       # missing
])
def test_decode_fp8_scale_checks(which, bad, match):
    q, k, v, sc = _decode_args(fp8=True)
    sc[which] = bad
    with pytest.raises(ValueError, match=match):
        ops.decode_splitk(q, k, v, **sc)


def test_decode_scales_are_fp8_only():
    q, k, v, _ = _decode_args()
    with pytest.raises(ValueError, match="E4M3"):
        ops.decode_splitk(q, k, v, k_scale=meta((2, 2, 4), f32), v_scale=meta((2, 2, 4), f32))


def test_decode_scale_block_for_fp8_codes_quantised_at_128():
    """Codes quantised with 128-token scale blocks decoded with the default
    64 would index twice as many scales: rejected."""
    q, k, v, sc = _decode_args(fp8=True, sb=128)
    sc.pop("scale_block")
    with pytest.raises(ValueError, match="scale_block 64"):
        ops.decode_splitk(q, k, v, **sc)


def _paged_args(B=2, Hq=8, Hk=2, D=128, npages=16, psize=64, fp8=False):
    q = meta((B, Hq, D))
    pool = meta((npages, Hk, psize, D), u8 if fp8 else bf16)
    table = meta((B, 4), i32)
    lens = meta((B,), i32)
    sc = dict(k_scales=meta((npages, Hk), f32), v_scales=meta((npages, Hk), f32)) if fp8 else {}
    return q, pool, pool, table, lens, sc


def test_valid_paged_arguments_reach_the_device_check():
    for fp8 in (False, True):
        q, kp, vp, t, n, sc = _paged_args(fp8=fp8)
        with pytest.raises(ValueError, match="device tensors"):
            ops.decode_paged(q, kp, vp, t, n, **sc)


def test_paged_pool_head_dim_must_match_q():
    q, kp, vp, t, n, _ = _paged_args()
    pool64 = meta((16, 2, 64, 64))
    with pytest.raises(ValueError, match="head_dim"):
        ops.decode_paged(q, pool64, pool64, t, n)


def test_paged_checks_table_and_scales():
    q, kp, vp, t, n, sc = _paged_args(fp8=True)
    with pytest.raises(ValueError, match="k_scales"):
        ops.decode_paged(q, kp, vp, t, n, k_scales=meta((15, 2), f32), v_scales=sc["v_scales"])
    with pytest.raises(ValueError, match="block_table"):
        ops.decode_paged(q, kp, vp, meta((3, 4), i32), n, **sc)
    with pytest.raises(ValueError, match="int32"):
        ops.decode_paged(q, kp, vp, t, meta((2,), torch.int64), **sc)
    q, kp, vp, t, n, _ = _paged_args()
    with pytest.raises(ValueError, match="E4M3"):
        ops.decode_paged(q, kp, vp, t, n, k_scales=meta((16, 2), f32))


def _scan_args(Bn=2, Dm=64, L=128, N=16):
    return dict(u=meta((Bn, Dm, L)), delta=meta((Bn, Dm, L)), A=meta((Dm, N), f32),
                B=meta((Bn, N, L)), C=meta((Bn, N, L)), D=meta((Dm,), f32),
                z=meta((Bn, Dm, L)), delta_bias=meta((Dm,), f32))


def test_valid_scan_arguments_reach_the_device_check():
    with pytest.raises(ValueError, match="device tensors"):
        ops.selective_scan(**_scan_args())


@pytest.mark.parametrize("name,shape,dtype", [
    ("z", (2, 64, 127), bf16),
    ("z", (2, 32, 128), bf16),
    ("D", (63,), f32),
    ("delta_bias", (64, 1), f32),
    ("delta", (2, 64, 129), bf16),
    ("B", (2, 8, 128), bf16),
    ("C", (1, 16, 128), bf16),
    ("A", (32, 16), f32),
])
def test_scan_shape_checks(name, shape, dtype):
    args = _scan_args()
    args[name] = meta(shape, dtype)
    with pytest.raises(ValueError, match=name):
        ops.selective_scan(**args)
