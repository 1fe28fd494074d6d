"""The HIP kernels against the committed golden fixtures (tests/golden/),
whose expected outputs are float64 closed forms computed by
tests/golden/make_golden.py independently of the oracle and the library.

Tolerances: fp32 1e-5 relative; f16 1e-3 absolute (the reference's own
functional-test bound, tests/test_translators.py:143 in Evan-Zhao/mlir-toy);
bf16 2e-2 absolute (and 2e-2 relative to max|ref| for decode, whose outputs
are small); fp8 KV 6e-2 end to end, absolute and relative to max|ref|; scan 2e-2 * max(1, |ref|); LSE 1e-3.
"""

import numpy as np
import pytest
import torch

from helpers import (TOL_BF16_ABS, TOL_BF16_REL, TOL_F32_REL, TOL_FP8_ABS, TOL_FP8_REL,
                     TOL_LSE_ABS, assert_rel_rows, from_bf16_bits, to_f32)
from test_golden import load, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from neptune_hip import ops as _ops
    return _ops


def _log(msg):
    print(msg, flush=True)


def _dev(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return from_bf16_bits(a).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("name,tol", [("attn_c1_fp32", None), ("attn_f16_mha", 1e-3),
                                      ("attn_bf16_causal_gqa", TOL_BF16_ABS)])
def test_attention_golden(ops, name, tol):
    _log(f"case: golden {name}")
    g = load(name)
    o, lse = ops.attention(_dev(g["q"]), _dev(g["k"]), _dev(g["v"]), causal=bool(g["causal"]),
                           return_lse=True)
    torch.cuda.synchronize()
    got = to_f32(o).astype(np.float64)
    if tol is None:
        assert rel_err(got, g["o"]) <= TOL_F32_REL
    else:
        assert np.abs(got - g["o"]).max() <= tol
    assert np.abs(to_f32(lse) - g["lse"]).max() <= TOL_LSE_ABS


def test_decode_golden(ops):
    _log("case: golden decode_bf16_gqa")
    g = load("decode_bf16_gqa")
    o, lse = ops.decode_splitk(_dev(g["q"]), _dev(g["k"]), _dev(g["v"]),
                               num_splits=int(g["num_splits"]), return_lse=True)
    torch.cuda.synchronize()
    err = np.abs(to_f32(o).astype(np.float64) - g["o"]).max()
    assert err <= TOL_BF16_ABS
    assert_rel_rows(to_f32(o), g["o"], TOL_BF16_REL, "golden bf16 decode")
    assert np.abs(to_f32(lse) - g["lse"]).max() <= TOL_LSE_ABS


def test_kv_quantize_golden(ops):
    _log("case: golden kv_quantize")
    g = load("decode_fp8")
    b = load("decode_bf16_gqa")
    for name in ("k", "v"):
        codes, scales = ops.kv_quantize_fp8(_dev(b[name]), scale_block=int(g["scale_block"]))
        torch.cuda.synchronize()
        assert (scales.cpu().numpy() == g[name + "_scale"]).all()
        assert (codes.cpu().numpy() == g[name + "_codes"]).all()


def test_decode_fp8_golden(ops):
    _log("case: golden decode_fp8")
    g = load("decode_fp8")
    o, lse = ops.decode_splitk(_dev(g["q"]), _dev(g["k_codes"]), _dev(g["v_codes"]),
                               k_scale=_dev(g["k_scale"]), v_scale=_dev(g["v_scale"]),
                               num_splits=int(g["num_splits"]),
                               scale_block=int(g["scale_block"]), return_lse=True)
    torch.cuda.synchronize()
    got = to_f32(o).astype(np.float64)
    err = np.abs(got - g["o"]).max()
    assert err <= TOL_BF16_ABS
    assert_rel_rows(got, g["o"], TOL_BF16_REL, "golden fp8 decode vs same codes")
    assert np.abs(got - g["o_bf16_kv"]).max() <= TOL_FP8_ABS
    assert_rel_rows(got, g["o_bf16_kv"], TOL_FP8_REL, "golden fp8 decode vs bf16 KV")
    assert np.abs(to_f32(lse) - g["lse"]).max() <= TOL_LSE_ABS


@pytest.mark.parametrize("name", ["scan_small", "scan_plain"])
def test_scan_golden(ops, name):
    _log(f"case: golden {name}")
    g = load(name)
    opt = lambda k: _dev(g[k]) if k in g else None
    y = ops.selective_scan(_dev(g["u"]), _dev(g["delta"]), _dev(g["A"]), _dev(g["B"]),
                           _dev(g["C"]), opt("D"), opt("z"), opt("delta_bias"),
                           delta_softplus=name == "scan_small")
    torch.cuda.synchronize()
    got = to_f32(y).astype(np.float64)
    assert (np.abs(got - g["y"]) <= 2e-2 * np.maximum(1.0, np.abs(g["y"]))).all()
