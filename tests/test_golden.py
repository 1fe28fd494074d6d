"""The CPU oracle against the committed golden fixtures (tests/golden/).

The fixtures' expected outputs come from tests/golden/make_golden.py, a
float64 numpy restatement that shares no code with the oracle, so each test
here pins an oracle function against an independent computation:

  * E4M3 decode: all 256 codes, bit for bit (NaN where the format has it);
  * E4M3 encode + per-block scale: the fixture's codes and scales exactly;
  * attention closed form (fp64) to 1e-6 relative, and the HTile-policy
    kernel restatement to the dtype's tolerance;
  * split-K decode (bf16 and fp8 KV) to the decode tolerances;
  * the sequential scan (fp64) to 1e-6 relative.
"""

from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import TOL_BF16_ABS, TOL_F32_REL, TOL_FP8_ABS, TOL_LSE_ABS

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_fixture_files_present():
    names = {p.stem for p in GOLDEN.glob("*.npz")}
    assert {"e4m3_table", "attn_c1_fp32", "attn_f16_mha", "attn_bf16_causal_gqa",
            "decode_bf16_gqa", "decode_fp8", "scan_small", "scan_plain"} <= names


def test_e4m3_decode_matches_table():
    g = load("e4m3_table")
    got = oracle.decode(g["codes"], oracle.FP8).astype(np.float64)
    want = g["values"]
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan] == want[~nan]).all()


@pytest.mark.parametrize("name,dtype,tol", [
    ("attn_c1_fp32", oracle.F32, None),
    # f16: the reference's own functional-test tolerance, atol 1e-3
    # (tests/test_translators.py:143 in Evan-Zhao/mlir-toy)
    ("attn_f16_mha", oracle.F16, 1e-3),
    ("attn_bf16_causal_gqa", oracle.BF16, TOL_BF16_ABS),
])
def test_attention_oracle_matches_golden(name, dtype, tol):
    g = load(name)
    causal = bool(g["causal"])
    o64, lse64 = oracle.attn_exact(g["q"], g["k"], g["v"], dtype, causal)
    assert rel_err(o64, g["o"]) <= 1e-6
    assert np.abs(lse64 - g["lse"]).max() <= 1e-5
    o, lse = oracle.attn_fwd(g["q"], g["k"], g["v"], dtype, causal)
    of = oracle.decode(o, dtype) if dtype == oracle.BF16 else o.astype(np.float32)
    if dtype == oracle.F32:
        assert rel_err(of, g["o"]) <= TOL_F32_REL
    else:
        assert np.abs(of.astype(np.float64) - g["o"]).max() <= tol
    assert np.abs(lse - g["lse"]).max() <= TOL_LSE_ABS


def test_decode_oracle_matches_golden():
    g = load("decode_bf16_gqa")
    o, lse, _ = oracle.decode_splitk(g["q"], g["k"], g["v"], oracle.BF16,
                                     num_splits=int(g["num_splits"]))
    of = oracle.decode(o, oracle.BF16).astype(np.float64)
    err = np.abs(of - g["o"]).max()
    assert err <= TOL_BF16_ABS and err <= 2e-2 * np.abs(g["o"]).max()
    assert np.abs(lse - g["lse"]).max() <= TOL_LSE_ABS


def test_kv_quantize_oracle_matches_golden_codes():
    g = load("decode_fp8")
    b = load("decode_bf16_gqa")
    sb = int(g["scale_block"])
    for name in ("k", "v"):
        codes, scales = oracle.kv_quantize_fp8(b[name], scale_block=sb)
        assert (scales == g[name + "_scale"]).all()
        assert (codes == g[name + "_codes"]).all()


def test_decode_fp8_oracle_matches_golden():
    g = load("decode_fp8")
    o, lse, _ = oracle.decode_splitk(g["q"], g["k_codes"], g["v_codes"], oracle.FP8,
                                     k_scale=g["k_scale"], v_scale=g["v_scale"],
                                     num_splits=int(g["num_splits"]),
                                     scale_block=int(g["scale_block"]))
    of = oracle.decode(o, oracle.BF16).astype(np.float64)
    # against the dequantised closed form: only the kernel policy's rounding
    err = np.abs(of - g["o"]).max()
    assert err <= TOL_BF16_ABS and err <= 2e-2 * np.abs(g["o"]).max()
    # end to end against bf16 KV: quantisation error included
    assert np.abs(of - g["o_bf16_kv"]).max() <= TOL_FP8_ABS
    assert np.abs(lse - g["lse"]).max() <= TOL_LSE_ABS


@pytest.mark.parametrize("name", ["scan_small", "scan_plain"])
def test_scan_oracle_matches_golden(name):
    g = load(name)
    softplus = name == "scan_small"
    y, y64 = oracle.selective_scan(g["u"], g["delta"], g["A"], g["B"], g["C"], g.get("D"),
                                   g.get("z"), g.get("delta_bias"), softplus=softplus)
    assert rel_err(y64, g["y"]) <= 1e-6
    yb = oracle.decode(y, oracle.BF16).astype(np.float64)
    assert (np.abs(yb - g["y"]) <= 2e-2 * np.maximum(1.0, np.abs(g["y"]))).all()
