"""The C-ABI driven from native C++ host code (tests/native/
neptune_abi_caller.cpp, built by __graft_entry__.build()): the program owns
its device buffers, calls include/neptune_hip.h's entry points and checks
the results itself, as a C++ runtime embedding the backend would (the
reference's plugin host finds its extern "C" entry by dlopen,
lib/HTile/HTileDialect.cpp:27-37).

On the CPU it exercises the host-side validation and the no-device path.
On the GPU it runs:
- neptune_attn_fwd on the attn_bf16_causal_gqa fixture;
- neptune_decode_splitk and neptune_decode_splitk_noalloc on decode_bf16_gqa
  and, with fp8 KV, on decode_fp8;
- neptune_selective_scan_fwd on scan_small.
The expected outputs are the fixtures' float64 closed forms."""

import os
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import TOL_BF16_ABS
from test_golden import load

ROOT = Path(__file__).resolve().parents[1]
# NEPTUNE_ABI_CALLER selects another build of the same program (the
# host-sanitizer build)
CALLER = Path(os.environ.get("NEPTUNE_ABI_CALLER") or
              ROOT / "tests" / "native" / "neptune_abi_caller")


def _run(*args):
    if not CALLER.is_file():
        pytest.fail(f"{CALLER} is not built: run __graft_entry__.build()")
    print("case: native caller", *args, flush=True)
    r = subprocess.run([str(CALLER), *map(str, args)], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr, flush=True)
    return r


def test_native_caller_validation():
    r = _run("validate")
    assert r.returncode == 0, r.stderr
    assert "validate: ok" in r.stdout


def _write(dirpath: Path, meta: dict, arrays: dict):
    dirpath.mkdir(parents=True, exist_ok=True)
    (dirpath / "meta.txt").write_text("".join(f"{k} {v}\n" for k, v in meta.items()))
    for name, a in arrays.items():
        np.ascontiguousarray(a).tofile(dirpath / f"{name}.bin")


@pytest.mark.gpu
def test_native_caller_attention_fixture(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    g = load("attn_bf16_causal_gqa")
    B, Hq, S, _ = g["q"].shape
    Hk, Sk = g["k"].shape[1], g["k"].shape[2]
    _write(tmp_path, dict(batch=B, heads_q=Hq, heads_kv=Hk, seq_q=S, seq_kv=Sk,
                          causal=int(g["causal"]), tol=TOL_BF16_ABS),
           dict(q=g["q"], k=g["k"], v=g["v"], o=g["o"].astype(np.float32),
                lse=g["lse"].astype(np.float32)))
    r = _run("attn", tmp_path)
    assert r.returncode == 0, r.stderr
    assert "attn: ok" in r.stdout


@pytest.mark.gpu
def test_native_caller_decode_fixture(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    g = load("decode_bf16_gqa")
    B, Hq, _ = g["q"].shape
    Hk, L = g["k"].shape[1], g["k"].shape[2]
    _write(tmp_path, dict(batch=B, heads_q=Hq, heads_kv=Hk, seq_kv=L,
                          num_splits=int(g["num_splits"]), tol=TOL_BF16_ABS),
           dict(q=g["q"], k=g["k"], v=g["v"], o=g["o"].astype(np.float32),
                lse=g["lse"].astype(np.float32)))
    r = _run("decode", tmp_path)
    assert r.returncode == 0, r.stderr
    assert "decode: ok" in r.stdout


@pytest.mark.gpu
def test_native_caller_fp8_decode_fixture(tmp_path):
    """fp8-E4M3 KV with per-block scales through both decode entry points;
    the expected output is the fixture's float64 closed form on the same
    codes and scales."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    g = load("decode_fp8")
    B, Hq, _ = g["q"].shape
    Hk, L = g["k_codes"].shape[1], g["k_codes"].shape[2]
    _write(tmp_path, dict(batch=B, heads_q=Hq, heads_kv=Hk, seq_kv=L,
                          num_splits=int(g["num_splits"]), scale_block=int(g["scale_block"]),
                          tol=TOL_BF16_ABS),
           dict(q=g["q"], k=g["k_codes"], v=g["v_codes"], k_scale=g["k_scale"],
                v_scale=g["v_scale"], o=g["o"].astype(np.float32),
                lse=g["lse"].astype(np.float32)))
    r = _run("fp8", tmp_path)
    assert r.returncode == 0, r.stderr
    assert "fp8: ok" in r.stdout


@pytest.mark.gpu
def test_native_caller_scan_fixture(tmp_path):
    """The selective scan with D, z and delta_bias (softplus on), against the
    fixture's float64 recurrence."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    g = load("scan_small")
    b, d, L = g["u"].shape
    _write(tmp_path, dict(batch=b, dim=d, seq_len=L, d_state=g["A"].shape[1]),
           {k: g[k] for k in ("u", "delta", "B", "C", "z", "A", "D", "delta_bias")} |
           dict(y=g["y"].astype(np.float32)))
    r = _run("scan", tmp_path)
    assert r.returncode == 0, r.stderr
    assert "scan: ok" in r.stdout
