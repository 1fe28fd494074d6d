"""HTile front end (no GPU): parsing, recognition of the attention tile
program, parameter extraction, rejection of other programs, and the launch
checks that run before any device call.

The reference's own program (tests/data/flash_attention_htile.mlir in
Evan-Zhao/mlir-toy) is parsed when the reference checkout is present; the
other programs come from tests/htile_gen.py.
"""

import math
from pathlib import Path

import pytest

from htile_gen import program
from neptune_hip import htile

REF_PROGRAM = Path("/root/reference/tests/data/flash_attention_htile.mlir")


def _prog(text):
    mod = htile.translate_source(text)
    assert len(mod.__all__) == 1
    return getattr(mod, mod.__all__[0]).program


@pytest.mark.skipif(not REF_PROGRAM.is_file(), reason="reference checkout not present")
def test_reference_program_is_recognised():
    p = htile.translate_file(str(REF_PROGRAM)).flash_attention_htile.program
    assert p.shape == (1, 32, 4096, 128) and p.dtype == "f16"
    assert (p.block_m, p.block_n, p.trip_count) == (128, 64, 64)
    assert p.grid == (32, 32, 1) and p.threads == (128, 1, 1)
    assert p.pipeline_stages == 2 and p.k_dimension_order == (0, 1)
    assert p.scale_log2 == pytest.approx(math.log2(math.e) / math.sqrt(128), rel=1e-15)


@pytest.mark.parametrize("form", ["pre", "post"])
@pytest.mark.parametrize("canonical", [False, True])
def test_generated_forms(form, canonical):
    p = _prog(program(B=2, H=4, S=1024, D=128, dtype="bf16", form=form, canonical=canonical))
    assert p.shape == (2, 4, 1024, 128) and p.dtype == "bf16"
    assert p.grid == (8, 4, 2) and p.trip_count == 16
    assert p.k_dimension_order == ((1, 0) if form == "post" else (0, 1))


def test_canonical_folds_batch_block_id():
    # grid_z == 1: the batch index of every access is the constant 0
    p = _prog(program(B=1, H=2, S=256, D=64, dtype="f16", canonical=True))
    assert p.grid == (2, 2, 1) and p.block_n == 64 and p.shape[3] == 64


def test_parameters_follow_the_program():
    p = _prog(program(B=1, H=3, S=512, D=64, dtype="f32", bm=64, bn=32, scale=0.25, stages=3,
                      grid=(4, 3, 1), trip=8))
    assert (p.block_m, p.block_n, p.trip_count) == (64, 32, 8)
    assert p.scale_log2 == 0.25 and p.pipeline_stages == 3 and p.grid == (4, 3, 1)


@pytest.mark.parametrize("canonical", [False, True])
@pytest.mark.parametrize("S", [1024, 128])  # S == D: the index pattern tells the storage order
def test_k_stored_transposed_binds_k_dim_order(canonical, S):
    p = _prog(program(B=1, H=2, S=S, D=128, dtype="bf16", k_mem="ds", stages=3,
                      canonical=canonical))
    assert p.k_dim_order == 1 and p.k_dimension_order == (0, 1)
    assert (p.block_n, p.trip_count, p.pipeline_stages) == (64, S // 64, 3)
    for form in ("pre", "post"):
        q = _prog(program(B=1, H=2, S=S, D=128, dtype="bf16", form=form, canonical=canonical))
        assert q.k_dim_order == 0


def test_k_stored_transposed_and_transposed_again_is_rejected():
    # [D, S] storage, plain [D, block_n] tile, then transpose_b: that is Q.K, not Q.K^T
    with pytest.raises(NotImplementedError, match="not a flash-attention tile program"):
        htile.translate_source(program(S=256, H=2, k_mem="ds", mutate="kt_transpose"))


def test_stage_counts_the_kernel_does_not_stage_are_rejected():
    with pytest.raises(NotImplementedError, match="pipeline_stages = 4"):
        htile.translate_source(program(S=256, H=2, stages=4))


def test_without_pipeline_hint():
    assert _prog(program(S=256, H=2, stages=None)).pipeline_stages is None


@pytest.mark.parametrize("mutate", ["delta_sign", "no_rescale", "q_row0"])
def test_other_recurrences_are_rejected(mutate):
    with pytest.raises(NotImplementedError, match="not a flash-attention tile program"):
        htile.translate_source(program(S=256, H=2, mutate=mutate))


@pytest.mark.parametrize("mutate", ["unsupported", "exp"])
def test_unsupported_ops_are_named(mutate):
    with pytest.raises(NotImplementedError, match="unsupported op"):
        htile.translate_source(program(S=256, H=2, mutate=mutate))


def test_malformed_input_is_a_value_error():
    with pytest.raises(ValueError):
        htile.translate_source("module { func.func @f(%q: memref<1x1x64x64xf16> {")


def test_launch_checks_run_before_the_device():
    torch = pytest.importorskip("torch")
    kern = htile.translate_source(program(B=1, H=2, S=256, D=64, dtype="f16")).flash_attention_htile
    t = torch.zeros((1, 2, 256, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="expected"):
        kern[(2, 2, 1)](t.float(), t, t, t)
    with pytest.raises(ValueError, match="outside the memrefs"):
        kern[(4, 2, 1)](t, t, t, t)
    with pytest.raises(ValueError, match="device tensors"):
        kern[(2, 2, 1)](t, t, t, t)


def test_launch_checks_the_transposed_k_shape():
    torch = pytest.importorskip("torch")
    kern = htile.translate_source(program(B=1, H=2, S=256, D=128, dtype="bf16",
                                          k_mem="ds")).flash_attention_htile
    t = torch.zeros((1, 2, 256, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"k: expected \[1, 2, 128, 256\]"):
        kern(t, t, t, t)


def test_cli_prints_the_binding(tmp_path, capsys):
    f = tmp_path / "p.mlir"
    f.write_text(program(B=1, H=2, S=256, D=64))
    assert htile.main([str(f)]) == 0
    assert '"trip_count": 4' in capsys.readouterr().out
