"""CPU tests of the reference-side binding (mlir-toy_amd/reference_binding/hip.py),
the module a maintainer of the reference adds as src/neptune_mlir/backends/hip.py.

* The torch dtype reaches the descriptor by equality: float16 -> F16,
  bfloat16 -> BF16, float32 -> F32 (str(torch.bfloat16) also ends in
  "float16", so a suffix test would bind bf16 as F16); other dtypes raise
  NotImplementedError before any call.
* Arguments that break what the generated kernel assumes (one device, one
  dtype, agreeing shapes, contiguous storage) are refused before any call.
* Through the real library's validation path (no device here), a shape the
  fp32 kernel covers and the 16-bit kernels do not (head_dim 32) is accepted
  for F32 (and then finds no device: RuntimeError) and refused as
  unsupported for F16 and BF16 (NotImplementedError), as the reference's
  translators raise (translators/common.py:187-197,217-224).
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from neptune_hip import _abi
from reference_binding import hip


class _Recorder:
    """Stands in for the library: records each descriptor it is given."""

    def __init__(self, status=0):
        self.seen = []
        self.status = status

    def neptune_attn_fwd(self, desc_ref, q, k, v, o, lse, stream):
        d = ctypes.cast(desc_ref, ctypes.POINTER(hip.AttnDesc)).contents
        self.seen.append((d.dtype, d.batch, d.heads_q, d.heads_kv, d.seq_q, d.seq_kv,
                          d.head_dim, lse, stream))
        return self.status

    def neptune_last_error(self):
        return b"recorded failure"


@pytest.fixture
def recorder(monkeypatch):
    rec = _Recorder()
    monkeypatch.setattr(hip, "_lib", rec)
    return rec


def _qkvo(dtype, shape=(1, 2, 16, 64), kv_seq=24):
    q = torch.zeros(shape, dtype=dtype)
    kv = (shape[0], shape[1], kv_seq, shape[3])
    return q, torch.zeros(kv, dtype=dtype), torch.zeros(kv, dtype=dtype), torch.empty_like(q)


@pytest.mark.parametrize("dtype,code", [(torch.float16, hip.F16), (torch.bfloat16, hip.BF16),
                                        (torch.float32, hip.F32)])
def test_dtype_maps_by_equality(recorder, dtype, code):
    hip.flash_attention_htile(*_qkvo(dtype))
    (got, b, hq, hkv, sq, skv, d, lse, stream), = recorder.seen
    assert got == code
    assert (b, hq, hkv, sq, skv, d) == (1, 2, 2, 16, 24, 64)
    assert lse is None and stream is None  # CPU tensors: the null stream


def test_header_enum_values():
    """The stub's constants are the header's neptune_dtype / neptune_status."""
    text = (Path(__file__).resolve().parents[1] / "include" / "neptune_hip.h").read_text()
    enum = {k: int(v) for k, v in re.findall(r"\b(NEPTUNE_\w+) = (\d+)", text)}
    assert (hip.F32, hip.F16, hip.BF16) == (enum["NEPTUNE_DTYPE_F32"], enum["NEPTUNE_DTYPE_F16"],
                                            enum["NEPTUNE_DTYPE_BF16"])
    assert (hip.OK, hip.ERR_INVALID_ARGUMENT, hip.ERR_UNSUPPORTED) == (
        enum["NEPTUNE_OK"], enum["NEPTUNE_ERR_INVALID_ARGUMENT"], enum["NEPTUNE_ERR_UNSUPPORTED"])
    assert ctypes.sizeof(hip.AttnDesc) == ctypes.sizeof(_abi.AttnDesc)


@pytest.mark.parametrize("dtype", [torch.float64, torch.int8])
def test_unsupported_dtype_raises_before_the_call(recorder, dtype):
    with pytest.raises(NotImplementedError):
        hip.flash_attention_htile(*_qkvo(dtype))
    assert recorder.seen == []


def test_mismatched_arguments_raise_before_the_call(recorder):
    q, k, v, o = _qkvo(torch.float16)
    bad = [
        ((q, k, v, torch.empty((1, 2, 8, 64), dtype=torch.float16)), RuntimeError),  # out shape
        ((q, k, v[:, :, :16], o), RuntimeError),                                  # v != k
        ((q, k.float(), v, o), RuntimeError),                                     # dtypes
        ((q.transpose(2, 3).contiguous().transpose(2, 3), k, v, o),               # strided q
         NotImplementedError),
    ]
    for args, exc in bad:
        with pytest.raises(exc):
            hip.flash_attention_htile(*args)
    assert recorder.seen == []


def test_status_maps_to_reference_exceptions(monkeypatch):
    for status, exc in ((hip.ERR_UNSUPPORTED, NotImplementedError),
                        (hip.ERR_INVALID_ARGUMENT, RuntimeError), (3, RuntimeError)):
        monkeypatch.setattr(hip, "_lib", _Recorder(status))
        with pytest.raises(exc, match="recorded failure"):
            hip.flash_attention_htile(*_qkvo(torch.float16))


@pytest.fixture
def real_lib(monkeypatch):
    if torch.cuda.is_available():
        pytest.skip("the no-device path needs a host without a HIP device")
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setenv(hip.NEPTUNE_HIP_ENV, str(_abi.find_library_path()))
    return hip.load()


def test_real_library_validates_each_dtype(real_lib):
    shape = (1, 2, 16, 32)  # head_dim 32: the fp32 kernel only
    with pytest.raises(RuntimeError, match="no HIP device"):
        hip.flash_attention_htile(*_qkvo(torch.float32, shape))
    for dtype in (torch.float16, torch.bfloat16):
        with pytest.raises(NotImplementedError, match="head_dim"):
            hip.flash_attention_htile(*_qkvo(dtype, shape))
    # a covered 16-bit shape passes validation and finds no device
    for dtype in (torch.float16, torch.bfloat16):
        with pytest.raises(RuntimeError, match="no HIP device"):
            hip.flash_attention_htile(*_qkvo(dtype, (1, 2, 16, 128)))


def test_load_without_a_path_says_what_to_set(monkeypatch):
    monkeypatch.delenv(hip.NEPTUNE_HIP_ENV, raising=False)
    with pytest.raises(RuntimeError, match=hip.NEPTUNE_HIP_ENV):
        hip.load()
