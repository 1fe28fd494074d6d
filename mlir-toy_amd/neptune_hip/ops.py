"""torch-tensor front of the C-ABI (device memory and streams only).

Every function hands raw device pointers, sizes and the current HIP stream
to libneptune_hip.so; no computation happens in Python and there is no
fallback path: if the library is missing, ``load_library`` raises.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _abi
from ._abi import check, load_library

LOG2E = 1.4426950408889634

_TORCH_TO_DTYPE = {
    torch.float32: _abi.DTYPE_F32,
    torch.float16: _abi.DTYPE_F16,
    torch.bfloat16: _abi.DTYPE_BF16,
}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_workspace(workspace: torch.Tensor | None) -> None:
    # the library writes numel * element_size bytes from data_ptr
    if workspace is not None and not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous tensor")


def _require_cuda(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("neptune_hip ops take device tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")


def _strides_bhs(t: torch.Tensor) -> tuple[int, int, int]:
    if t.dim() != 4 or t.stride(-1) != 1:
        raise ValueError("expected a [batch, heads, seq, head_dim] tensor with unit head_dim stride")
    return (t.stride(0), t.stride(1), t.stride(2))


def scale_to_log2(scale: float | None, head_dim: int) -> float:
    """Softmax scale (default 1/sqrt(D)) expressed in the exp2 domain."""
    if scale is None:
        return 0.0  # library default: log2(e)/sqrt(head_dim), HTile:24
    return float(scale) * LOG2E


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = False,
    scale: float | None = None,
    return_lse: bool = False,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    scale_log2: float | None = None,
    pipeline_stages: int = 0,
    k_dim_order: int = 0,
):
    """softmax(q k^T * scale) v with the HTile numeric policy.

    q [B, Hq, Sq, D], k/v [B, Hkv, Skv, D] in float32, float16 or bfloat16;
    returns out [B, Hq, Sq, D] (and lse [B, Hq, Sq] fp32 if asked).
    ``scale_log2`` gives the score scale already in the exp2 domain (the
    HTile program's own constant, HTile:24), in place of ``scale``.
    ``pipeline_stages`` (0 = default 2, or 1..3) sets how many K/V tiles the
    kernel stages in LDS ahead of use; with ``k_dim_order=1`` k is given as
    [B, Hkv, D, Skv] (seq contiguous), the order of a dimension_order =
    [1, 0] tile load. Neither changes the result.
    """
    if scale is not None and scale_log2 is not None:
        raise ValueError("give scale or scale_log2, not both")
    _require_cuda(q, k, v, out, lse)
    if q.dtype not in _TORCH_TO_DTYPE or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share one of {list(_TORCH_TO_DTYPE)}")
    B, Hq, Sq, D = q.shape
    if k_dim_order not in (0, 1):
        raise ValueError("k_dim_order must be 0 or 1")
    if k_dim_order:
        Bk, Hk, Dk, Sk = k.shape
    else:
        Bk, Hk, Sk, Dk = k.shape
    if (Bk, Dk) != (B, D) or tuple(v.shape) != (Bk, Hk, Sk, Dk):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype:
        raise ValueError("out must match q's shape and dtype")
    if lse is not None:
        if tuple(lse.shape) != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
            raise ValueError("lse must be a contiguous float32 [B, Hq, Sq] tensor")
        return_lse = True
    elif return_lse:
        lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device)
    desc = _abi.AttnDesc()
    desc.batch, desc.heads_q, desc.heads_kv = B, Hq, Hk
    desc.seq_q, desc.seq_kv, desc.head_dim = Sq, Sk, D
    desc.q_stride[:] = _strides_bhs(q)
    desc.k_stride[:] = _strides_bhs(k)
    desc.v_stride[:] = _strides_bhs(v)
    desc.o_stride[:] = _strides_bhs(out)
    desc.dtype = _TORCH_TO_DTYPE[q.dtype]
    desc.causal = 1 if causal else 0
    desc.scale_log2 = float(scale_log2) if scale_log2 is not None else scale_to_log2(scale, D)
    desc.pipeline_stages = int(pipeline_stages)
    desc.k_dim_order = int(k_dim_order)
    lib = load_library()
    with torch.cuda.device(q.device):
        check(
            lib.neptune_attn_fwd(
                ctypes.byref(desc),
                q.data_ptr(),
                k.data_ptr(),
                v.data_ptr(),
                out.data_ptr(),
                lse.data_ptr() if lse is not None else None,
                _stream(q),
            ),
            lib,
        )
    return (out, lse) if return_lse else out


def _decode_desc(q, k, num_splits, scale_block, scale, kv_dtype) -> _abi.DecodeDesc:
    B, Hq, D = q.shape
    Bk, Hk, L, Dk = k.shape
    desc = _abi.DecodeDesc()
    desc.batch, desc.heads_q, desc.heads_kv = B, Hq, Hk
    desc.seq_kv, desc.head_dim = L, D
    desc.num_splits = num_splits
    desc.scale_block = scale_block
    desc.q_dtype = _abi.DTYPE_BF16
    desc.kv_dtype = kv_dtype
    desc.scale_log2 = scale_to_log2(scale, D)
    return desc


def decode_workspace_bytes(q, k, *, num_splits: int = 0, fp8: bool = False) -> int:
    desc = _decode_desc(_as_q3(q), k, num_splits, 64, None,
                        _abi.DTYPE_FP8_E4M3 if fp8 else _abi.DTYPE_BF16)
    n = ctypes.c_size_t()
    lib = load_library()
    check(lib.neptune_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)), lib)
    return n.value


def _as_q3(q: torch.Tensor) -> torch.Tensor:
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("decode takes one query token per sequence")
        q = q[:, :, 0, :]
    return q


def decode_splitk(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    num_splits: int = 0,
    scale_block: int = 64,
    scale: float | None = None,
    return_lse: bool = False,
    workspace: torch.Tensor | None = None,
):
    """Split-K flash-decoding over grouped KV heads.

    q [B, Hq, D] (or [B, Hq, 1, D]) bf16; k/v [B, Hkv, L, D] bf16, or E4M3
    codes (uint8 / torch.float8_e4m3fn) with k_scale/v_scale
    [B, Hkv, ceil(L/scale_block)] fp32. Returns o [B, Hq, D] bf16.
    """
    q3 = _as_q3(q)
    fp8 = k.dtype in (torch.uint8, torch.float8_e4m3fn)
    if q3.dtype != torch.bfloat16:
        raise ValueError("decode query must be bfloat16")
    if not fp8 and k.dtype != torch.bfloat16:
        raise ValueError("decode KV must be bfloat16 or E4M3 codes")
    if q3.dim() != 3 or k.dim() != 4:
        raise ValueError("decode takes q [B, Hq, D] and k, v [B, Hkv, L, D]")
    if v.dtype != k.dtype or tuple(v.shape) != tuple(k.shape):
        raise ValueError("k and v must match")
    B, _, D = q3.shape
    Bk, Hk, L, Dk = k.shape
    if (Bk, Dk) != (B, D):
        raise ValueError(f"k {tuple(k.shape)} does not match q {tuple(q3.shape)} in batch or "
                         "head_dim")
    for t in (q3, k, v):
        if not t.is_contiguous():
            raise ValueError("decode tensors must be contiguous")
    if fp8:
        if scale_block <= 0:
            raise ValueError("scale_block must be positive")
        want = (B, Hk, -(-L // scale_block))
        for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
            if t is None or t.dtype != torch.float32 or not t.is_contiguous() or \
                    tuple(t.shape) != want:
                raise ValueError(f"fp8 KV needs {name}: contiguous float32 {list(want)} "
                                 f"(scale_block {scale_block})")
    elif k_scale is not None or v_scale is not None:
        raise ValueError("k_scale / v_scale apply to E4M3 KV only")
    _require_cuda(q3, k, v, k_scale, v_scale, workspace)
    _check_workspace(workspace)
    desc = _decode_desc(q3, k, num_splits, scale_block, scale,
                        _abi.DTYPE_FP8_E4M3 if fp8 else _abi.DTYPE_BF16)
    lib = load_library()
    n = ctypes.c_size_t()
    check(lib.neptune_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)), lib)
    if workspace is None:
        workspace = torch.empty(max(n.value, 1), dtype=torch.uint8, device=q3.device)
    out = torch.empty_like(q3)
    lse = torch.empty(q3.shape[:2], dtype=torch.float32, device=q3.device) if return_lse else None
    with torch.cuda.device(q3.device):
        check(
            lib.neptune_decode_splitk(
                ctypes.byref(desc),
                q3.data_ptr(),
                k.data_ptr(),
                v.data_ptr(),
                k_scale.data_ptr() if k_scale is not None else None,
                v_scale.data_ptr() if v_scale is not None else None,
                out.data_ptr(),
                lse.data_ptr() if lse is not None else None,
                workspace.data_ptr(),
                workspace.numel() * workspace.element_size(),
                _stream(q3),
            ),
            lib,
        )
    return (out, lse) if return_lse else out


def decode_paged(
    q: torch.Tensor,
    k_pages: torch.Tensor,
    v_pages: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    max_seq_len: int | None = None,
    num_splits: int = 0,
    scale: float | None = None,
    return_lse: bool = False,
    workspace: torch.Tensor | None = None,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
):
    """Split-K decode over a paged KV cache.

    q [B, Hq, D] bf16; k_pages / v_pages [num_pages, Hkv, page_size, D]
    views (any page/head/position strides with D contiguous, e.g. a permuted
    [num_pages, page_size, Hkv, D] pool) of bf16, or of E4M3 codes (uint8 /
    torch.float8_e4m3fn) with k_scales / v_scales fp32 [num_pages, Hkv]
    (one scale per page and kv head); block_table [B, max_pages] and
    seq_lens [B] int32 on the device. ``max_seq_len`` (default
    max_pages * page_size) is the longest sequence and sets the split
    layout. Returns o [B, Hq, D] bf16.
    """
    q3 = _as_q3(q)
    fp8 = k_pages.dtype in (torch.uint8, torch.float8_e4m3fn)
    if q3.dtype != torch.bfloat16 or k_pages.dtype != v_pages.dtype or \
            not (fp8 or k_pages.dtype == torch.bfloat16):
        raise ValueError("paged decode takes bfloat16 q and bfloat16 or E4M3 KV pages")
    if k_pages.dim() != 4 or tuple(k_pages.shape) != tuple(v_pages.shape) or \
            k_pages.stride(-1) != 1 or v_pages.stride(-1) != 1:
        raise ValueError("k_pages / v_pages: matching [pages, Hkv, page_size, D] views, D contiguous")
    for name, t in (("block_table", block_table), ("seq_lens", seq_lens)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor")
    npages, Hk, psize, D = k_pages.shape
    if q3.dim() != 3 or q3.shape[2] != D:
        raise ValueError(f"q {tuple(q3.shape)} does not match the pools' head_dim {D}")
    if fp8:
        for name, t in (("k_scales", k_scales), ("v_scales", v_scales)):
            if t is None or t.dtype != torch.float32 or not t.is_contiguous() or \
                    tuple(t.shape) != (npages, Hk):
                raise ValueError(f"fp8 pages need {name}: contiguous float32 [num_pages, Hkv]")
    elif k_scales is not None or v_scales is not None:
        raise ValueError("k_scales / v_scales apply to E4M3 pools only")
    B = q3.shape[0]
    if block_table.dim() != 2 or block_table.shape[0] != B or tuple(seq_lens.shape) != (B,):
        raise ValueError("block_table [B, max_pages] and seq_lens [B] must match q's batch")
    _require_cuda(q3, k_pages, v_pages, block_table, seq_lens, workspace, k_scales, v_scales)
    _check_workspace(workspace)
    max_pages = block_table.shape[1]
    L = int(max_seq_len) if max_seq_len is not None else max_pages * psize
    k4 = torch.empty((B, Hk, L, D), dtype=k_pages.dtype, device="meta")
    desc = _decode_desc(q3, k4, num_splits, psize if fp8 else 64, scale,
                        _abi.DTYPE_FP8_E4M3 if fp8 else _abi.DTYPE_BF16)
    pk = _abi.PagedKvDesc()
    pk.num_pages, pk.page_size, pk.max_pages = npages, psize, max_pages
    pk.k_stride[:] = (k_pages.stride(0), k_pages.stride(1), k_pages.stride(2))
    pk.v_stride[:] = (v_pages.stride(0), v_pages.stride(1), v_pages.stride(2))
    lib = load_library()
    n = ctypes.c_size_t()
    check(lib.neptune_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)), lib)
    if workspace is None:
        workspace = torch.empty(max(n.value, 1), dtype=torch.uint8, device=q3.device)
    out = torch.empty_like(q3)
    lse = torch.empty(q3.shape[:2], dtype=torch.float32, device=q3.device) if return_lse else None
    tail = (block_table.data_ptr(), seq_lens.data_ptr(), out.data_ptr(),
            lse.data_ptr() if lse is not None else None, workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), _stream(q3))
    with torch.cuda.device(q3.device):
        if fp8:
            st = lib.neptune_decode_paged_fp8(
                ctypes.byref(desc), ctypes.byref(pk), q3.data_ptr(), k_pages.data_ptr(),
                v_pages.data_ptr(), k_scales.data_ptr(), v_scales.data_ptr(), *tail)
        else:
            st = lib.neptune_decode_paged(
                ctypes.byref(desc), ctypes.byref(pk), q3.data_ptr(), k_pages.data_ptr(),
                v_pages.data_ptr(), *tail)
        check(st, lib)
    return (out, lse) if return_lse else out


def kv_quantize_fp8(kv: torch.Tensor, *, scale_block: int = 64):
    """bf16 [B, Hkv, L, D] -> (E4M3 codes uint8, scales fp32 [B, Hkv, nblocks])."""
    _require_cuda(kv)
    if kv.dtype != torch.bfloat16 or kv.dim() != 4 or not kv.is_contiguous():
        raise ValueError("kv_quantize_fp8 takes a contiguous bf16 [B, Hkv, L, D] tensor")
    B, Hk, L, D = kv.shape
    nsb = -(-L // scale_block)
    codes = torch.empty(kv.shape, dtype=torch.uint8, device=kv.device)
    scales = torch.empty((B, Hk, nsb), dtype=torch.float32, device=kv.device)
    lib = load_library()
    with torch.cuda.device(kv.device):
        check(
            lib.neptune_kv_quantize_fp8(
                B, Hk, L, D, scale_block, kv.data_ptr(), codes.data_ptr(), scales.data_ptr(),
                _stream(kv),
            ),
            lib,
        )
    return codes, scales


def selective_scan(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: torch.Tensor | None = None,
    z: torch.Tensor | None = None,
    delta_bias: torch.Tensor | None = None,
    delta_softplus: bool = True,
) -> torch.Tensor:
    """Mamba-1 selective scan (selective_scan_fn argument order).

    u, delta, z [batch, dim, L] and B, C [batch, d_state, L] bf16; A
    [dim, d_state], D and delta_bias [dim] fp32. Returns y [batch, dim, L] bf16.
    """
    for name, t in (("u", u), ("delta", delta), ("B", B), ("C", C), ("z", z)):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous bfloat16")
    for name, t in (("A", A), ("D", D), ("delta_bias", delta_bias)):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous float32")
    if u.dim() != 3 or A.dim() != 2:
        raise ValueError("selective_scan takes u [batch, dim, L] and A [dim, d_state]")
    bsz, dim, L = u.shape
    N = A.shape[1]
    want = {"delta": (bsz, dim, L), "A": (dim, N), "B": (bsz, N, L), "C": (bsz, N, L),
            "z": (bsz, dim, L), "D": (dim,), "delta_bias": (dim,)}
    for name, t in (("delta", delta), ("A", A), ("B", B), ("C", C), ("z", z), ("D", D),
                    ("delta_bias", delta_bias)):
        if t is not None and tuple(t.shape) != want[name]:
            raise ValueError(f"selective_scan: {name} is {tuple(t.shape)}, expected "
                             f"{want[name]}")
    _require_cuda(u, delta, A, B, C, D, z, delta_bias)
    y = torch.empty_like(u)
    desc = _abi.ScanDesc(bsz, dim, L, N, _abi.DTYPE_BF16, 1 if delta_softplus else 0)
    lib = load_library()
    with torch.cuda.device(u.device):
        check(
            lib.neptune_selective_scan_fwd(
                ctypes.byref(desc),
                u.data_ptr(),
                delta.data_ptr(),
                A.data_ptr(),
                B.data_ptr(),
                C.data_ptr(),
                D.data_ptr() if D is not None else None,
                z.data_ptr() if z is not None else None,
                delta_bias.data_ptr() if delta_bias is not None else None,
                y.data_ptr(),
                _stream(u),
            ),
            lib,
        )
    return y


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
