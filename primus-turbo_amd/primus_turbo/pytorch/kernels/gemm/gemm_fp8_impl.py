"""Dense FP8 GEMM impl (replaces primus_turbo/pytorch/kernels/gemm/gemm_fp8_impl.py).

``gemm_fp8_impl`` keeps the reference custom-op signature (the backend
arguments are accepted and ignored: there is one implementation, the gfx950
kernel).  ``gemm_fp8_nt`` is the lower-level NT entry with explicit scale
addressing used by the autograd functions.
"""

from __future__ import annotations

from typing import Tuple

import torch

from primus_turbo.pytorch import _C
from primus_turbo.pytorch.core.low_precision import ScalingGranularity


def get_gemm_logical_shape(a: torch.Tensor, b: torch.Tensor, trans_a: bool, trans_b: bool) -> Tuple[int, int, int]:
    assert a.ndim == 2 and b.ndim == 2, f"Expected 2D tensors, got a.ndim={a.ndim}, b.ndim={b.ndim}"
    M = a.shape[1] if trans_a else a.shape[0]
    Ka = a.shape[0] if trans_a else a.shape[1]
    Kb = b.shape[1] if trans_b else b.shape[0]
    N = b.shape[0] if trans_b else b.shape[1]
    assert Ka == Kb, f"GEMM K mismatch: a has K={Ka}, b has K={Kb}"
    return M, N, Ka


def _gran_code(granularity) -> int:
    if isinstance(granularity, ScalingGranularity):
        return granularity.value
    return int(granularity)


def _scale_arg(s: torch.Tensor, gran: int) -> torch.Tensor:
    if gran == ScalingGranularity.MX_BLOCKWISE.value:
        return s.contiguous().view(torch.uint8)
    if s.dtype == torch.float32 and s.is_contiguous():
        return s
    return s.contiguous().to(torch.float32)


def _strided_scale_arg(s: torch.Tensor, gran: int) -> Tuple[torch.Tensor, int]:
    """Scale storage for explicitly strided addressing (layout kept) and the
    byte extent the kernel may read."""
    if gran == ScalingGranularity.MX_BLOCKWISE.value:
        s = s.contiguous().view(torch.uint8)
        return s, s.numel()
    if s.dtype != torch.float32:
        s = s.to(torch.float32)
    if s.numel() == 0:
        return s, 0
    last = sum((d - 1) * st for d, st in zip(s.shape, s.stride()))
    return s, (last + 1) * 4


def gemm_fp8_impl(
    a: torch.Tensor,
    a_scale_inv: torch.Tensor,
    trans_a: bool,
    b: torch.Tensor,
    b_scale_inv: torch.Tensor,
    trans_b: bool,
    out_dtype: torch.dtype,
    trans_c: bool,
    granularity: int,
    default_backend: int = 0,
) -> torch.Tensor:
    """C = op(A) @ op(B) (C^T if trans_c) on fp8 operands with the granularity's scales.

    Scale layouts are those of the reference's backends
    (primus_turbo/triton/gemm/gemm_fp8_kernel.py:1013-1154 for BLOCKWISE).
    """
    gran = _gran_code(granularity)
    M, N, K = get_gemm_logical_shape(a, b, trans_a, trans_b)
    a = a.contiguous()
    b = b.contiguous()
    sa = _scale_arg(a_scale_inv, gran)
    sb = _scale_arg(b_scale_inv, gran)
    out = torch.empty((N, M) if trans_c else (M, N), dtype=out_dtype, device=a.device)
    ws = _C.workspace(
        _C.query("pta_gemm_fp8_workspace_size", M, N, K, int(trans_a), int(trans_b), gran), a.device
    )
    _C.call(
        "pta_gemm_fp8", _C.ptr(a), _C.fp8_code(a.dtype), _C.ptr(sa), int(trans_a), _C.ptr(b), _C.fp8_code(b.dtype),
        _C.ptr(sb), int(trans_b), _C.ptr(out), _C.out_dtype_code(out_dtype), int(trans_c), M, N, K, gran,
        _C.ptr(ws), 0 if ws is None else ws.numel(), _C.stream(a.device),
    )
    _C.check_waits("gemm_fp8", ws)
    return out


def gemm_fp8_nt(
    a: torch.Tensor,
    b: torch.Tensor,
    out_dtype: torch.dtype,
    granularity,
    a_scale: torch.Tensor,
    sa_strides: Tuple[int, int] = (0, 0),
    a_scale_2d: bool = False,
    b_scale: torch.Tensor = None,
    sb_strides: Tuple[int, int] = (0, 0),
    b_scale_2d: bool = False,
    out: torch.Tensor = None,
    K: int = None,
    large_tiles_only: bool = False,
) -> torch.Tensor:
    """C[M, N] = A[M, K] . B[N, K]^T with explicit scale addressing.

    Blockwise scales are read as scale[r * stride_r + kb * stride_k] with
    r the row (or row // 128 for a 2-D operand) and kb = k // 128.  K defaults
    to A's width; B may be wider (zero-padded copies).  The kernel is chosen
    as for ``gemm_fp8_impl`` (small-tile kernel for few 256 x 256 tiles, K
    split for up to half a round of them); ``large_tiles_only`` runs the
    256 x 256 kernel whatever the shape (same bits as the small-tile kernel).
    """
    gran = _gran_code(granularity)
    assert a.dim() == 2 and b.dim() == 2
    assert a.stride(1) == 1 and b.stride(1) == 1
    M = a.shape[0]
    N = b.shape[0]
    if K is None:
        K = a.shape[1]
    assert a.shape[1] >= K and b.shape[1] >= K, "operands shorter than K"
    # columns past K (if any) are never read
    # the strides address the scale storage as it is laid out (no reordering copy)
    sa, sa_bytes = _strided_scale_arg(a_scale, gran)
    sb, sb_bytes = _strided_scale_arg(b_scale, gran)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=a.device)
    args = (
        _C.ptr(a), _C.fp8_code(a.dtype), a.stride(0), _C.ptr(b), _C.fp8_code(b.dtype), b.stride(0), _C.ptr(out),
        _C.out_dtype_code(out.dtype), out.stride(0), M, N, K, gran, _C.ptr(sa), sa_strides[0], sa_strides[1],
        int(a_scale_2d), sa_bytes, _C.ptr(sb), sb_strides[0], sb_strides[1], int(b_scale_2d), sb_bytes,
    )
    if large_tiles_only:
        _C.call("pta_gemm_fp8_nt_strided", *args, _C.stream(a.device))
        return out
    ws_n = _C.query("pta_gemm_fp8_nt_strided_ws_size", M, N, K, gran, a.stride(0), b.stride(0), sa_bytes, sb_bytes)
    ws = _C.workspace(ws_n, a.device)
    _C.call("pta_gemm_fp8_nt_strided_ws", *args, _C.ptr(ws), 0 if ws is None else ws.numel(), _C.stream(a.device))
    _C.check_waits("gemm_fp8", ws)
    return out
