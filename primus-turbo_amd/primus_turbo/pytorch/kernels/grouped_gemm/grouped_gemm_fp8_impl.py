"""Grouped FP8 GEMM impls (replace the reference's
primus_turbo/pytorch/kernels/grouped_gemm/grouped_gemm_fp8_impl.py:817-901).

Group offsets stay on the device: no host synchronisation, so the calls can be
captured in a HIP graph.
"""

from __future__ import annotations

import torch

from primus_turbo.pytorch import _C
from primus_turbo.pytorch.core.low_precision import ScalingGranularity


def _gran_code(g) -> int:
    return g.value if isinstance(g, ScalingGranularity) else int(g)


def _scale(s: torch.Tensor, gran: int) -> torch.Tensor:
    if gran == ScalingGranularity.MX_BLOCKWISE.value:
        return s.contiguous().view(torch.uint8)
    return s.contiguous().to(torch.float32)


def grouped_gemm_fp8_impl(
    a: torch.Tensor,
    b: torch.Tensor,
    a_scales: torch.Tensor,
    b_scales: torch.Tensor,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    trans_a: bool,
    trans_b: bool,
    out_dtype: torch.dtype,
    granularity: int,
    num_cu: int | None = None,
    default_backend: int = 0,
    maybe_pre_sync: bool = False,
    group_offs_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """out[offs[g]:offs[g+1]] = a[offs[g]:offs[g+1]] @ op(b[g]); rows past offs[G] are zero.

    With ``group_offs_out`` the rows of ``a`` follow the padded layout
    ``group_offs`` and group g's output rows are packed at
    ``out[group_offs_out[g]:group_offs_out[g+1]]`` (the MX grouped forward;
    ``out`` keeps a's row count and the caller slices the packed rows).

    a [M_total, K]; b [G, N, K] (trans_b) or [G, K, N].  Blockwise: a_scales
    transposed [K/128, M_total], b_scales [G, N/128, K/128] (trans_b) or
    [G, K/128, N/128].  Rowwise: a_scales [M_total(, 1)], b_scales [G, N(, 1)].
    Tensorwise: scalars.
    """
    assert not trans_a, "trans_a is not supported"
    gran = _gran_code(granularity)
    a = a.contiguous()
    b = b.contiguous()
    G = b.shape[0]
    M_total, K = a.shape
    N = b.shape[1] if trans_b else b.shape[2]
    assert (b.shape[2] if trans_b else b.shape[1]) == K, "K mismatch"
    out = torch.empty((M_total, N), dtype=out_dtype, device=a.device)
    ws = _C.workspace(
        _C.query("pta_grouped_gemm_fp8_workspace_size", M_total, N, K, G, int(trans_b), gran), a.device
    )
    offs = group_offs.to(torch.int64).contiguous()
    offs_out = None if group_offs_out is None else group_offs_out.to(torch.int64).contiguous()
    _C.call(
        "pta_grouped_gemm_fp8", _C.ptr(a), _C.fp8_code(a.dtype), _C.ptr(_scale(a_scales, gran)), _C.ptr(b),
        _C.fp8_code(b.dtype), _C.ptr(_scale(b_scales, gran)), int(trans_b), _C.ptr(offs), _C.ptr(offs_out), G,
        M_total, N, K,
        _C.ptr(out), _C.out_dtype_code(out_dtype), gran, int(num_cu or 0), _C.ptr(ws),
        0 if ws is None else ws.numel(), _C.stream(a.device),
    )
    return out


def grouped_gemm_fp8_variable_k_impl(
    a: torch.Tensor,
    b: torch.Tensor,
    a_scales: torch.Tensor,
    b_scales: torch.Tensor,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    trans_a: bool,
    trans_b: bool,
    trans_c: bool,
    out_dtype: torch.dtype,
    granularity: int,
    num_cu: int | None = None,
    default_backend: int = 0,
    maybe_pre_sync: bool = False,
) -> torch.Tensor:
    """out[g] = a[seg_g]^T @ b[seg_g] (transposed with trans_c); empty groups give zeros.

    a [M_total, OUT_M], b [M_total, OUT_N].  Blockwise requires 128-aligned
    segments with scales [M_total/128, OUT_*]; rowwise takes per-column scales
    [OUT_*]; tensorwise takes scalars.

    MX_BLOCKWISE follows the reference's MX wgrad call
    (ops/grouped_gemm_fp8.py:760-775): a and b are the colwise quantized
    tensors, already transposed and padded per group, a [OUT_M, K_pad],
    b [OUT_N, K_pad] with E8M0 scales [OUT_*, K_pad/32] and 128-aligned
    group_offs; out[g] = a[:, seg_g] @ b[:, seg_g]^T.
    """
    gran = _gran_code(granularity)
    if gran == ScalingGranularity.MX_BLOCKWISE.value:
        return grouped_gemm_fp8_variable_k_nt_impl(a, b, a_scales, b_scales, group_lens.shape[0], group_offs,
                                                   trans_c, out_dtype, gran)
    assert trans_a and not trans_b, "variable-K grouped GEMM expects trans_a=True, trans_b=False"
    if gran == ScalingGranularity.BLOCKWISE.value:
        # a 128-row scale block of a [M_total/128, OUT] column scale must not
        # straddle two groups: the kernel indexes scale rows by padded segment
        # offset / 128, which is only the quantizer's row when the offsets are
        # 128-aligned (the segment quant's vk_offs are).  One host read, left
        # out under stream capture (no host read may happen there).
        if not torch.cuda.is_current_stream_capturing() and bool(
                torch.any(group_offs.to(torch.int64) % 128 != 0).item()):
            raise RuntimeError("variable-K BLOCKWISE grouped GEMM needs 128-aligned group offsets "
                               "(the segment quant's padded offsets)")
    a = a.contiguous()
    b = b.contiguous()
    M_total, OUT_M = a.shape
    OUT_N = b.shape[1]
    G = group_lens.shape[0]
    out = torch.empty((G, OUT_N, OUT_M) if trans_c else (G, OUT_M, OUT_N), dtype=out_dtype, device=a.device)
    ws = _C.workspace(
        _C.query("pta_grouped_gemm_fp8_variable_k_workspace_size", M_total, OUT_M, OUT_N, G, gran), a.device
    )
    offs = group_offs.to(torch.int64).contiguous()
    _C.call(
        "pta_grouped_gemm_fp8_variable_k", _C.ptr(a), _C.fp8_code(a.dtype), _C.ptr(_scale(a_scales, gran)),
        _C.ptr(b), _C.fp8_code(b.dtype), _C.ptr(_scale(b_scales, gran)), _C.ptr(offs), G, M_total, OUT_M, OUT_N,
        _C.ptr(out), _C.out_dtype_code(out_dtype), int(trans_c), gran, int(num_cu or 0), _C.ptr(ws),
        0 if ws is None else ws.numel(), _C.stream(a.device),
    )
    return out


def grouped_gemm_fp8_variable_k_nt_impl(
    a_t: torch.Tensor,
    b_t: torch.Tensor,
    a_scales: torch.Tensor,
    b_scales: torch.Tensor,
    G: int,
    padded_offs: torch.Tensor,
    trans_c: bool,
    out_dtype: torch.dtype,
    granularity: int,
) -> torch.Tensor:
    """out[g] = a_t[:, seg_g] @ b_t[:, seg_g]^T (transposed with trans_c) on
    column copies already transposed and padded per group: a_t [OUT_M, K_pad],
    b_t [OUT_N, K_pad], seg_g = columns [padded_offs[g], padded_offs[g+1])
    (multiples of 128).  MX: E8M0 scales [OUT_*, K_pad/32]; BLOCKWISE: the
    segment quant's column scales [K_pad/128, OUT_*].  Empty groups give zeros."""
    gran = _gran_code(granularity)
    a_t = a_t.contiguous()
    b_t = b_t.contiguous()
    OUT_M, K_pad = a_t.shape
    OUT_N = b_t.shape[0]
    assert b_t.shape[1] == K_pad, "padded K mismatch"
    out = torch.empty((G, OUT_N, OUT_M) if trans_c else (G, OUT_M, OUT_N), dtype=out_dtype, device=a_t.device)
    offs = padded_offs.to(torch.int64).contiguous()
    _C.call(
        "pta_grouped_gemm_fp8_variable_k_nt", _C.ptr(a_t), _C.fp8_code(a_t.dtype), _C.ptr(_scale(a_scales, gran)),
        _C.ptr(b_t), _C.fp8_code(b_t.dtype), _C.ptr(_scale(b_scales, gran)), _C.ptr(offs), G, K_pad, OUT_M, OUT_N,
        _C.ptr(out), _C.out_dtype_code(out_dtype), int(trans_c), gran, _C.stream(a_t.device),
    )
    return out
