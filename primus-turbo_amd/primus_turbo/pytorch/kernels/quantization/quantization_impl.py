"""Quantization impls: allocate outputs with torch, launch the gfx950 kernels.

Function names, argument meaning and output layouts follow the reference's
primus_turbo/pytorch/kernels/quantization/quantization_impl.py and the native
ops of csrc/pytorch/quantization/quantization.cpp.  Every call goes through
``libprimus_turbo_amd.so``; there is no fallback path.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from primus_turbo.pytorch import _C
from primus_turbo.pytorch.core.low_precision import (
    MXFP8_BLOCK_SIZE,
    MXFP8_PADDING_ALIGN_SIZE,
    ScalingRecipe,
)


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def _check_hp(x: torch.Tensor):
    assert x.is_cuda, "input must be a GPU tensor"
    assert x.dtype in (torch.bfloat16, torch.float16, torch.float32), f"unsupported input dtype {x.dtype}"


# ---------------------------------------------------------------------------
# tensorwise / rowwise  (quantization.cpp:42-206)
# ---------------------------------------------------------------------------
def quantize_fp8_tensorwise_impl(
    x: torch.Tensor, out_dtype: torch.dtype, scale: Optional[torch.Tensor] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_hp(x)
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    scale_inv = torch.empty((), dtype=torch.float32, device=x.device)
    ws = None
    if scale is None:
        ws = _C.workspace(_C.query("pta_quantize_fp8_tensorwise_workspace_size", x.numel()), x.device)
    else:
        assert scale.numel() == 1, "tensorwise scale must be scalar tensor"
        scale = scale.to(torch.float32).contiguous()
    _C.call(
        "pta_quantize_fp8_tensorwise", _C.ptr(x), _C.in_dtype_code(x.dtype), x.numel(), _C.ptr(scale),
        _C.ptr(q), _C.fp8_code(out_dtype), _C.ptr(scale_inv), _C.ptr(ws), 0 if ws is None else ws.numel(),
        _C.stream(x.device),
    )
    _C.check_waits("quantize_fp8 (tensorwise)", ws)
    return q, scale_inv


def quantize_fp8_rowwise_impl(
    x: torch.Tensor, out_dtype: torch.dtype, axis: int, scale: Optional[torch.Tensor] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_hp(x)
    assert x.is_contiguous(), "The x tensor must be contiguous."
    assert axis is not None, "axis must be specified for rowwise quantization"
    nd = x.dim()
    ax = axis if axis >= 0 else axis + nd
    assert 0 <= ax < nd, f"axis {axis} out of range for a {nd}-D tensor"
    shape = list(x.shape)
    outer = 1
    for s in shape[:ax]:
        outer *= s
    length = shape[ax]
    inner = 1
    for s in shape[ax + 1 :]:
        inner *= s
    sshape = list(shape)
    sshape[ax] = 1
    q = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    scale_inv = torch.empty(sshape, dtype=torch.float32, device=x.device)
    if scale is not None:
        assert list(scale.shape) == sshape, "rowwise scale shape mismatch"
        scale = scale.to(torch.float32).contiguous()
    ws = _C.workspace(_C.query("pta_quantize_fp8_rowwise_workspace_size", outer, length, inner), x.device)
    _C.call(
        "pta_quantize_fp8_rowwise", _C.ptr(x), _C.in_dtype_code(x.dtype), outer, length, inner, _C.ptr(scale),
        _C.ptr(q), _C.fp8_code(out_dtype), _C.ptr(scale_inv), _C.ptr(ws), 0 if ws is None else ws.numel(),
        _C.stream(x.device),
    )
    return q, scale_inv


def dequantize_fp8_tensorwise_impl(x: torch.Tensor, out_dtype: torch.dtype, scale_inv: torch.Tensor):
    x = x.contiguous()
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    s = scale_inv.to(torch.float32).contiguous()
    _C.call(
        "pta_dequantize_fp8_tensorwise", _C.ptr(x), _C.fp8_code(x.dtype), x.numel(), _C.ptr(s), _C.ptr(y),
        _C.out_dtype_code(out_dtype), _C.stream(x.device),
    )
    return y


def dequantize_fp8_rowwise_impl(x: torch.Tensor, out_dtype: torch.dtype, axis: int, scale_inv: torch.Tensor):
    assert x.is_contiguous(), "The x tensor must be contiguous."
    assert scale_inv.is_contiguous(), "The scale_inv tensor must be contiguous."
    nd = x.dim()
    ax = axis if axis >= 0 else axis + nd
    shape = list(x.shape)
    outer = 1
    for s in shape[:ax]:
        outer *= s
    inner = 1
    for s in shape[ax + 1 :]:
        inner *= s
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    _C.call(
        "pta_dequantize_fp8_rowwise", _C.ptr(x), _C.fp8_code(x.dtype), outer, shape[ax], inner,
        _C.ptr(scale_inv), _C.ptr(y), _C.out_dtype_code(out_dtype), _C.stream(x.device),
    )
    return y


# ---------------------------------------------------------------------------
# blockwise  (quantization_impl.py:74-486)
# ---------------------------------------------------------------------------
def quant_fp8_blockwise_impl(
    x: torch.Tensor, dtype: torch.dtype, axis: int, block_size: int = 128
) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_hp(x)
    assert x.is_contiguous() and x.dim() == 2, "Input must be 2D and contiguous"
    assert axis in (-2, -1, 0, 1), f"axis must be 0 or 1 (or -1, -2), got {axis}"
    axis = axis % 2
    M, N = x.shape
    q = torch.empty((M, N), dtype=dtype, device=x.device)
    sshape = (M, ceil_div(N, block_size)) if axis == 1 else (ceil_div(M, block_size), N)
    s = torch.empty(sshape, dtype=torch.float32, device=x.device)
    _C.call(
        "pta_quantize_fp8_blockwise", _C.ptr(x), _C.in_dtype_code(x.dtype), M, N, block_size, axis, _C.ptr(q),
        _C.ptr(s), _C.fp8_code(dtype), _C.stream(x.device),
    )
    return q, s


def quant_fp8_blockwise_dual_impl(
    x: torch.Tensor,
    dtype: torch.dtype,
    block_size: int = 128,
    col_transposed: bool = False,
    row_scale_kmajor: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Row (1 x bs) and column (bs x 1) quantization in one read of ``x``.

    Two extensions used by the autograd functions (the defaults give the
    reference's layouts):
    - ``col_transposed=True`` writes the column-quantized bytes as
      ``[N, roundup(M, 128)]`` (zero padded) so the wgrad GEMM reads them
      K-contiguously (the reference's is ``[M, N]``);
    - ``row_scale_kmajor=True`` returns the row scales as a ``[M, N/bs]`` view
      of ``[N/bs, M]`` storage (strides ``(1, M)``): the GEMM then reads the
      scales of one K block for 16 consecutive rows from one cache line.
    """
    _check_hp(x)
    assert x.is_contiguous() and x.dim() == 2, "Input must be 2D and contiguous"
    M, N = x.shape
    nb = ceil_div(N, block_size)
    q_row = torch.empty((M, N), dtype=dtype, device=x.device)
    if row_scale_kmajor:
        s_row = torch.empty((nb, M), dtype=torch.float32, device=x.device).t()
    else:
        s_row = torch.empty((M, nb), dtype=torch.float32, device=x.device)
    q_col = torch.empty((N, ceil_div(M, 128) * 128) if col_transposed else (M, N), dtype=dtype, device=x.device)
    s_col = torch.empty((ceil_div(M, block_size), N), dtype=torch.float32, device=x.device)
    layout = (_C.DUAL_COL_TRANSPOSED if col_transposed else 0) | (_C.DUAL_ROW_SCALE_KMAJOR if row_scale_kmajor else 0)
    _C.call(
        "pta_quantize_fp8_blockwise_dual", _C.ptr(x), _C.in_dtype_code(x.dtype), M, N, block_size, _C.ptr(q_row),
        _C.ptr(s_row), _C.ptr(q_col), _C.ptr(s_col), layout, _C.fp8_code(dtype), _C.stream(x.device),
    )
    return q_row, s_row, q_col, s_col


def quant_fp8_blockwise_for_weight_impl(
    w: torch.Tensor, dtype: torch.dtype, block_size: int = 128, with_transpose: bool = False
):
    """128 x 128 weight blocks; returns (q, s) or (q, s, q_t) with ``with_transpose``
    (q_t: the same bytes as [B, N, roundup(M, 128)], zero padded)."""
    _check_hp(w)
    assert w.dim() in (2, 3)
    w = w.contiguous()
    squeeze = w.dim() == 2
    B, M, N = (1, *w.shape) if squeeze else tuple(w.shape)
    q = torch.empty((B, M, N), dtype=dtype, device=w.device)
    s = torch.empty((B, ceil_div(M, block_size), ceil_div(N, block_size)), dtype=torch.float32, device=w.device)
    q_t = torch.empty((B, N, ceil_div(M, 128) * 128), dtype=dtype, device=w.device) if with_transpose else None
    _C.call(
        "pta_quantize_fp8_blockwise_for_weight", _C.ptr(w), _C.in_dtype_code(w.dtype), B, M, N, block_size,
        _C.ptr(q), _C.ptr(s), _C.ptr(q_t), _C.fp8_code(dtype), _C.stream(w.device),
    )
    if squeeze:
        q, s = q[0], s[0]
        q_t = q_t[0] if q_t is not None else None
    if with_transpose:
        return q, s, q_t
    return q, s


def dequant_fp8_blockwise_impl(
    x_fp8: torch.Tensor, scale_inv: torch.Tensor, out_dtype: torch.dtype, axis: int, block_size: int = 128
) -> torch.Tensor:
    assert x_fp8.dim() == 2, "Input must be 2D"
    x_fp8 = x_fp8.contiguous()
    M, N = x_fp8.shape
    out = torch.empty((M, N), dtype=out_dtype, device=x_fp8.device)
    _C.call(
        "pta_dequantize_fp8_blockwise", _C.ptr(x_fp8), _C.fp8_code(x_fp8.dtype), 1, M, N, block_size, axis % 2,
        _C.ptr(scale_inv.contiguous()), _C.ptr(out), _C.out_dtype_code(out_dtype), _C.stream(x_fp8.device),
    )
    return out


def dequant_fp8_blockwise_for_weight_impl(
    w_fp8: torch.Tensor, scale_inv: torch.Tensor, out_dtype: torch.dtype, block_size: int = 128
) -> torch.Tensor:
    assert w_fp8.dim() in (2, 3)
    w_fp8 = w_fp8.contiguous()
    B, M, N = (1, *w_fp8.shape) if w_fp8.dim() == 2 else tuple(w_fp8.shape)
    out = torch.empty(w_fp8.shape, dtype=out_dtype, device=w_fp8.device)
    _C.call(
        "pta_dequantize_fp8_blockwise", _C.ptr(w_fp8), _C.fp8_code(w_fp8.dtype), B, M, N, block_size, 2,
        _C.ptr(scale_inv.contiguous()), _C.ptr(out), _C.out_dtype_code(out_dtype), _C.stream(w_fp8.device),
    )
    return out


def quant_fp8_blockwise_segment_m_row_col_impl(
    x: torch.Tensor,
    dtype: torch.dtype,
    block_size: int,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    gemm_other_dim: Optional[int] = None,
    col_transposed: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused row + segment-padded column quantization of a grouped tensor.

    Returns (x_fp8_row [M,N], x_fp8_col_padded [M+G*bs, N], x_scales_row [N/bs, M],
    x_scales_col_padded [(M+G*bs)/bs, N], var_k_group_lens [G], var_k_group_offs [G+1]).
    ``gemm_other_dim`` is accepted for signature compatibility; one kernel serves all sizes.
    ``col_transposed=True`` (used by the grouped autograd function) returns the
    column copy transposed, [N, roundup(M, 128) + G*bs]: the K-contiguous
    operand of the variable-K wgrad GEMM, with no separate transpose pass.
    """
    _check_hp(x)
    assert x.is_contiguous() and x.dim() == 2
    M, N = x.shape
    G = group_lens.size(0)
    Mpad = M + G * block_size
    dev = x.device
    q_row = torch.empty((M, N), dtype=dtype, device=dev)
    if col_transposed:
        q_col = torch.empty((N, ceil_div(M, 128) * 128 + G * block_size), dtype=dtype, device=dev)
    else:
        q_col = torch.empty((Mpad, N), dtype=dtype, device=dev)
    s_row = torch.empty((ceil_div(N, block_size), M), dtype=torch.float32, device=dev)
    s_col = torch.empty((ceil_div(Mpad, block_size), N), dtype=torch.float32, device=dev)
    vk_lens = torch.empty(G, dtype=torch.int64, device=dev)
    vk_offs = torch.empty(G + 1, dtype=torch.int64, device=dev)
    _C.call(
        "pta_quantize_fp8_blockwise_segment_m_row_col", _C.ptr(x), _C.in_dtype_code(x.dtype), M, N, G,
        _C.ptr(group_lens.contiguous()), _C.ptr(group_offs.contiguous()), block_size, _C.ptr(q_row), _C.ptr(q_col),
        _C.ptr(s_row), _C.ptr(s_col), _C.ptr(vk_lens), _C.ptr(vk_offs), _C.fp8_code(dtype),
        _C.SEGMENT_COL_TRANSPOSED if col_transposed else 0, _C.stream(dev),
    )
    return q_row, q_col, s_row, s_col, vk_lens, vk_offs


# ---------------------------------------------------------------------------
# MXFP8  (quantization.cpp:736-967, dequantization_mxfp8.cu)
# ---------------------------------------------------------------------------
def _check_recipe(r: Optional[ScalingRecipe]):
    if r is None:
        return ScalingRecipe()
    if r.use_sr or r.use_rht:
        raise NotImplementedError("stochastic rounding and the Hadamard transform are MXFP4 features")
    if r.shuffle_out:
        # the reference leaves the MXFP8 output shuffle undefined (a TODO in
        # tests/pytorch/ops/test_quantization.py:507); only the scale shuffle exists
        raise NotImplementedError("shuffle_out is not defined for MXFP8")
    return r


def shuffle_scale_impl(scale: torch.Tensor, layout=(16, 16)) -> torch.Tensor:
    """E8M0 scales [M, N] -> the 16 x 16 MFMA layout [roundup(M, 256),
    roundup(N, 8)], zero padded (shuffle_scale in csrc/pytorch/shuffle/shuffle.cpp,
    kernel csrc/kernels/shuffle/shuffle.cu:12-73)."""
    assert tuple(layout) == (16, 16), "Unsupported shuffle layout."
    assert scale.dim() == 2, "Scale must be 2D"
    assert scale.dtype in (torch.float8_e8m0fnu, torch.uint8), "Scale must be Float8_e8m0fnu."
    x = scale.contiguous().view(torch.uint8)
    M, N = x.shape
    y = torch.empty((ceil_div(M, 256) * 256, ceil_div(N, 8) * 8), dtype=torch.uint8, device=x.device)
    _C.call("pta_shuffle_e8m0_scale", _C.ptr(x), M, N, _C.ptr(y), _C.stream(x.device))
    return y.view(torch.float8_e8m0fnu)


def _shuffle_batched(e: torch.Tensor, G: int, rows: int) -> torch.Tensor:
    """Scale shuffle of each of the G row blocks of e[G*rows, cols] (3-D
    inputs keep one padded block per batch, quantization.cpp:934-955)."""
    if G == 1:
        return shuffle_scale_impl(e)
    parts = [shuffle_scale_impl(e[g * rows:(g + 1) * rows]) for g in range(G)]
    return torch.cat([p.view(torch.uint8) for p in parts]).view(torch.float8_e8m0fnu)


def quantize_mxfp8_impl(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    axis: Optional[int],
    block_size: int,
    with_trans: bool = False,
    scaling_recipe: Optional[ScalingRecipe] = None,
    scaling_recipe_for_trans: Optional[ScalingRecipe] = None,
    exp_kmajor: bool = False,
):
    """MXFP8 quantization (quantization_impl.py:489-543 in the reference).

    ``exp_kmajor=True`` (an extension used by the autograd function) returns
    each exponent array as its ``[cols_pad/128, rows, 4]`` K-block-major
    storage (``PTA_MX_EXP_KMAJOR``) instead of ``[rows, cols_pad/32]``: the
    kernel then writes one 512-byte run per 128x128 tile and the GEMM reads
    the exponents of one K block for 64 rows from 256 contiguous bytes.
    """
    _check_hp(x)
    assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
    assert x.dtype in (torch.bfloat16, torch.float16), "Input must be BFloat16 or Half"
    x = x.contiguous()
    rr = _check_recipe(scaling_recipe)
    rc = _check_recipe(scaling_recipe_for_trans) if with_trans else rr
    if x.dim() == 2:
        G, M, N = 1, x.shape[0], x.shape[1]
    elif x.dim() == 3:
        G, M, N = x.shape
    else:
        raise ValueError(f"The input tensor must be 2D or 3D but got {x.dim()}D.")
    assert N % MXFP8_BLOCK_SIZE == 0, f"N must be divisible by {MXFP8_BLOCK_SIZE}"
    if with_trans:
        assert axis is None, "The axis must be None when with_trans is True."
        row, col = True, True
    else:
        if x.dim() == 2:
            assert axis in (0, 1), "The axis must be 0 or 1 when with_trans is False and x is 2D."
            row = axis == 1
        else:
            assert axis in (1, 2), "The axis must be 1 or 2 when with_trans is False and x is 3D."
            row = axis == 2
        col = not row
    Mp, Np = ceil_div(M, MXFP8_PADDING_ALIGN_SIZE) * 128, ceil_div(N, MXFP8_PADDING_ALIGN_SIZE) * 128
    dev = x.device
    q_row = e_row = q_col = e_col = None
    if row:
        q_row = torch.empty((G * M, Np), dtype=out_dtype, device=dev)
        e_row = torch.empty((Np // 128, G * M, 4) if exp_kmajor else (G * M, Np // 32), dtype=torch.uint8, device=dev)
    if col:
        q_col = torch.empty((G * N, Mp), dtype=out_dtype, device=dev)
        e_col = torch.empty((Mp // 128, G * N, 4) if exp_kmajor else (G * N, Mp // 32), dtype=torch.uint8, device=dev)
    _C.call(
        "pta_quantize_mxfp8", _C.ptr(x), _C.in_dtype_code(x.dtype), G, M, N, _C.ptr(q_row), _C.ptr(e_row),
        int(rr.use_2d_block), _C.ptr(q_col), _C.ptr(e_col), int(rc.use_2d_block), _C.fp8_code(out_dtype),
        _C.MX_EXP_KMAJOR if exp_kmajor else 0, _C.stream(dev),
    )

    def shape3(t, rows):
        if exp_kmajor and t.dtype == torch.uint8:
            return t  # K-block-major exponent storage, returned as is
        return t.view(G, -1, t.shape[-1]) if x.dim() == 3 else t

    if rr.shuffle_scale or rc.shuffle_scale:
        assert not exp_kmajor, "the scale shuffle and the K-block-major exponents are exclusive"
        if row and rr.shuffle_scale:
            e_row = _shuffle_batched(e_row, G, M).view(torch.uint8)
        if col and rc.shuffle_scale:
            e_col = _shuffle_batched(e_col, G, N).view(torch.uint8)

    outs = []
    if row:
        outs += [shape3(q_row, M), shape3(e_row, M).view(torch.float8_e8m0fnu)]
    if col:
        outs += [shape3(q_col, N), shape3(e_col, N).view(torch.float8_e8m0fnu)]
    return tuple(outs)


def grouped_quantize_mxfp8_impl(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    axis: Optional[int],
    block_size: int,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    with_trans: bool = False,
    scaling_recipe: Optional[ScalingRecipe] = None,
    scaling_recipe_for_trans: Optional[ScalingRecipe] = None,
):
    """MXFP8 quantization of grouped rows with per-group M padding (32 rowwise,
    128 colwise), padded layouts computed on the device
    (reference: quantization_impl.py:546-612, quantization.cpp:969-1195).

    with_trans: (q_row [M_pad_row, N_pad], s_row, q_col [N, M_pad_col], s_col,
    group_lens_padded_rowwise, group_offs_padded_rowwise,
    group_lens_padded_colwise, group_offs_padded_colwise).
    axis 1 (rowwise) / 0 (colwise): (q, s, group_lens_padded, group_offs_padded).
    """
    _check_hp(x)
    assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
    assert x.dtype in (torch.bfloat16, torch.float16), "Input must be BFloat16 or Half"
    assert x.dim() == 2 and x.is_contiguous(), "Input must be a contiguous 2D tensor"
    rr = _check_recipe(scaling_recipe)
    rc = _check_recipe(scaling_recipe_for_trans) if with_trans else rr
    if rr.use_2d_block or rc.use_2d_block:
        raise NotImplementedError("2-D exponent blocks are not implemented for grouped MXFP8 quantization")
    if rr.shuffle_scale or rc.shuffle_scale:
        raise NotImplementedError("the scale shuffle is not implemented for grouped MXFP8 quantization")
    M, N = x.shape
    assert N % MXFP8_BLOCK_SIZE == 0, f"N must be divisible by {MXFP8_BLOCK_SIZE}"
    G = group_lens.numel()
    dev = x.device
    if with_trans:
        row, col = True, True
    else:
        assert axis in (0, 1), "The axis must be 0 or 1 when with_trans is False."
        row, col = axis == 1, axis == 0
    Mr = ceil_div(M + G * 32, 32) * 32
    Mc = ceil_div(M + G * 128, 128) * 128
    Np = ceil_div(N, 128) * 128
    lens = group_lens.to(torch.int64).contiguous()
    offs = group_offs.to(torch.int64).contiguous()
    lr, orw = torch.empty_like(lens), torch.empty(G + 1, dtype=torch.int64, device=dev)
    lc, oc = torch.empty_like(lens), torch.empty(G + 1, dtype=torch.int64, device=dev)
    q_row = e_row = q_col = e_col = None
    if row:
        q_row = torch.empty((Mr, Np), dtype=out_dtype, device=dev)
        e_row = torch.empty((Mr, Np // 32), dtype=torch.uint8, device=dev)
    if col:
        q_col = torch.empty((N, Mc), dtype=out_dtype, device=dev)
        e_col = torch.empty((N, Mc // 32), dtype=torch.uint8, device=dev)
    _C.call(
        "pta_grouped_quantize_mxfp8", _C.ptr(x), _C.in_dtype_code(x.dtype), M, N, G, _C.ptr(lens), _C.ptr(offs),
        _C.ptr(q_row), _C.ptr(e_row), 0, _C.ptr(lr), _C.ptr(orw), _C.ptr(q_col), _C.ptr(e_col), 0, _C.ptr(lc),
        _C.ptr(oc), _C.fp8_code(out_dtype), _C.stream(dev),
    )
    e8 = torch.float8_e8m0fnu
    if with_trans:
        return q_row, e_row.view(e8), q_col, e_col.view(e8), lr, orw, lc, oc
    if row:
        return q_row, e_row.view(e8), lr, orw
    return q_col, e_col.view(e8), lc, oc


def dequantize_mxfp8_impl(
    x: torch.Tensor, out_dtype: torch.dtype, axis: int, block_size: int, scale_inv: torch.Tensor
) -> torch.Tensor:
    """Rowwise (axis 1 / 2): y has q's shape.  Colwise 2-D (axis 0): y[M_pad, N]
    = the transpose of q[N, M_pad].  Colwise 3-D (axis 1): y keeps q's layout
    [B, N, M_pad], as the reference's dequantize_mxfp8 returns it
    (quantization.cpp:283-357: a [B, N, M_pad] permutation of its output)."""
    assert x.is_contiguous(), "The x tensor must be contiguous."
    assert x.dim() in (2, 3), "The x must be a 2D or 3D tensor."
    assert scale_inv.dim() == x.dim(), "The scale_inv rank must match x."
    assert out_dtype in (torch.float16, torch.bfloat16, torch.float32)
    assert x.size(-1) % block_size == 0
    if x.dim() == 2:
        assert axis in (0, 1)
        rowwise = axis == 1
    else:
        assert axis in (1, 2)
        rowwise = axis == 2
    e = scale_inv.contiguous().view(torch.uint8)
    if x.dim() == 2:
        R, C = x.shape
        y = torch.empty((R, C) if rowwise else (C, R), dtype=out_dtype, device=x.device)
        _C.call(
            "pta_dequantize_mxfp8", _C.ptr(x), _C.fp8_code(x.dtype), R, C, _C.ptr(e), int(not rowwise), _C.ptr(y),
            _C.out_dtype_code(out_dtype), _C.stream(x.device),
        )
        return y
    # 3-D: every row of q[B, R, C] carries its own exponents in both directions,
    # and neither direction transposes the result, so one launch over B * R rows
    G, R, C = x.shape
    y = torch.empty((G, R, C), dtype=out_dtype, device=x.device)
    _C.call(
        "pta_dequantize_mxfp8", _C.ptr(x), _C.fp8_code(x.dtype), G * R, C, _C.ptr(e), 0, _C.ptr(y),
        _C.out_dtype_code(out_dtype), _C.stream(x.device),
    )
    return y


def grouped_dequantize_mxfp8_impl(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    axis: int,
    block_size: int,
    scale_inv: torch.Tensor,
    group_offs: torch.Tensor,
    group_offs_padded: torch.Tensor,
    total_M: Optional[int] = None,
) -> torch.Tensor:
    """Grouped MX dequantize back to packed rows (quantization_impl.py:727-754):
    axis 1 (rowwise, x = [padded rows, N_pad]) gives [total_M, N_pad]; axis 0
    (colwise, x = the transposed copy [N, padded rows]) gives [total_M, N]."""
    assert x.is_contiguous(), "The x tensor must be contiguous."
    assert x.dim() == 2, "The x must be 2D tensor."
    assert scale_inv.dim() == 2, "The scale_inv must be 2D tensor."
    assert scale_inv.is_contiguous(), "The scale_inv tensor must be contiguous."
    assert axis in (0, 1), "The axis must be 0 or 1."
    assert out_dtype in (torch.float16, torch.bfloat16, torch.float32), f"unsupported out dtype {out_dtype}"
    R, C = x.shape
    assert C % block_size == 0, "The last dimension of the x tensor must be divisible by the block size."
    G = group_offs.numel() - 1
    assert G >= 1 and group_offs_padded.numel() == group_offs.numel()
    if total_M is None:
        total_M = int(group_offs[-1].item())
    y = torch.empty((total_M, C if axis == 1 else R), dtype=out_dtype, device=x.device)
    _C.call(
        "pta_grouped_dequantize_mxfp8", _C.ptr(x), _C.fp8_code(x.dtype), R, C,
        _C.ptr(scale_inv.view(torch.uint8)), int(axis == 0), _C.ptr(group_offs.contiguous()),
        _C.ptr(group_offs_padded.contiguous()), G, total_M, _C.ptr(y), _C.out_dtype_code(out_dtype),
        _C.stream(x.device),
    )
    return y


def transpose_fp8(x: torch.Tensor) -> torch.Tensor:
    """Byte transpose of the last two dims of a 2D / 3D fp8 tensor."""
    x = x.contiguous()
    if x.dim() == 2:
        B, M, N = 1, x.shape[0], x.shape[1]
        y = torch.empty((N, M), dtype=x.dtype, device=x.device)
    else:
        B, M, N = x.shape
        y = torch.empty((B, N, M), dtype=x.dtype, device=x.device)
    _C.call("pta_transpose_u8", _C.ptr(x), B, M, N, _C.ptr(y), _C.stream(x.device))
    return y


# ---------------------------------------------------------------------------
# torch.compile support: the public quantize / dequantize ops are also
# registered as opaque custom ops with shape-only fake implementations, as the
# reference registers its impls (quantization_impl.py:74-486, native Meta
# kernels at csrc/pytorch/bindings_pytorch.cpp:182-231).  Eager calls keep the
# direct path: the custom-op dispatcher adds ~15 us of host time per call.
# ---------------------------------------------------------------------------
def _register(name: str, schema: str, impl, fake) -> None:
    op = torch.library.custom_op(f"primus_turbo_amd::{name}", impl, mutates_args=(), schema=schema)
    op.register_fake(fake)


def impl_for(name: str, raw):
    """``raw`` in eager mode; the registered custom op while torch.compile traces."""
    if torch.compiler.is_compiling():
        return getattr(torch.ops.primus_turbo_amd, name)
    return raw


def _f32(shape, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(shape, dtype=torch.float32, device=like.device)


def _fake_rowwise(x, out_dtype, axis, scale=None):
    ax = axis % x.dim()
    sshape = list(x.shape)
    sshape[ax] = 1
    return torch.empty(x.shape, dtype=out_dtype, device=x.device), _f32(sshape, x)


def _fake_block(x, dtype, axis, block_size=128):
    M, N = x.shape
    sshape = (M, ceil_div(N, block_size)) if axis % 2 == 1 else (ceil_div(M, block_size), N)
    return torch.empty((M, N), dtype=dtype, device=x.device), _f32(sshape, x)


def _fake_dual(x, dtype, block_size=128):
    M, N = x.shape
    return (torch.empty((M, N), dtype=dtype, device=x.device), _f32((M, ceil_div(N, block_size)), x),
            torch.empty((M, N), dtype=dtype, device=x.device), _f32((ceil_div(M, block_size), N), x))


def _fake_weight(w, dtype, block_size=128):
    lead = tuple(w.shape[:-2])
    M, N = w.shape[-2], w.shape[-1]
    return (torch.empty(w.shape, dtype=dtype, device=w.device),
            _f32(lead + (ceil_div(M, block_size), ceil_div(N, block_size)), w))


_register("quantize_fp8_tensorwise", "(Tensor x, ScalarType out_dtype, Tensor? scale=None) -> (Tensor, Tensor)",
          quantize_fp8_tensorwise_impl,
          lambda x, out_dtype, scale=None: (torch.empty(x.shape, dtype=out_dtype, device=x.device), _f32((), x)))
_register("quantize_fp8_rowwise", "(Tensor x, ScalarType out_dtype, int axis, Tensor? scale=None) -> (Tensor, Tensor)",
          quantize_fp8_rowwise_impl, _fake_rowwise)
_register("dequantize_fp8_tensorwise", "(Tensor x, ScalarType out_dtype, Tensor scale_inv) -> Tensor",
          dequantize_fp8_tensorwise_impl,
          lambda x, out_dtype, scale_inv: torch.empty(x.shape, dtype=out_dtype, device=x.device))
_register("dequantize_fp8_rowwise", "(Tensor x, ScalarType out_dtype, int axis, Tensor scale_inv) -> Tensor",
          dequantize_fp8_rowwise_impl,
          lambda x, out_dtype, axis, scale_inv: torch.empty(x.shape, dtype=out_dtype, device=x.device))
_register("quant_fp8_blockwise", "(Tensor x, ScalarType dtype, int axis, int block_size=128) -> (Tensor, Tensor)",
          quant_fp8_blockwise_impl, _fake_block)
_register("quant_fp8_blockwise_dual", "(Tensor x, ScalarType dtype, int block_size=128) -> (Tensor, Tensor, Tensor, Tensor)",
          lambda x, dtype, block_size=128: quant_fp8_blockwise_dual_impl(x, dtype, block_size), _fake_dual)
_register("quant_fp8_blockwise_for_weight", "(Tensor w, ScalarType dtype, int block_size=128) -> (Tensor, Tensor)",
          lambda w, dtype, block_size=128: tuple(t.contiguous() for t in quant_fp8_blockwise_for_weight_impl(w, dtype, block_size)),
          _fake_weight)
_register("dequant_fp8_blockwise",
          "(Tensor x_fp8, Tensor scale_inv, ScalarType out_dtype, int axis, int block_size=128) -> Tensor",
          dequant_fp8_blockwise_impl,
          lambda x_fp8, scale_inv, out_dtype, axis, block_size=128: torch.empty(x_fp8.shape, dtype=out_dtype,
                                                                                device=x_fp8.device))
_register("dequant_fp8_blockwise_for_weight",
          "(Tensor w_fp8, Tensor scale_inv, ScalarType out_dtype, int block_size=128) -> Tensor",
          dequant_fp8_blockwise_for_weight_impl,
          lambda w_fp8, scale_inv, out_dtype, block_size=128: torch.empty(w_fp8.shape, dtype=out_dtype,
                                                                          device=w_fp8.device))


def _mx_impl_flat(x, out_dtype, axis, block_size, with_trans, use_2d_row, shuffle_row, use_2d_col, shuffle_col):
    rr = ScalingRecipe(use_2d_block=use_2d_row, shuffle_scale=shuffle_row)
    rc = ScalingRecipe(use_2d_block=use_2d_col, shuffle_scale=shuffle_col)
    return list(quantize_mxfp8_impl(x, out_dtype, axis, block_size, with_trans, rr, rc if with_trans else None))


def _mx_fake_flat(x, out_dtype, axis, block_size, with_trans, use_2d_row, shuffle_row, use_2d_col, shuffle_col):
    G, M, N = (1, x.shape[0], x.shape[1]) if x.dim() == 2 else tuple(x.shape)
    Mp, Np = ceil_div(M, MXFP8_PADDING_ALIGN_SIZE) * 128, ceil_div(N, MXFP8_PADDING_ALIGN_SIZE) * 128
    if with_trans:
        row, col = True, True
    else:
        row = axis == (1 if x.dim() == 2 else 2)
        col = not row
    e8 = torch.float8_e8m0fnu

    def pair(rows, cols, shuffle):
        q = torch.empty((G * rows, cols), dtype=out_dtype, device=x.device)
        if shuffle:
            e = torch.empty((G * ceil_div(rows, 256) * 256, ceil_div(cols // 32, 8) * 8), dtype=e8, device=x.device)
        else:
            e = torch.empty((G * rows, cols // 32), dtype=e8, device=x.device)
        if x.dim() == 3:
            q, e = q.view(G, -1, q.shape[-1]), e.view(G, -1, e.shape[-1])
        return [q, e]

    outs = []
    if row:
        outs += pair(M, Np, shuffle_row)
    if col:
        outs += pair(N, Mp, shuffle_col)
    return outs


def _mx_deq_fake(x, out_dtype, axis, block_size, scale_inv):
    shape = list(x.shape)
    if x.dim() == 2 and axis == 0:  # 2-D colwise transposes back; 3-D keeps q's layout
        shape[-1], shape[-2] = shape[-2], shape[-1]
    return torch.empty(shape, dtype=out_dtype, device=x.device)


_register("quantize_mxfp8",
          "(Tensor x, ScalarType out_dtype, int? axis, int block_size, bool with_trans, bool use_2d_row, "
          "bool shuffle_row, bool use_2d_col, bool shuffle_col) -> Tensor[]", _mx_impl_flat, _mx_fake_flat)
_register("dequantize_mxfp8", "(Tensor x, ScalarType out_dtype, int axis, int block_size, Tensor scale_inv) -> Tensor",
          dequantize_mxfp8_impl, _mx_deq_fake)


def quantize_mxfp8_op(x, out_dtype, axis, block_size, with_trans=False, scaling_recipe=None,
                      scaling_recipe_for_trans=None):
    """quantize_mxfp8_impl for the public ops: the direct call in eager mode,
    the registered custom op (recipes passed as flags) under torch.compile."""
    if not torch.compiler.is_compiling():
        return quantize_mxfp8_impl(x, out_dtype, axis, block_size, with_trans, scaling_recipe,
                                   scaling_recipe_for_trans)
    rr = _check_recipe(scaling_recipe)
    rc = _check_recipe(scaling_recipe_for_trans) if with_trans else rr
    return tuple(torch.ops.primus_turbo_amd.quantize_mxfp8(x, out_dtype, axis, block_size, with_trans,
                                                           rr.use_2d_block, rr.shuffle_scale, rc.use_2d_block,
                                                           rc.shuffle_scale))
