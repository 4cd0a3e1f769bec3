"""Public FP8 quantization ops (same signatures as the reference's
primus_turbo/pytorch/ops/quantization.py:52-269)."""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from primus_turbo.pytorch.core.low_precision import (
    MXFP8_BLOCK_SIZE,
    ScalingGranularity,
    ScalingRecipe,
)
from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
    dequant_fp8_blockwise_for_weight_impl,
    dequant_fp8_blockwise_impl,
    dequantize_fp8_rowwise_impl,
    dequantize_fp8_tensorwise_impl,
    dequantize_mxfp8_impl,
    grouped_dequantize_mxfp8_impl,
    grouped_quantize_mxfp8_impl,
    impl_for,
    quantize_mxfp8_op,
    quant_fp8_blockwise_dual_impl,
    quant_fp8_blockwise_for_weight_impl,
    quant_fp8_blockwise_impl,
    quantize_fp8_rowwise_impl,
    quantize_fp8_tensorwise_impl,
)

__all__ = [
    "quantize_fp8",
    "quantize_fp8_with_trans",
    "dequantize_fp8",
    "grouped_quantize_fp8",
    "grouped_quantize_fp8_with_trans",
    "grouped_dequantize_fp8",
]


def quantize_fp8(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    *,
    block_size: Optional[int] = None,
    axis: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """FP8 quantize; returns (fp8 tensor, scale_inv).

    TENSORWISE: 0-dim scale_inv.  ROWWISE: ``axis`` required, scale_inv keeps
    x's shape with ``axis`` set to 1.  BLOCKWISE: 1 x block (axis 1) or
    block x 1 (axis 0) scales, or block x block weight scales with
    ``scaling_recipe.use_2d_block``.  MX_BLOCKWISE: block 32, E8M0 scales;
    axis 1 (2D) / 2 (3D) is rowwise, axis 0 / 1 is colwise with transposed output.
    """
    if granularity == ScalingGranularity.TENSORWISE:
        return impl_for("quantize_fp8_tensorwise", quantize_fp8_tensorwise_impl)(x, out_dtype)
    elif granularity == ScalingGranularity.ROWWISE:
        return impl_for("quantize_fp8_rowwise", quantize_fp8_rowwise_impl)(x, out_dtype, axis)
    elif granularity == ScalingGranularity.BLOCKWISE:
        assert block_size is not None, "block_size must be specified for BLOCKWISE quantization"
        if scaling_recipe is not None and scaling_recipe.use_2d_block:
            return impl_for("quant_fp8_blockwise_for_weight", quant_fp8_blockwise_for_weight_impl)(x, out_dtype, block_size)
        assert axis is not None, "axis must be specified for 1D BLOCKWISE quantization"
        return impl_for("quant_fp8_blockwise", quant_fp8_blockwise_impl)(x, out_dtype, axis, block_size)
    elif granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return quantize_mxfp8_op(x, out_dtype, axis, block_size, False, scaling_recipe)
    else:
        raise NotImplementedError(f"Unknown granularity {granularity}")


def quantize_fp8_with_trans(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    *,
    block_size: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
    scaling_recipe_for_trans: Optional[ScalingRecipe] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Row- and column-direction quantization in one pass: (q_row, s_row, q_col, s_col)."""
    if granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return quantize_mxfp8_op(x, out_dtype, None, block_size, True, scaling_recipe, scaling_recipe_for_trans)
    elif granularity == ScalingGranularity.BLOCKWISE:
        return impl_for("quant_fp8_blockwise_dual", quant_fp8_blockwise_dual_impl)(x, out_dtype, block_size)
    else:
        raise NotImplementedError(f"Unknown granularity {granularity}")


def grouped_quantize_fp8(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    *,
    block_size: Optional[int] = None,
    axis: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
):
    """Grouped MXFP8 quantization along one axis (ops/quantization.py:144-180):
    returns (q, scale, group_lens_padded, group_offs_padded)."""
    if granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return grouped_quantize_mxfp8_impl(x, out_dtype, axis, block_size, group_lens, group_offs, False,
                                           scaling_recipe)
    raise NotImplementedError(f"Unknown granularity {granularity}")


def grouped_quantize_fp8_with_trans(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    group_lens: torch.Tensor,
    group_offs: torch.Tensor,
    *,
    block_size: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
    scaling_recipe_for_trans: Optional[ScalingRecipe] = None,
):
    """Grouped MXFP8 rowwise + colwise quantization (ops/quantization.py:183-222):
    returns (q_row, s_row, q_col, s_col, group_lens_padded_rowwise,
    group_offs_padded_rowwise, group_lens_padded_colwise, group_offs_padded_colwise)."""
    if granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return grouped_quantize_mxfp8_impl(x, out_dtype, None, block_size, group_lens, group_offs, True,
                                           scaling_recipe, scaling_recipe_for_trans)
    raise NotImplementedError(f"Unknown granularity {granularity}")


def dequantize_fp8(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    *,
    block_size: Optional[int] = None,
    axis: Optional[int] = None,
    scale_inv: torch.Tensor,
    scaling_recipe: Optional[ScalingRecipe] = None,
):
    """FP8 dequantize: out_dtype(float(x) * scale_inv) with the granularity's scale layout."""
    if granularity == ScalingGranularity.TENSORWISE:
        return impl_for("dequantize_fp8_tensorwise", dequantize_fp8_tensorwise_impl)(x, out_dtype, scale_inv)
    elif granularity == ScalingGranularity.ROWWISE:
        if axis is None:
            raise ValueError("axis must be specified for rowwise FP8 de-quantization")
        return impl_for("dequantize_fp8_rowwise", dequantize_fp8_rowwise_impl)(x, out_dtype, axis, scale_inv)
    elif granularity == ScalingGranularity.BLOCKWISE:
        assert block_size is not None, "block_size must be specified for BLOCKWISE de-quantization"
        if scaling_recipe is not None and scaling_recipe.use_2d_block:
            return impl_for("dequant_fp8_blockwise_for_weight", dequant_fp8_blockwise_for_weight_impl)(
                x, scale_inv, out_dtype, block_size)
        assert axis is not None, "axis must be specified for 1D BLOCKWISE de-quantization"
        return impl_for("dequant_fp8_blockwise", dequant_fp8_blockwise_impl)(x, scale_inv, out_dtype, axis, block_size)
    elif granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return impl_for("dequantize_mxfp8", dequantize_mxfp8_impl)(x, out_dtype, axis, block_size, scale_inv)
    else:
        raise NotImplementedError(f"Unknown granularity {granularity}")


def grouped_dequantize_fp8(
    x: torch.Tensor,
    out_dtype: torch.dtype,
    granularity: ScalingGranularity,
    group_offs: torch.Tensor,
    group_offs_padded: torch.Tensor,
    *,
    block_size: Optional[int] = None,
    axis: Optional[int] = None,
    scale_inv: torch.Tensor,
    scaling_recipe: Optional[ScalingRecipe] = None,
    total_M: Optional[int] = None,
) -> torch.Tensor:
    """Grouped FP8 dequantize (ops/quantization.py:272-296): MX_BLOCKWISE only."""
    if granularity == ScalingGranularity.MX_BLOCKWISE:
        assert block_size == MXFP8_BLOCK_SIZE, f"The block size must be {MXFP8_BLOCK_SIZE} for MXFP8 quantization"
        return grouped_dequantize_mxfp8_impl(
            x, out_dtype, axis, block_size, scale_inv, group_offs, group_offs_padded, total_M
        )
    raise NotImplementedError(f"Unknown granularity {granularity}")
