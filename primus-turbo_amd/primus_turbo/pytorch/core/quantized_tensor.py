"""Pre-quantized tensor types (API subset of the reference's
primus_turbo/pytorch/core/quantized_tensor.py:113-956).

``QuantizedTensor`` carries fp8 ``qdata`` + ``scale_inv`` and the quantization
metadata; ``gemm_fp8`` / ``grouped_gemm_fp8`` accept it (or a
``QuantizedTensorPair`` with a column-direction copy) in place of a
high-precision tensor.  Unlike the reference this is a plain Python object,
not a ``torch.Tensor`` wrapper subclass: view / reshape / transpose are
explicit methods.
"""

from __future__ import annotations

from typing import Any, NamedTuple, Optional, Tuple

import torch

from primus_turbo.pytorch.core.low_precision import (
    MXFP8_BLOCK_SIZE,
    Float8QuantConfig,
    ScalingGranularity,
    ScalingRecipe,
    float8_e4m3,
    float8_e5m2,
)

_SUPPORTED_QUANTIZED_DTYPES = (float8_e4m3, float8_e5m2)


def _normalize_axis(axis: Optional[int], ndim: int) -> Optional[int]:
    if axis is None:
        return None
    return axis % ndim


def check_quantized_tensor(
    quantized_tensor: "QuantizedTensor",
    config: Any,
    axis: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
) -> None:
    """Assert granularity / block_size (and optionally axis and recipe) match ``config``."""
    assert quantized_tensor.granularity == config.granularity, (
        f"QuantizedTensor granularity {quantized_tensor.granularity} does not match config "
        f"granularity {config.granularity}"
    )
    assert quantized_tensor.block_size == config.block_size, (
        f"QuantizedTensor block_size {quantized_tensor.block_size} does not match config "
        f"block_size {config.block_size}"
    )
    if axis is not None:
        normalized_axis = _normalize_axis(axis, quantized_tensor.qdata.ndim)
        assert quantized_tensor.quantized_axis == normalized_axis, (
            f"QuantizedTensor quantized_axis {quantized_tensor.quantized_axis} does not match axis={normalized_axis}"
        )
    if scaling_recipe is not None:
        assert quantized_tensor.scaling_recipe == scaling_recipe, (
            f"QuantizedTensor scaling_recipe {quantized_tensor.scaling_recipe} does not match "
            f"config scaling_recipe {scaling_recipe}"
        )


class QuantizedTensor:
    """fp8 data + scale_inv + quantization metadata."""

    def __init__(
        self,
        data: torch.Tensor,
        scale_inv: torch.Tensor,
        *,
        shape: torch.Size,
        orig_dtype: torch.dtype,
        dest_dtype: torch.dtype,
        granularity: ScalingGranularity,
        block_size: Optional[int] = None,
        scaling_recipe: Optional[ScalingRecipe] = None,
        quantized_axis: Optional[int] = None,
        group_lens: Optional[torch.Tensor] = None,
        group_offs: Optional[torch.Tensor] = None,
        is_grouped_tensor: bool = False,
        requires_grad: bool = False,
    ):
        assert dest_dtype in _SUPPORTED_QUANTIZED_DTYPES, "Unsupported quantized dtype"
        self._data = data
        self._scale_inv = scale_inv
        self._shape = torch.Size(shape)
        self._orig_dtype = orig_dtype
        self._dest_dtype = dest_dtype
        self._granularity = granularity
        self._block_size = block_size
        self._scaling_recipe = scaling_recipe
        self._quantized_axis = quantized_axis
        self._group_lens = group_lens
        self._group_offs = group_offs
        self._is_grouped_tensor = is_grouped_tensor
        self.requires_grad = requires_grad

    # ---- factory ---------------------------------------------------------
    @classmethod
    def quantize(
        cls,
        hp_tensor: torch.Tensor,
        dest_dtype: torch.dtype,
        granularity: ScalingGranularity,
        *,
        axis: Optional[int] = None,
        group_lens: Optional[torch.Tensor] = None,
        block_size: Optional[int] = None,
        scaling_recipe: Optional[ScalingRecipe] = None,
    ) -> "QuantizedTensor":
        from primus_turbo.pytorch.ops.quantization import quantize_fp8

        assert hp_tensor.ndim in (2, 3), f"data must be a 2D or 3D tensor, got {hp_tensor.ndim}D"
        assert dest_dtype in _SUPPORTED_QUANTIZED_DTYPES, "Unsupported quantized dtype"
        if granularity != ScalingGranularity.TENSORWISE:
            assert axis is not None, "axis must be provided for non-TENSORWISE granularity"
        if granularity == ScalingGranularity.BLOCKWISE:
            assert block_size is not None, "block_size must be provided for BLOCKWISE"
        if granularity == ScalingGranularity.MX_BLOCKWISE:
            assert block_size == MXFP8_BLOCK_SIZE, "block_size must be MXFP8_BLOCK_SIZE for MX_BLOCKWISE"
            assert scaling_recipe is not None, "scaling_recipe must be provided for MX_BLOCKWISE"
        is_grouped = group_lens is not None
        if is_grouped:
            # tensorwise / rowwise grouped tensors quantize like plain tensors
            # (quantized_tensor.py:292-310 in the reference)
            assert granularity in (ScalingGranularity.TENSORWISE, ScalingGranularity.ROWWISE), (
                "grouped QuantizedTensor supports TENSORWISE and ROWWISE in this build"
            )
            from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens

            group_offs = group_offs_from_lens(group_lens)
        else:
            group_offs = None
        ax = _normalize_axis(axis, hp_tensor.ndim)
        data, scale_inv = quantize_fp8(
            hp_tensor.detach(), dest_dtype, granularity, block_size=block_size, axis=ax, scaling_recipe=scaling_recipe
        )
        return cls(
            data,
            scale_inv,
            shape=hp_tensor.shape,
            orig_dtype=hp_tensor.dtype,
            dest_dtype=dest_dtype,
            granularity=granularity,
            block_size=block_size,
            scaling_recipe=scaling_recipe,
            quantized_axis=axis,
            group_lens=group_lens,
            group_offs=group_offs,
            is_grouped_tensor=is_grouped,
            requires_grad=hp_tensor.requires_grad,
        )

    # ---- properties --------------------------------------------------------
    @property
    def qdata(self) -> torch.Tensor:
        return self._data

    @property
    def scale_inv(self) -> torch.Tensor:
        return self._scale_inv

    @property
    def shape(self) -> torch.Size:
        return self._shape

    def size(self, dim: Optional[int] = None):
        return self._shape if dim is None else self._shape[dim]

    def dim(self) -> int:
        return len(self._shape)

    @property
    def ndim(self) -> int:
        return len(self._shape)

    @property
    def device(self):
        return self._data.device

    @property
    def dtype(self) -> torch.dtype:
        return self._orig_dtype

    @property
    def real_dtype(self) -> torch.dtype:
        return self._data.dtype

    @property
    def granularity(self) -> ScalingGranularity:
        return self._granularity

    @property
    def block_size(self) -> Optional[int]:
        return self._block_size

    @property
    def scaling_recipe(self) -> Optional[ScalingRecipe]:
        return self._scaling_recipe

    @property
    def quantized_axis(self) -> Optional[int]:
        return _normalize_axis(self._quantized_axis, self._data.ndim)

    @property
    def group_lens(self) -> torch.Tensor:
        assert self._is_grouped_tensor, "This is not a grouped tensor."
        return self._group_lens

    @property
    def group_offs(self) -> torch.Tensor:
        assert self._is_grouped_tensor, "This is not a grouped tensor."
        return self._group_offs

    @property
    def _is_grouped(self) -> bool:
        return self._is_grouped_tensor

    # ---- conversions -------------------------------------------------------
    def dequantize(self) -> torch.Tensor:
        from primus_turbo.pytorch.ops.quantization import dequantize_fp8

        out = dequantize_fp8(
            self._data,
            self._orig_dtype,
            self._granularity,
            block_size=self._block_size,
            axis=self.quantized_axis,
            scale_inv=self._scale_inv,
            scaling_recipe=self._scaling_recipe,
        )
        if self._granularity == ScalingGranularity.MX_BLOCKWISE:
            if out.ndim == 2:
                out = out[: self._shape[0], : self._shape[1]]
            else:
                out = out[:, : self._shape[-2], : self._shape[-1]]
            out = out.contiguous()
        return out

    def t(self) -> "QuantizedTensor":
        assert self.dim() == 2, "t() expects a 2D QuantizedTensor"
        return self.transpose(0, 1)

    def transpose(self, dim0: int, dim1: int) -> "QuantizedTensor":
        """TENSORWISE: byte transpose (exact); other granularities re-quantize
        the dequantized transpose along axis -2, as the reference does
        (quantized_tensor.py:740-775)."""
        from primus_turbo.pytorch.kernels.quantization.quantization_impl import transpose_fp8

        nd = self.dim()
        d0, d1 = dim0 % nd, dim1 % nd
        if d0 == d1:
            return self
        assert {d0, d1} == {nd - 2, nd - 1}, "only the last two dims can be transposed"
        new_shape = list(self._shape)
        new_shape[d0], new_shape[d1] = new_shape[d1], new_shape[d0]
        if self._granularity == ScalingGranularity.TENSORWISE:
            return QuantizedTensor(
                transpose_fp8(self._data),
                self._scale_inv,
                shape=torch.Size(new_shape),
                orig_dtype=self._orig_dtype,
                dest_dtype=self._dest_dtype,
                granularity=self._granularity,
                block_size=self._block_size,
                scaling_recipe=self._scaling_recipe,
                quantized_axis=self._quantized_axis,
            )
        hp_t = self.dequantize().transpose(d0, d1).contiguous()
        return QuantizedTensor.quantize(
            hp_t,
            self._dest_dtype,
            self._granularity,
            axis=-2,
            block_size=self._block_size,
            scaling_recipe=self._scaling_recipe,
        )

    def contiguous(self) -> "QuantizedTensor":
        return self

    def __repr__(self) -> str:
        return (
            f"QuantizedTensor(shape={tuple(self._shape)}, dtype={self._dest_dtype}, granularity="
            f"{self._granularity.name}, block_size={self._block_size}, axis={self._quantized_axis})"
        )


class QuantizedTensorPair(NamedTuple):
    """Row-wise quantized tensor and its (optional) column-wise copy."""

    data: QuantizedTensor
    data_t: Optional[QuantizedTensor] = None


def create_quantized_weight(
    weight: torch.Tensor,
    dest_dtype: torch.dtype,
    quant_config: Float8QuantConfig,
    need_weight_transpose_cache: bool = False,
) -> Tuple[QuantizedTensor, Optional[QuantizedTensor]]:
    """Quantize a weight once (quantized_tensor.py:897-956 in the reference)."""
    if quant_config.granularity in (ScalingGranularity.BLOCKWISE, ScalingGranularity.MX_BLOCKWISE):
        recipe = ScalingRecipe(use_2d_block=True)
    else:
        recipe = ScalingRecipe()
    qw = QuantizedTensor.quantize(
        weight, dest_dtype, quant_config.granularity, block_size=quant_config.block_size,
        scaling_recipe=recipe, axis=-1,
    )
    qw_t = None
    if need_weight_transpose_cache:
        g = quant_config.granularity
        if g == ScalingGranularity.TENSORWISE:
            qw_t = qw.transpose(-2, -1)
        elif g == ScalingGranularity.ROWWISE:
            qw_t = QuantizedTensor.quantize(
                weight.transpose(-2, -1).contiguous(), dest_dtype, g, block_size=quant_config.block_size,
                scaling_recipe=recipe, axis=-2,
            )
        else:
            qw_t = QuantizedTensor.quantize(
                weight, dest_dtype, g, block_size=quant_config.block_size, scaling_recipe=recipe, axis=-2
            )
    return qw, qw_t
