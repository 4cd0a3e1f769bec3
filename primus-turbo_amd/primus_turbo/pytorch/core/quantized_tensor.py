"""Pre-quantized tensor types (the reference's
primus_turbo/pytorch/core/quantized_tensor.py:113-956).

``QuantizedTensor`` is a ``torch.Tensor`` wrapper subclass: its outer shape
and dtype are those of the high-precision tensor it came from, and it carries
the fp8 ``qdata``, ``scale_inv`` and the quantization metadata.  ``gemm_fp8``
/ ``grouped_gemm_fp8`` accept it (or a ``QuantizedTensorPair`` with a
column-direction copy) in place of a high-precision tensor.  ATen ops reaching
it are limited to the ones the reference supports without dequantizing:
view / reshape (inner-dim padding kept for MX), select, detach / alias and
t / transpose (exact for TENSORWISE, dequantize + re-quantize otherwise).
"""

from __future__ import annotations

from typing import Any, Callable, NamedTuple, Optional, Tuple

import torch

from primus_turbo.pytorch.core.low_precision import (
    MXFP8_BLOCK_SIZE,
    MXFP8_PADDING_ALIGN_SIZE,
    Float8QuantConfig,
    ScalingGranularity,
    ScalingRecipe,
    float8_e4m3,
    float8_e5m2,
)

_SUPPORTED_QUANTIZED_DTYPES = (float8_e4m3, float8_e5m2)
_SUPPORTED_GRANS = (
    ScalingGranularity.TENSORWISE,
    ScalingGranularity.ROWWISE,
    ScalingGranularity.BLOCKWISE,
    ScalingGranularity.MX_BLOCKWISE,
)


def _normalize_axis(axis: Optional[int], ndim: int) -> Optional[int]:
    if axis is None:
        return None
    return axis % ndim


def _inner_align(granularity: ScalingGranularity) -> int:
    """MX data is stored with its inner dim padded to 128; other layouts are tight."""
    return MXFP8_PADDING_ALIGN_SIZE if granularity == ScalingGranularity.MX_BLOCKWISE else 1


def _padded_shape(shape, align: int):
    if align <= 1 or len(shape) == 0:
        return tuple(shape)
    last = (shape[-1] + align - 1) // align * align
    return (*shape[:-1], last)


def check_quantized_tensor(
    quantized_tensor: "QuantizedTensor",
    config: Any,
    axis: Optional[int] = None,
    scaling_recipe: Optional[ScalingRecipe] = None,
) -> None:
    """Assert granularity / block_size (and optionally axis and recipe) match ``config``
    (quantized_tensor.py:113-145)."""
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


class QuantizedTensor(torch.Tensor):
    """fp8 data + scale_inv + quantization metadata behind the high-precision
    tensor's shape and dtype."""

    @staticmethod
    def __new__(
        cls,
        data: torch.Tensor,
        scale_inv: Optional[torch.Tensor],
        *,
        shape: torch.Size,
        orig_dtype: torch.dtype,
        dest_dtype: torch.dtype,
        granularity: ScalingGranularity,
        orig_group_lens: Optional[torch.Tensor] = None,
        orig_group_offs: Optional[torch.Tensor] = None,
        group_lens: Optional[torch.Tensor] = None,
        group_offs: Optional[torch.Tensor] = None,
        is_grouped_tensor: bool = False,
        block_size: Optional[int] = None,
        scaling_recipe: Optional[ScalingRecipe] = None,
        quantized_axis: Optional[int] = None,
        requires_grad: bool = False,
    ):
        assert dest_dtype in _SUPPORTED_QUANTIZED_DTYPES, "Unsupported quantized dtype"
        assert data.is_contiguous(), "data must be contiguous"
        assert scale_inv is None or scale_inv.is_contiguous(), "scale_inv must be contiguous"
        self = torch.Tensor._make_wrapper_subclass(
            cls, torch.Size(shape), dtype=orig_dtype, layout=data.layout, device=data.device,
            requires_grad=requires_grad,
        )
        self._data = data
        self._scale_inv = scale_inv
        self._orig_dtype = orig_dtype
        self._dest_dtype = dest_dtype
        self._granularity = granularity
        self._block_size = block_size
        self._scaling_recipe = scaling_recipe
        self._quantized_axis = quantized_axis
        self._group_lens = group_lens
        self._group_offs = group_offs
        self._orig_group_lens = orig_group_lens
        self._orig_group_offs = orig_group_offs
        self._is_grouped_tensor = is_grouped_tensor
        return self

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
        """Quantize ``hp_tensor`` (2-D or 3-D) and wrap the result
        (quantized_tensor.py:204-370).  With ``group_lens`` the rows of a 2-D
        packed-M tensor are split into groups: TENSORWISE / ROWWISE quantize
        it like a plain tensor, MX_BLOCKWISE pads each group (grouped
        quantize), BLOCKWISE is not available for grouped tensors (as in the
        reference, whose grouped quantize raises for it)."""
        assert hp_tensor.ndim in (2, 3), f"data must be a 2D or 3D tensor, got {hp_tensor.ndim}D"
        assert dest_dtype in _SUPPORTED_QUANTIZED_DTYPES, "Unsupported quantized dtype"
        assert granularity in _SUPPORTED_GRANS, f"Unsupported granularity {granularity}"
        if granularity == ScalingGranularity.BLOCKWISE:
            assert block_size is not None, "block_size must be provided for BLOCKWISE"
        if granularity == ScalingGranularity.MX_BLOCKWISE:
            assert block_size == MXFP8_BLOCK_SIZE, "block_size must be MXFP8_BLOCK_SIZE for MX_BLOCKWISE"
            assert scaling_recipe is not None, "scaling_recipe must be provided for MX_BLOCKWISE"
        if granularity != ScalingGranularity.TENSORWISE:
            assert axis is not None, "axis must be provided for non-TENSORWISE granularity"

        is_grouped = group_lens is not None
        orig_lens = orig_offs = lens = offs = None
        if is_grouped:
            assert hp_tensor.ndim == 2, f"Grouped quantized tensor expects a 2D packed-M tensor, got {hp_tensor.ndim}D"
            assert group_lens.is_cuda, "group_lens must be on CUDA"
            from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens

            orig_lens, orig_offs = group_lens, group_offs_from_lens(group_lens)
            if granularity in (ScalingGranularity.TENSORWISE, ScalingGranularity.ROWWISE):
                lens, offs = orig_lens, orig_offs
                data, scale_inv = cls._quantize(hp_tensor, dest_dtype, granularity, block_size, axis, scaling_recipe)
            else:
                from primus_turbo.pytorch.ops.quantization import grouped_quantize_fp8

                data, scale_inv, lens, offs = grouped_quantize_fp8(
                    hp_tensor.detach(), dest_dtype, granularity, orig_lens, orig_offs, block_size=block_size,
                    axis=_normalize_axis(axis, hp_tensor.ndim), scaling_recipe=scaling_recipe,
                )
        else:
            data, scale_inv = cls._quantize(hp_tensor, dest_dtype, granularity, block_size, axis, scaling_recipe)
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
            orig_group_lens=orig_lens,
            orig_group_offs=orig_offs,
            group_lens=lens,
            group_offs=offs,
            is_grouped_tensor=is_grouped,
            requires_grad=hp_tensor.requires_grad,
        )

    @staticmethod
    @torch.no_grad()
    def _quantize(hp, dest_dtype, granularity, block_size, axis, scaling_recipe):
        from primus_turbo.pytorch.ops.quantization import quantize_fp8

        return quantize_fp8(
            hp.detach(), dest_dtype, granularity, block_size=block_size, axis=_normalize_axis(axis, hp.ndim),
            scaling_recipe=scaling_recipe,
        )

    # ---- properties --------------------------------------------------------
    @property
    def qdata(self) -> torch.Tensor:
        assert self._data is not None, "qdata is None. Please call quantize() to quantize the data."
        return self._data

    @property
    def scale_inv(self) -> torch.Tensor:
        assert self._scale_inv is not None, "scale_inv is None. Please call quantize() to quantize the data."
        return self._scale_inv

    @property
    def dtype(self) -> torch.dtype:  # type: ignore[override]
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
        """Per-group row counts of the quantized layout (padded for MX)."""
        assert self._is_grouped_tensor, "This is not a grouped tensor."
        return self._group_lens

    @property
    def group_offs(self) -> torch.Tensor:
        """Prefix sums of ``group_lens`` along the quantized M axis."""
        assert self._is_grouped_tensor, "This is not a grouped tensor."
        return self._group_offs

    @property
    def _is_grouped(self) -> bool:
        return self._is_grouped_tensor

    # ---- conversions -------------------------------------------------------
    @torch.no_grad()
    def dequantize(self) -> torch.Tensor:
        """Back to the original dtype and shape (quantized_tensor.py:510-616)."""
        from primus_turbo.pytorch.ops.quantization import dequantize_fp8, grouped_dequantize_fp8

        g = self._granularity
        if self._is_grouped_tensor and g in (ScalingGranularity.BLOCKWISE, ScalingGranularity.MX_BLOCKWISE):
            out = grouped_dequantize_fp8(
                self._data, self._orig_dtype, g, self._orig_group_offs, self._group_offs,
                block_size=self._block_size, axis=self.quantized_axis, scale_inv=self._scale_inv,
                scaling_recipe=self._scaling_recipe, total_M=self.shape[0],
            )
        else:
            out = dequantize_fp8(
                self._data, self._orig_dtype, g, block_size=self._block_size, axis=self.quantized_axis,
                scale_inv=self._scale_inv, scaling_recipe=self._scaling_recipe,
            )
            if g == ScalingGranularity.MX_BLOCKWISE and out.dim() == 3 and self.quantized_axis == 1:
                out = out.transpose(1, 2)  # 3-D colwise MX dequantizes in the stored [B, N, M_pad] layout
        # MX outputs carry the 128-padding of the stored layout
        return out[..., : self.shape[-2], : self.shape[-1]].contiguous()

    def __repr__(self, *, tensor_contents=None) -> str:  # noqa: D105
        return (
            f"QuantizedTensor(shape={tuple(self.shape)}, dtype={self._dest_dtype}, granularity="
            f"{self._granularity.name}, block_size={self._block_size}, axis={self._quantized_axis}"
            f"{', grouped' if self._is_grouped_tensor else ''})"
        )

    # ---- torch.compile / FSDP hooks ----------------------------------------
    _INNER = ("_data", "_scale_inv", "_orig_group_lens", "_orig_group_offs", "_group_lens", "_group_offs")
    _META = ("_orig_dtype", "_dest_dtype", "_granularity", "_block_size", "_scaling_recipe",
             "_is_grouped_tensor", "_quantized_axis")

    def __tensor_flatten__(self):
        names = [n for n in self._INNER if getattr(self, n) is not None]
        return names, {n: getattr(self, n) for n in self._META}

    @staticmethod
    def __tensor_unflatten__(inner_tensors, metadata, outer_size, outer_stride):
        del outer_stride  # the wrapper is always dense
        return QuantizedTensor(
            inner_tensors["_data"],
            inner_tensors.get("_scale_inv"),
            shape=outer_size,
            orig_dtype=metadata["_orig_dtype"],
            dest_dtype=metadata["_dest_dtype"],
            granularity=metadata["_granularity"],
            block_size=metadata["_block_size"],
            scaling_recipe=metadata["_scaling_recipe"],
            quantized_axis=metadata["_quantized_axis"],
            orig_group_lens=inner_tensors.get("_orig_group_lens"),
            orig_group_offs=inner_tensors.get("_orig_group_offs"),
            group_lens=inner_tensors.get("_group_lens"),
            group_offs=inner_tensors.get("_group_offs"),
            is_grouped_tensor=metadata["_is_grouped_tensor"],
        )

    # ---- views without dequantizing -----------------------------------------
    def _rewrap(self, data: torch.Tensor, scale_inv: Optional[torch.Tensor], shape) -> "QuantizedTensor":
        """Same metadata (grouped fields included) over new buffers and shape."""
        return QuantizedTensor(
            data,
            scale_inv,
            shape=torch.Size(shape),
            orig_dtype=self._orig_dtype,
            dest_dtype=self._dest_dtype,
            granularity=self._granularity,
            block_size=self._block_size,
            scaling_recipe=self._scaling_recipe,
            quantized_axis=self._quantized_axis,
            orig_group_lens=self._orig_group_lens,
            orig_group_offs=self._orig_group_offs,
            group_lens=self._group_lens,
            group_offs=self._group_offs,
            is_grouped_tensor=self._is_grouped_tensor,
            requires_grad=data.requires_grad,
        )

    def _reshaped(self, shape, op: Callable) -> "QuantizedTensor":
        """Apply a view / reshape to the buffers: the data takes the target
        shape (inner dim padded as stored), MX exponents follow with one byte
        per 32 elements; other scales are kept (same rank required)."""
        shape = torch.Size(shape)
        assert len(shape) == self._data.ndim, "view / reshape must keep the rank of the quantized data"
        if shape == self.shape:
            return self._rewrap(self._data, self._scale_inv, shape)
        data_shape = _padded_shape(shape, _inner_align(self._granularity))
        data = op(self._data, data_shape)
        sinv = self._scale_inv
        if self._granularity == ScalingGranularity.MX_BLOCKWISE and sinv is not None:
            sinv = op(sinv, (*data_shape[:-1], (data_shape[-1] + self._block_size - 1) // self._block_size))
        return self._rewrap(data, sinv, shape)

    def view(self, *shape) -> "QuantizedTensor":
        """View without dequantizing (autograd-aware)."""
        return _ViewFn.apply(self, _shape_arg(shape))

    def reshape(self, *shape) -> "QuantizedTensor":
        """Reshape without dequantizing (autograd-aware)."""
        return _ReshapeFn.apply(self, _shape_arg(shape))

    def _transposed(self, dim0: int, dim1: int) -> "QuantizedTensor":
        """TENSORWISE: byte transpose with the same scalar scale (exact); other
        granularities: dequantize, transpose, re-quantize along axis -2
        (quantized_tensor.py:740-779)."""
        from primus_turbo.pytorch.kernels.quantization.quantization_impl import transpose_fp8

        nd = self.dim()
        d0, d1 = dim0 % nd, dim1 % nd
        if d0 == d1:
            return self._rewrap(self._data, self._scale_inv, self.shape)
        assert not self._is_grouped_tensor, "transpose is not supported for grouped QuantizedTensor"
        assert {d0, d1} == {nd - 2, nd - 1}, "only the last two dims can be transposed"
        new_shape = list(self.shape)
        new_shape[d0], new_shape[d1] = new_shape[d1], new_shape[d0]
        if self._granularity == ScalingGranularity.TENSORWISE:
            return self._rewrap(transpose_fp8(self._data), self._scale_inv, new_shape)
        hp_t = self.dequantize().transpose(d0, d1).contiguous()
        return QuantizedTensor.quantize(
            hp_t, self._dest_dtype, self._granularity, axis=-2, block_size=self._block_size,
            scaling_recipe=self._scaling_recipe,
        )

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        t = args[0] if args else None
        if isinstance(t, QuantizedTensor):
            if func in (torch.ops.aten.view.default, torch.ops.aten._unsafe_view.default):
                return t._reshaped(args[1], torch.Tensor.view)
            if func == torch.ops.aten.reshape.default:
                return t._reshaped(args[1], torch.Tensor.reshape)
            if func == torch.ops.aten.select.int:
                return func(t._data, *args[1:], **kwargs)
            if func in (torch.ops.aten.detach.default, torch.ops.aten.alias.default):
                return t._rewrap(t._data.detach(), None if t._scale_inv is None else t._scale_inv.detach(), t.shape)
            if func == torch.ops.aten.t.default:
                assert t.dim() == 2, "t() expects a 2D QuantizedTensor"
                return t._transposed(0, 1)
            if func == torch.ops.aten.transpose.int:
                return t._transposed(args[1], args[2])
        raise NotImplementedError(f"Unsupported dispatch: {func}")

    __torch_function__ = torch._C._disabled_torch_function_impl


def _shape_arg(shape) -> Tuple[int, ...]:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list, torch.Size)):
        shape = tuple(shape[0])
    return tuple(int(s) for s in shape)


class _ViewFn(torch.autograd.Function):
    """View of a QuantizedTensor; the gradient flows back in the input's shape."""

    @staticmethod
    def forward(ctx, tensor: QuantizedTensor, shape: Tuple[int, ...]) -> QuantizedTensor:
        ctx.in_shape = tensor.shape
        return tensor._reshaped(_resolve(shape, tensor.shape), torch.Tensor.view)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        return grad.reshape(ctx.in_shape), None


class _ReshapeFn(torch.autograd.Function):
    """Reshape of a QuantizedTensor; the gradient flows back in the input's shape."""

    @staticmethod
    def forward(ctx, tensor: QuantizedTensor, shape: Tuple[int, ...]) -> QuantizedTensor:
        ctx.in_shape = tensor.shape
        return tensor._reshaped(_resolve(shape, tensor.shape), torch.Tensor.reshape)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        return grad.reshape(ctx.in_shape), None


def _resolve(shape: Tuple[int, ...], src: torch.Size) -> Tuple[int, ...]:
    """Replace a single -1 in ``shape`` by the size that keeps the element count."""
    if -1 not in shape:
        return shape
    known = 1
    for s in shape:
        if s != -1:
            known *= s
    total = 1
    for s in src:
        total *= s
    return tuple(total // known if s == -1 else s for s in shape)


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
