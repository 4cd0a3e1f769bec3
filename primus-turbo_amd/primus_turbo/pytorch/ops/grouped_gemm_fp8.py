"""grouped_gemm_fp8: MoE expert GEMMs with FP8 quantization and autograd
(drop-in for primus_turbo/pytorch/ops/grouped_gemm_fp8.py:75-904).

Group lengths and offsets stay on the device throughout (no host sync).
"""

from __future__ import annotations

from typing import Optional, Union

import torch

from primus_turbo.pytorch.core.low_precision import (
    Float8QuantConfig,
    Format,
    ScalingGranularity,
    ScalingRecipe,
    float8_e4m3,
    float8_e5m2,
)
from primus_turbo.pytorch.core.quantized_tensor import (
    QuantizedTensor,
    QuantizedTensorPair,
    check_quantized_tensor,
)
from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_fp8_impl import (
    grouped_gemm_fp8_impl,
    grouped_gemm_fp8_variable_k_impl,
    grouped_gemm_fp8_variable_k_nt_impl,
)
from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
    grouped_quantize_mxfp8_impl,
    quant_fp8_blockwise_for_weight_impl,
    quant_fp8_blockwise_segment_m_row_col_impl,
    quantize_mxfp8_impl,
    transpose_fp8,
)

__all__ = ["grouped_gemm_fp8"]


def _get_fp8_dtype(format: Format, is_fwd_stage: bool):
    if format == Format.E4M3:
        return float8_e4m3
    elif format == Format.E5M2:
        return float8_e5m2
    elif format == Format.HYBRID:
        return float8_e4m3 if is_fwd_stage else float8_e5m2
    raise ValueError(f"Unsupported FP8 format: {format}")


class FP8GroupedGemmBlockFunc(torch.autograd.Function):
    """BLOCKWISE (grouped_gemm_fp8.py:75-211): 1 x 128 activations, 128 x 128 weights,
    128-padded segments for the variable-K wgrad."""

    @staticmethod
    def forward(ctx, a, b, group_lens, group_offs, trans_b, out_dtype, config, num_cu):
        assert config.granularity == ScalingGranularity.BLOCKWISE
        assert config.block_size in [128], "Only block_size 128 is supported currently."
        assert a.ndim == 2, "Input tensor must be 2-dimensional."
        assert b.ndim == 3, "Weight tensor must be 3-dimensional."
        assert group_lens.size(0) == b.size(0), "group_lens size must match b size(0)."
        assert out_dtype in [torch.float16, torch.bfloat16]
        fdt = _get_fp8_dtype(config.format, True)
        bs = config.block_size
        # column copy transposed ([K, M_pad], K-contiguous for the variable-K wgrad)
        a_row, a_colT, a_s_row, a_s_col, _, _ = quant_fp8_blockwise_segment_m_row_col_impl(
            a.detach().contiguous(), fdt, bs, group_lens, group_offs, col_transposed=True
        )
        b_fp8, b_s, b_fp8_t = quant_fp8_blockwise_for_weight_impl(b.detach().contiguous(), fdt, block_size=bs,
                                                                  with_transpose=True)
        d0, d1 = b.shape[1], b.shape[2]
        # both GEMMs run NT: the operand whose rows are the GEMM's N dimension
        # is the stored weight or its transposed copy (rows padded to 128 with
        # zero bytes, sliced back to the true length when they differ); the
        # 128 x 128 scales follow with their block axes exchanged as needed.
        b_t_s = b_s.transpose(1, 2).contiguous()
        bt = b_fp8_t if b_fp8_t.shape[2] == d0 else b_fp8_t[:, :, :d0].contiguous()
        if trans_b:  # fwd rows n = b rows; dgrad rows k = transposed copy
            fwd_b, fwd_s, bwd_b, bwd_s = b_fp8, b_s, bt, b_t_s
        else:        # fwd rows n = transposed copy; dgrad rows k = b rows
            fwd_b, fwd_s, bwd_b, bwd_s = bt, b_t_s, b_fp8, b_s
        out = grouped_gemm_fp8_impl(a_row, fwd_b, a_s_row, fwd_s, group_lens, group_offs, False, True, out_dtype,
                                    config.granularity.value, num_cu)
        ctx.save_for_backward(a_colT, a_s_col, bwd_b, bwd_s, group_lens, group_offs)
        ctx.trans_b, ctx.config, ctx.out_dtype, ctx.num_cu = trans_b, config, out_dtype, num_cu
        return out

    @staticmethod
    def backward(ctx, grad_out):
        a_colT, a_s_col, bwd_b, bwd_s, group_lens, group_offs = ctx.saved_tensors
        bs = ctx.config.block_size
        gdt = _get_fp8_dtype(ctx.config.format, False)
        g_row, g_colT, g_s_row, g_s_col, vk_lens, vk_offs = quant_fp8_blockwise_segment_m_row_col_impl(
            grad_out.contiguous(), gdt, bs, group_lens, group_offs, col_transposed=True
        )
        # dgrad: grad_a[m, k] = sum_n grad_out[m, n] b[g](n, k), NT on rows k
        grad_a = grouped_gemm_fp8_impl(g_row, bwd_b, g_s_row, bwd_s, group_lens, group_offs, False, True,
                                       ctx.out_dtype, ctx.config.granularity.value, ctx.num_cu)
        # wgrad over each group's 128-padded rows, NT on the transposed column copies:
        # dW[g] [N, K] = g_colT[:, seg] . a_colT[:, seg]^T (or [K, N] for trans_b=False)
        G = group_lens.shape[0]
        gran = ctx.config.granularity.value
        if ctx.trans_b:
            grad_b = grouped_gemm_fp8_variable_k_nt_impl(g_colT, a_colT, g_s_col, a_s_col, G, vk_offs, False,
                                                         ctx.out_dtype, gran)
        else:
            grad_b = grouped_gemm_fp8_variable_k_nt_impl(a_colT, g_colT, a_s_col, g_s_col, G, vk_offs, False,
                                                         ctx.out_dtype, gran)
        return grad_a, grad_b, None, None, None, None, None, None


class FP8GroupedGemmRowFunc(torch.autograd.Function):
    """ROWWISE (grouped_gemm_fp8.py:214-379)."""

    @staticmethod
    def forward(ctx, a, b, a_t, b_t, group_lens, group_offs, trans_b, out_dtype, config, num_cu):
        g = ScalingGranularity.ROWWISE
        if isinstance(a, QuantizedTensor):
            check_quantized_tensor(a, config, axis=-1)
            qa = a
        else:
            qa = QuantizedTensor.quantize(a, _get_fp8_dtype(config.format, True), g, axis=-1,
                                          block_size=config.block_size, group_lens=group_lens)
        b_row_axis = -1 if trans_b else -2
        b_col_axis = -2 if trans_b else -1
        if isinstance(b, QuantizedTensor):
            check_quantized_tensor(b, config, axis=b_row_axis)
            qb = b
        else:
            qb = QuantizedTensor.quantize(b, _get_fp8_dtype(config.format, True), g, axis=b_row_axis,
                                          block_size=config.block_size)
        out = grouped_gemm_fp8_impl(qa.qdata, qb.qdata, qa.scale_inv, qb.scale_inv, group_lens, group_offs, False,
                                    trans_b, out_dtype, g.value, num_cu)
        qa_t = a_t if a_t is not None else QuantizedTensor.quantize(
            qa.dequantize(), qa.real_dtype, g, axis=-2, block_size=config.block_size, group_lens=group_lens)
        qb_t = b_t if b_t is not None else QuantizedTensor.quantize(
            qb.dequantize(), qb.real_dtype, g, axis=b_col_axis, block_size=config.block_size)
        ctx.save_for_backward(qa_t.qdata, qb_t.qdata, qa_t.scale_inv, qb_t.scale_inv, group_lens, group_offs)
        ctx.trans_b, ctx.config, ctx.out_dtype, ctx.num_cu = trans_b, config, out_dtype, num_cu
        return out

    @staticmethod
    def backward(ctx, grad_out):
        g = ScalingGranularity.ROWWISE
        a_col, b_col, a_s_col, b_s_col, group_lens, group_offs = ctx.saved_tensors
        gdt = _get_fp8_dtype(ctx.config.format, False)
        grad_out = grad_out.contiguous()
        qg = QuantizedTensor.quantize(grad_out, gdt, g, axis=-1, block_size=ctx.config.block_size,
                                      group_lens=group_lens)
        grad_a = grouped_gemm_fp8_impl(qg.qdata, b_col, qg.scale_inv, b_s_col, group_lens, group_offs, False,
                                       not ctx.trans_b, ctx.out_dtype, g.value, ctx.num_cu)
        qg_t = QuantizedTensor.quantize(grad_out, gdt, g, axis=-2, block_size=ctx.config.block_size,
                                        group_lens=group_lens)
        grad_b = grouped_gemm_fp8_variable_k_impl(a_col, qg_t.qdata, a_s_col, qg_t.scale_inv, group_lens,
                                                  group_offs, True, False, ctx.trans_b, ctx.out_dtype, g.value,
                                                  ctx.num_cu)
        return grad_a, grad_b, None, None, None, None, None, None, None, None


class FP8GroupedGemmTensorFunc(torch.autograd.Function):
    """TENSORWISE (grouped_gemm_fp8.py:382-567)."""

    @staticmethod
    def forward(ctx, a, b, a_t, b_t, group_lens, group_offs, trans_b, out_dtype, config, num_cu):
        g = ScalingGranularity.TENSORWISE
        nt_bwd = trans_b
        if isinstance(a, QuantizedTensor):
            check_quantized_tensor(a, config)
            qa = a
        else:
            qa = QuantizedTensor.quantize(a, _get_fp8_dtype(config.format, True), g, axis=-1, group_lens=group_lens)
        if isinstance(b, QuantizedTensor):
            check_quantized_tensor(b, config)
            qb = b
        else:
            qb = QuantizedTensor.quantize(b, _get_fp8_dtype(config.format, True), g, axis=-1)
        out = grouped_gemm_fp8_impl(qa.qdata, qb.qdata, qa.scale_inv, qb.scale_inv, group_lens, group_offs, False,
                                    trans_b, out_dtype, g.value, num_cu)
        if nt_bwd:
            qb_t = b_t if isinstance(b_t, QuantizedTensor) else qb.transpose(-1, -2)
            ctx.save_for_backward(qa.qdata, qb_t.qdata, qa.scale_inv, qb_t.scale_inv, group_lens, group_offs)
        else:
            ctx.save_for_backward(qa.qdata, qb.qdata, qa.scale_inv, qb.scale_inv, group_lens, group_offs)
        ctx.trans_b, ctx.nt_bwd, ctx.config, ctx.out_dtype, ctx.num_cu = trans_b, nt_bwd, config, out_dtype, num_cu
        return out

    @staticmethod
    def backward(ctx, grad_out):
        g = ScalingGranularity.TENSORWISE
        a8, b8, sa, sb, group_lens, group_offs = ctx.saved_tensors
        gdt = _get_fp8_dtype(ctx.config.format, False)
        qg = QuantizedTensor.quantize(grad_out.contiguous(), gdt, g, axis=-1, group_lens=group_lens)
        trans = True if ctx.nt_bwd else (not ctx.trans_b)
        grad_a = grouped_gemm_fp8_impl(qg.qdata, b8, qg.scale_inv, sb, group_lens, group_offs, False, trans,
                                       ctx.out_dtype, g.value, ctx.num_cu)
        grad_b = grouped_gemm_fp8_variable_k_impl(a8, qg.qdata, sa, qg.scale_inv, group_lens, group_offs, True,
                                                  False, ctx.trans_b, ctx.out_dtype, g.value, ctx.num_cu)
        return grad_a, grad_b, None, None, None, None, None, None, None, None


class FP8GroupedGemmMXFunc(torch.autograd.Function):
    """MX_BLOCKWISE (grouped_gemm_fp8.py:593-795), NT only: activations in the
    32-row-padded grouped layout (1 x 32 exponents), weights with 32 x 32
    exponents; the forward and dgrad read padded rows and write the packed rows
    given by group_offs; wgrad is variable-K over the 128-padded colwise copies."""

    @staticmethod
    def forward(ctx, a, b, group_lens, group_offs, trans_b, out_dtype, config, num_cu):
        assert config.granularity == ScalingGranularity.MX_BLOCKWISE
        assert a.ndim == 2 and b.ndim == 3
        assert trans_b, "MXFP8 grouped GEMM only supports trans_b=True (NT layout)."
        if isinstance(a, QuantizedTensor):
            a = a.dequantize()
        if isinstance(b, QuantizedTensor):
            b = b.dequantize()
        a_dtype = _get_fp8_dtype(config.format, True)
        bs = config.block_size
        a_row, a_srow, a_col, a_scol, _, offs_pad_row, _, _ = grouped_quantize_mxfp8_impl(
            a.contiguous(), a_dtype, None, bs, group_lens, group_offs, True)
        b_row, b_srow, b_col, b_scol = quantize_mxfp8_impl(
            b.contiguous(), a_dtype, None, bs, with_trans=True, scaling_recipe=ScalingRecipe(use_2d_block=True),
            scaling_recipe_for_trans=ScalingRecipe(use_2d_block=True))
        total_m = a.size(0)
        out = grouped_gemm_fp8_impl(a_row, b_row, a_srow, b_srow, group_lens, offs_pad_row, False, True, out_dtype,
                                    ScalingGranularity.MX_BLOCKWISE.value, num_cu, group_offs_out=group_offs)
        out = out[:total_m]
        ctx.save_for_backward(a_col, a_scol, b_col, b_scol, group_lens, group_offs)
        ctx.config, ctx.out_dtype, ctx.num_cu, ctx.total_m = config, out_dtype, num_cu, total_m
        return out

    @staticmethod
    def backward(ctx, grad_out):
        a_col, a_scol, b_col, b_scol, group_lens, group_offs = ctx.saved_tensors
        g_dtype = _get_fp8_dtype(ctx.config.format, False)
        mx = ScalingGranularity.MX_BLOCKWISE.value
        g_row, g_srow, g_col, g_scol, _, offs_pad_row, lens_pad_col, offs_pad_col = grouped_quantize_mxfp8_impl(
            grad_out.contiguous(), g_dtype, None, ctx.config.block_size, group_lens, group_offs, True)
        grad_a = grouped_gemm_fp8_impl(g_row, b_col, g_srow, b_scol, group_lens, offs_pad_row, False, True,
                                       ctx.out_dtype, mx, ctx.num_cu, group_offs_out=group_offs)[: ctx.total_m]
        grad_b = grouped_gemm_fp8_variable_k_impl(g_col, a_col, g_scol, a_scol, lens_pad_col, offs_pad_col, False,
                                                  False, False, ctx.out_dtype, mx, ctx.num_cu)
        return grad_a, grad_b, None, None, None, None, None, None


@torch._dynamo.disable(recursive=True)
def grouped_gemm_fp8(
    a: Union[torch.Tensor, QuantizedTensor, QuantizedTensorPair],
    b: Union[torch.Tensor, QuantizedTensor, QuantizedTensorPair],
    group_lens: torch.Tensor,
    group_offs: Optional[torch.Tensor] = None,
    trans_b: bool = True,
    out_dtype: Optional[torch.dtype] = None,
    config: Optional[Float8QuantConfig] = None,
    num_cu: int | None = None,
) -> torch.Tensor:
    """out[offs[g]:offs[g+1]] = a[offs[g]:offs[g+1]] @ op(b[g]) with FP8 quantization.

    a [M_total, K]; b [G, N, K] (trans_b) or [G, K, N]; group_lens [G] int64 on
    the device.  config defaults to TENSORWISE E4M3.
    """
    if config is None:
        config = Float8QuantConfig()
    if group_offs is None:
        group_offs = group_offs_from_lens(group_lens)
    a_data, a_data_t = (a.data, a.data_t) if isinstance(a, QuantizedTensorPair) else (a, None)
    b_data, b_data_t = (b.data, b.data_t) if isinstance(b, QuantizedTensorPair) else (b, None)
    if out_dtype is None:
        out_dtype = torch.promote_types(a_data.dtype, b_data.dtype)
    if config.granularity == ScalingGranularity.TENSORWISE:
        return FP8GroupedGemmTensorFunc.apply(a_data, b_data, a_data_t, b_data_t, group_lens, group_offs, trans_b,
                                              out_dtype, config, num_cu)
    elif config.granularity == ScalingGranularity.ROWWISE:
        return FP8GroupedGemmRowFunc.apply(a_data, b_data, a_data_t, b_data_t, group_lens, group_offs, trans_b,
                                           out_dtype, config, num_cu)
    elif config.granularity == ScalingGranularity.BLOCKWISE:
        return FP8GroupedGemmBlockFunc.apply(a, b, group_lens, group_offs, trans_b, out_dtype, config, num_cu)
    elif config.granularity == ScalingGranularity.MX_BLOCKWISE:
        return FP8GroupedGemmMXFunc.apply(a_data, b_data, group_lens, group_offs, trans_b, out_dtype, config, num_cu)
    raise ValueError(f"Unsupported FP8 ScalingGranularity: {config.granularity}")
