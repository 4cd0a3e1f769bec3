"""MoE token permute / unpermute with autograd (same API as the reference's
primus_turbo/pytorch/ops/moe/moe_permute.py:17-420).

``moe_permute`` packs the dispatched tokens expert-major (each expert's rows
contiguous, optionally padded per expert to ``pad_multiple`` with zero rows):
the layout and ``tokens_per_expert`` that ``grouped_gemm_fp8`` consumes as
``group_lens``.  ``moe_unpermute`` sums each token's expert rows back (fp32
accumulation).  Each is the other's backward.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from primus_turbo.pytorch.kernels.moe.moe_permute_impl import (
    permute_impl,
    permute_preprocessing_impl,
    unpermute_impl,
)

__all__ = ["moe_permute", "moe_unpermute"]


class _MoEPermute(torch.autograd.Function):
    """Forward: preprocessing + scatter.  Backward: gather-reduce of the
    gradient (+ probs gradient) (moe_permute.py:17-218)."""

    @staticmethod
    def forward(ctx, tokens, expert_map, num_local_experts, num_topk, pad_multiple=0, num_permuted_tokens=-1,
                scaling_factor=None, probs=None, scales_per_token=0, use_fp8=False, probs_topk_stride=0):
        dev = tokens.device
        H = int(tokens.shape[-1])
        T = int(tokens.shape[0])
        probs_topk_stride = int(probs_topk_stride) if probs is not None else 0
        row_width = probs_topk_stride if probs_topk_stride > 0 else num_local_experts
        ctx.num_dispatched, ctx.hidden_size, ctx.num_local_experts = T, H, num_local_experts
        ctx.use_fp8, ctx.with_probs = use_fp8, probs is not None
        ctx.probs_dtype = probs.dtype if probs is not None else None
        ctx.probs_topk_stride, ctx.probs_row_width = probs_topk_stride, row_width

        if use_fp8 and scaling_factor is not None:
            assert scales_per_token > 0, "scales_per_token must be > 0 when use_fp8=True"
        assert not (use_fp8 and probs is not None and tokens.requires_grad), (
            "moe_permute: FP8 + probs backward is unsupported"
        )

        if T == 0:
            row_id_map = torch.zeros((pad_multiple, 2 * num_local_experts + 1), dtype=torch.int32, device=dev)
            tpe = torch.zeros((num_local_experts,), dtype=torch.int64, device=dev)
            overflow = torch.zeros((1,), dtype=torch.int32, device=dev)
            ndisp = torch.zeros((1,), dtype=torch.int32, device=dev)
            out = tokens.new_empty((0, H))
            osf = (scaling_factor.new_empty((0, scales_per_token))
                   if use_fp8 and scaling_factor is not None else None)
            opr = probs.new_zeros((0,)) if probs is not None else None
            ctx.save_for_backward(row_id_map, ndisp)
            return out, row_id_map, tpe, overflow, ndisp, osf, opr

        row_id_map, tpe, overflow, ndisp = permute_preprocessing_impl(
            expert_map, num_local_experts, num_topk, pad_multiple, num_permuted_tokens, probs_topk_stride
        )
        # the output row count is a host value: the cap, or the padded total (one host sync)
        P = int(num_permuted_tokens) if num_permuted_tokens > 0 else int(tpe.sum().item())
        out = torch.empty((P, H), dtype=tokens.dtype, device=dev)
        osf = (torch.empty((P, scales_per_token), dtype=scaling_factor.dtype, device=dev)
               if use_fp8 and scaling_factor is not None else None)
        opr = torch.empty((P,), dtype=probs.dtype, device=dev) if probs is not None else None
        permute_impl(tokens.contiguous(), out, scaling_factor, osf, probs, opr, row_id_map, ndisp, pad_multiple,
                     num_local_experts, H, scales_per_token, use_fp8, probs is not None, P, probs_topk_stride)
        ctx.save_for_backward(row_id_map, ndisp)
        return out, row_id_map, tpe, overflow, ndisp, osf, opr

    @staticmethod
    def backward(ctx, g_out, g_rim, g_tpe, g_ovf, g_nd, g_sf, g_probs):
        assert not ctx.use_fp8, "_MoEPermute.backward: FP8 backward not supported"
        row_id_map, ndisp = ctx.saved_tensors
        g_out = g_out.contiguous()
        dev = g_out.device
        g_tokens = torch.empty((ctx.num_dispatched, ctx.hidden_size), dtype=g_out.dtype, device=dev)
        if ctx.with_probs and g_probs is not None:
            g_probs = g_probs.contiguous()
            g_in_probs = torch.empty((ctx.num_dispatched, ctx.probs_row_width), dtype=ctx.probs_dtype, device=dev)
        else:
            g_probs, g_in_probs = None, None
        if ctx.num_dispatched > 0:
            unpermute_impl(g_out, g_tokens, g_probs, g_in_probs, row_id_map, ndisp, ctx.num_local_experts,
                           ctx.hidden_size, g_in_probs is not None, ctx.probs_topk_stride)
        return g_tokens, None, None, None, None, None, None, g_in_probs, None, None, None


class _MoEUnpermute(torch.autograd.Function):
    """Forward: gather-reduce.  Backward: scatter of the gradient (+ probs
    gradient) (moe_permute.py:221-350)."""

    @staticmethod
    def forward(ctx, permuted_tokens, row_id_map, ndisp, restore_shape, num_local_experts, permuted_probs,
                probs_topk_stride, pad_multiple):
        dev = permuted_tokens.device
        P = int(permuted_tokens.shape[0])
        T, H = int(restore_shape[0]), int(restore_shape[1])
        row_width = probs_topk_stride if probs_topk_stride > 0 else num_local_experts
        ctx.num_permuted, ctx.hidden_size, ctx.num_local_experts = P, H, num_local_experts
        ctx.with_probs = permuted_probs is not None
        ctx.permuted_probs_dtype = permuted_probs.dtype if permuted_probs is not None else None
        ctx.probs_topk_stride, ctx.probs_row_width, ctx.pad_multiple = probs_topk_stride, row_width, pad_multiple
        out = torch.empty((T, H), dtype=permuted_tokens.dtype, device=dev)
        oprobs = (torch.empty((T, row_width), dtype=permuted_probs.dtype, device=dev)
                  if permuted_probs is not None else None)
        ctx.save_for_backward(row_id_map, ndisp)
        if P == 0 or T == 0:
            return out, oprobs
        unpermute_impl(permuted_tokens.contiguous(), out,
                       permuted_probs.contiguous() if permuted_probs is not None else None, oprobs, row_id_map,
                       ndisp, num_local_experts, H, permuted_probs is not None, probs_topk_stride)
        return out, oprobs

    @staticmethod
    def backward(ctx, g_out, g_oprobs):
        row_id_map, ndisp = ctx.saved_tensors
        g_out = g_out.contiguous()
        dev = g_out.device
        # padding rows of the gradient are written as zeros by the scatter itself
        g_perm = torch.empty((ctx.num_permuted, ctx.hidden_size), dtype=g_out.dtype, device=dev)
        if ctx.with_probs and g_oprobs is not None:
            g_oprobs = g_oprobs.contiguous()
            g_pprobs = torch.empty((ctx.num_permuted,), dtype=ctx.permuted_probs_dtype, device=dev)
        else:
            g_oprobs, g_pprobs = None, None
        if ctx.num_permuted > 0 and g_out.shape[0] > 0:
            permute_impl(g_out, g_perm, None, None, g_oprobs, g_pprobs, row_id_map, ndisp, ctx.pad_multiple,
                         ctx.num_local_experts, ctx.hidden_size, 0, False, g_pprobs is not None, ctx.num_permuted,
                         ctx.probs_topk_stride)
        return g_perm, None, None, None, None, g_pprobs, None, None


def moe_permute(
    tokens: torch.Tensor,
    expert_map: torch.Tensor,
    *,
    num_local_experts: int,
    num_topk: int = 0,
    pad_multiple: int = 0,
    num_permuted_tokens: int = -1,
    scaling_factor: Optional[torch.Tensor] = None,
    probs: Optional[torch.Tensor] = None,
    probs_layout: str = "topk",
    scales_per_token: int = 0,
    use_fp8: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor],
           Optional[torch.Tensor]]:
    """Fused preprocessing + permute (moe_permute.py:353-393).

    ``expert_map`` is a bool routing map [T, num_local_experts] or top-k
    expert indices [T, num_topk] (int32/int64; entries outside
    [0, num_local_experts) are ignored).  Returns (permuted_tokens,
    row_id_map, tokens_per_expert, overflow_flag, num_dispatched_tokens,
    permuted_scaling_factor, permuted_probs); pass ``num_dispatched_tokens``
    straight to ``moe_unpermute``."""
    if probs_layout not in ("routing_map", "topk"):
        raise ValueError(f"moe_permute: probs_layout must be 'routing_map' or 'topk', got {probs_layout!r}")
    if probs_layout == "topk" and num_topk <= 0:
        raise ValueError("moe_permute: probs_layout='topk' requires num_topk > 0")
    probs_topk_stride = num_topk if probs_layout == "topk" else 0
    return _MoEPermute.apply(tokens, expert_map, num_local_experts, num_topk, pad_multiple, num_permuted_tokens,
                             scaling_factor, probs, scales_per_token, use_fp8, probs_topk_stride)


def moe_unpermute(
    permuted_tokens: torch.Tensor,
    row_id_map: torch.Tensor,
    num_dispatched_tokens_tensor: torch.Tensor,
    *,
    restore_shape: torch.Size,
    num_local_experts: int,
    permuted_probs: Optional[torch.Tensor] = None,
    probs_topk_stride: int = 0,
    pad_multiple: int = 0,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Unpermute back into ``restore_shape`` (= the permuted input's shape)
    (moe_permute.py:396-420).  ``probs_topk_stride`` selects the width of
    ``unpermuted_probs`` (0: [T, num_local_experts], > 0: [T, stride]) and
    ``pad_multiple`` must equal the forward's (it is used by the backward)."""
    return _MoEUnpermute.apply(permuted_tokens, row_id_map, num_dispatched_tokens_tensor, restore_shape,
                               num_local_experts, permuted_probs, probs_topk_stride, pad_multiple)
