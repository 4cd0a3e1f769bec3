"""MoE token permute / unpermute with autograd.

Public API (``moe_permute`` / ``moe_unpermute``: names, keyword arguments and
return tuples) follows the reference's primus_turbo/pytorch/ops/moe/
moe_permute.py:353-420.

``moe_permute`` packs the dispatched tokens expert-major (each expert's rows
contiguous, optionally padded per expert to ``pad_multiple`` with zero rows):
the layout and ``tokens_per_expert`` that ``grouped_gemm_fp8`` consumes as
``group_lens``.  ``moe_unpermute`` sums each token's expert rows back (fp32
accumulation, row_id_map order).

Design: a ``_Routing`` record holds everything both directions need (the
row_id_map, the device-side dispatched count and the layout parameters).  Two
movers, ``_expert_major`` (scatter) and ``_token_major`` (gather-reduce),
implement the two directions once; each autograd Function runs one of them
forward and the other backward.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from primus_turbo.pytorch.kernels.moe.moe_permute_impl import (
    permute_impl,
    permute_preprocessing_impl,
    unpermute_impl,
)

__all__ = ["moe_permute", "moe_unpermute"]


@dataclass
class _Routing:
    row_id_map: torch.Tensor  # [T + pad_multiple, 2E + 1] int32
    num_dispatched: torch.Tensor  # [1] int32, device
    num_experts: int
    pad_multiple: int
    probs_stride: int  # > 0: probs rows are top-k aligned with this width; 0: num_experts wide

    @property
    def probs_width(self) -> int:
        return self.probs_stride if self.probs_stride > 0 else self.num_experts


def _route(expert_map, num_tokens, num_experts, num_topk, pad_multiple, cap, probs_stride, device):
    """Slot assignment for every (token, local expert) pair.  Returns the
    routing record plus tokens_per_expert and the overflow flag."""
    if num_tokens == 0:
        # nothing to assign: an all-zero map of padding rows only
        rim = torch.zeros((pad_multiple, 2 * num_experts + 1), dtype=torch.int32, device=device)
        nd = torch.zeros((1,), dtype=torch.int32, device=device)
        tpe = torch.zeros((num_experts,), dtype=torch.int64, device=device)
        ovf = torch.zeros((1,), dtype=torch.int32, device=device)
    else:
        rim, tpe, ovf, nd = permute_preprocessing_impl(expert_map, num_experts, num_topk, pad_multiple, cap,
                                                       probs_stride)
    return _Routing(rim, nd, num_experts, pad_multiple, probs_stride), tpe, ovf


def _expert_major(r: _Routing, src: torch.Tensor, n_rows: int, probs: Optional[torch.Tensor] = None,
                  scales: Optional[torch.Tensor] = None, scales_per_token: int = 0, fp8: bool = False):
    """Scatter token rows (and their probs / fp8 scaling factors) into
    ``n_rows`` expert-major rows; padding rows come out zero."""
    dev, H = src.device, int(src.shape[-1])
    rows = torch.empty((n_rows, H), dtype=src.dtype, device=dev)
    out_probs = torch.empty((n_rows,), dtype=probs.dtype, device=dev) if probs is not None else None
    out_scales = (torch.empty((n_rows, scales_per_token), dtype=scales.dtype, device=dev)
                  if scales is not None else None)
    if n_rows > 0 and src.shape[0] > 0:
        permute_impl(src.contiguous(), rows, scales, out_scales,
                     probs.contiguous() if probs is not None else None, out_probs, r.row_id_map,
                     r.num_dispatched, r.pad_multiple, r.num_experts, H, scales_per_token, fp8,
                     probs is not None, n_rows, r.probs_stride)
    return rows, out_probs, out_scales


def _token_major(r: _Routing, src: torch.Tensor, n_tokens: int, probs: Optional[torch.Tensor] = None):
    """Gather-reduce expert-major rows (and per-row probs) back into
    ``n_tokens`` token rows.  Every token row is written: tokens with no
    routed row, and rows past the dispatched count, come out zero."""
    dev, H = src.device, int(src.shape[-1])
    tokens = torch.empty((n_tokens, H), dtype=src.dtype, device=dev)
    out_probs = (torch.empty((n_tokens, r.probs_width), dtype=probs.dtype, device=dev)
                 if probs is not None else None)
    if n_tokens > 0:
        unpermute_impl(src.contiguous(), tokens, probs.contiguous() if probs is not None else None, out_probs,
                       r.row_id_map, r.num_dispatched, r.num_experts, H, probs is not None, r.probs_stride)
    return tokens, out_probs


def _save(ctx, r: _Routing) -> None:
    ctx.save_for_backward(r.row_id_map, r.num_dispatched)
    ctx.layout = (r.num_experts, r.pad_multiple, r.probs_stride)


def _load(ctx) -> _Routing:
    rim, nd = ctx.saved_tensors
    return _Routing(rim, nd, *ctx.layout)


class _Permute(torch.autograd.Function):
    """Forward scatters the tokens expert-major; backward gathers the row
    gradients (and the probs gradient) back per token."""

    @staticmethod
    def forward(ctx, tokens, expert_map, num_local_experts, num_topk, pad_multiple, num_permuted_tokens,
                scaling_factor, probs, scales_per_token, use_fp8, probs_topk_stride):
        if use_fp8 and scaling_factor is not None:
            assert scales_per_token > 0, "fp8 scaling factors need scales_per_token > 0"
        assert not (use_fp8 and probs is not None and tokens.requires_grad), (
            "moe_permute: fp8 tokens with probs have no backward"
        )
        T = int(tokens.shape[0])
        stride = int(probs_topk_stride) if probs is not None else 0
        r, tpe, ovf = _route(expert_map, T, num_local_experts, num_topk, pad_multiple, num_permuted_tokens,
                             stride, tokens.device)
        # the row count is a host value: the cap, or the padded total (one host
        # read); no tokens, no rows
        if T == 0:
            n_rows = 0
        elif num_permuted_tokens > 0:
            n_rows = int(num_permuted_tokens)
        else:
            n_rows = int(tpe.sum().item())
        sf = scaling_factor if use_fp8 else None
        rows, out_probs, out_sf = _expert_major(r, tokens, n_rows, probs, sf, scales_per_token, use_fp8)
        _save(ctx, r)
        ctx.n_tokens, ctx.fp8, ctx.has_probs = T, use_fp8, probs is not None
        return rows, r.row_id_map, tpe, ovf, r.num_dispatched, out_sf, out_probs

    @staticmethod
    def backward(ctx, g_rows, _g_map, _g_tpe, _g_ovf, _g_nd, _g_sf, g_probs):
        assert not ctx.fp8, "moe_permute: fp8 tokens have no backward"
        g_probs = g_probs if ctx.has_probs else None
        g_tokens, g_in_probs = _token_major(_load(ctx), g_rows, ctx.n_tokens, g_probs)
        return g_tokens, None, None, None, None, None, None, g_in_probs, None, None, None


class _Unpermute(torch.autograd.Function):
    """Forward gathers expert-major rows back per token; backward scatters
    the token gradients (and the probs gradient) expert-major again."""

    @staticmethod
    def forward(ctx, permuted_tokens, row_id_map, num_dispatched, restore_shape, num_local_experts,
                permuted_probs, probs_topk_stride, pad_multiple):
        r = _Routing(row_id_map, num_dispatched, num_local_experts, pad_multiple, int(probs_topk_stride))
        tokens, probs = _token_major(r, permuted_tokens, int(restore_shape[0]), permuted_probs)
        _save(ctx, r)
        ctx.n_rows, ctx.has_probs = int(permuted_tokens.shape[0]), permuted_probs is not None
        return tokens, probs

    @staticmethod
    def backward(ctx, g_tokens, g_probs):
        g_probs = g_probs if ctx.has_probs else None
        g_rows, g_row_probs, _ = _expert_major(_load(ctx), g_tokens, ctx.n_rows, g_probs)
        return g_rows, None, None, None, None, g_row_probs, None, None


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
    """Fused slot assignment + permute (reference moe_permute.py:353-393).

    ``expert_map`` is a bool routing map [T, num_local_experts] or top-k
    expert indices [T, num_topk] (int32/int64; entries outside
    [0, num_local_experts) are ignored).  ``probs_layout`` "topk" reads probs
    as [T, num_topk] aligned with the index map, "routing_map" as
    [T, num_local_experts].  Returns (permuted_tokens, row_id_map,
    tokens_per_expert, overflow_flag, num_dispatched_tokens,
    permuted_scaling_factor, permuted_probs); pass ``num_dispatched_tokens``
    straight to ``moe_unpermute``.  A bad ``probs_layout`` raises ValueError."""
    if probs_layout == "topk":
        if num_topk <= 0:
            raise ValueError(f"moe_permute: probs_layout 'topk' needs num_topk > 0 (got {num_topk})")
        stride = num_topk
    elif probs_layout == "routing_map":
        stride = 0
    else:
        raise ValueError(f"moe_permute: unknown probs_layout {probs_layout!r} (expected 'topk' or 'routing_map')")
    return _Permute.apply(tokens, expert_map, num_local_experts, num_topk, pad_multiple, num_permuted_tokens,
                          scaling_factor, probs, scales_per_token, use_fp8, stride)


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
    """Unpermute back into ``restore_shape`` (the permuted tokens' original
    [T, hidden] shape) (reference moe_permute.py:396-420).
    ``probs_topk_stride`` selects the width of the returned probs (0:
    [T, num_local_experts], > 0: [T, stride]); ``pad_multiple`` must equal the
    forward's (the backward scatter lays out the padding rows with it).  Every
    output row is written, zero for tokens with no routed row."""
    return _Unpermute.apply(permuted_tokens, row_id_map, num_dispatched_tokens_tensor, restore_shape,
                            num_local_experts, permuted_probs, probs_topk_stride, pad_multiple)
