"""Host side of the MoE permutation kernels: argument checks, output
allocation and the calls into libprimus_turbo_amd.so.

The three functions mirror the reference's native ops
``permute_preprocessing`` / ``permute`` / ``unpermute``
(csrc/pytorch/moe_permute/moe_permute.cpp:39-276): same arguments, same output
shapes and dtypes, RuntimeError on a failed check (the reference's
PRIMUS_TURBO_CHECK).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from primus_turbo.pytorch import _C


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


_MAP_KIND = {torch.bool: _C.MOE_MAP_BOOL, torch.int32: _C.MOE_MAP_I32, torch.int64: _C.MOE_MAP_I64}


def permute_preprocessing_impl(
    expert_map: torch.Tensor,
    num_local_experts: int,
    num_topk: int,
    pad_multiple: int,
    num_permuted_tokens: int,
    probs_topk_stride: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(row_id_map [T + pad_multiple, 2E + 1] int32, tokens_per_expert [E] int64,
    overflow_flag [1] int32, num_dispatched_tokens [1] int32)
    (moe_permute.cpp:39-97)."""
    _check(expert_map.is_cuda, "routing_map must be CUDA")
    _check(expert_map.dtype in _MAP_KIND, "expert_map must be bool or int or int64")
    _check(expert_map.dim() == 2, "expert_map must be 2D")
    _check(expert_map.is_contiguous(), "expert_map must be contiguous")
    if expert_map.dtype == torch.bool:
        _check(expert_map.shape[1] == num_local_experts,
               "bool expert_map second dimension must equal num_local_experts")
    else:
        _check(expert_map.shape[1] == num_topk, "index expert_map second dimension must equal num_topk")
    T = expert_map.shape[0]
    E = int(num_local_experts)
    dev = expert_map.device
    row_id_map = torch.empty((T + pad_multiple, 2 * E + 1), dtype=torch.int32, device=dev)
    tokens_per_expert = torch.empty((E,), dtype=torch.int64, device=dev)
    overflow_flag = torch.empty((1,), dtype=torch.int32, device=dev)
    num_dispatched = torch.empty((1,), dtype=torch.int32, device=dev)
    ws = _C.workspace(_C.query("pta_moe_permute_preprocess_workspace_size", T, E), dev)
    _C.call(
        "pta_moe_permute_preprocess", _C.ptr(expert_map), _MAP_KIND[expert_map.dtype], T, E, int(num_topk),
        int(pad_multiple), int(num_permuted_tokens), int(probs_topk_stride), _C.ptr(row_id_map),
        _C.ptr(tokens_per_expert), _C.ptr(overflow_flag), _C.ptr(num_dispatched), _C.ptr(ws),
        0 if ws is None else ws.numel(), _C.stream(dev),
    )
    return row_id_map, tokens_per_expert, overflow_flag, num_dispatched


def _f32_opt(t: Optional[torch.Tensor], name: str) -> None:
    if t is not None:
        _check(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32,
               f"permute: {name} must be contiguous float32 CUDA tensor")


def permute_impl(
    tokens: torch.Tensor,
    output_tokens: torch.Tensor,
    scaling_factor: Optional[torch.Tensor],
    output_scaling_factor: Optional[torch.Tensor],
    probs: Optional[torch.Tensor],
    output_probs: Optional[torch.Tensor],
    row_id_map: torch.Tensor,
    num_dispatched_tokens: torch.Tensor,
    pad_multiple: int,
    num_local_experts: int,
    hidden_size: int,
    scales_per_token: int,
    use_fp8: bool,
    with_probs: bool,
    num_permuted_tokens: int,
    probs_stride: int,
) -> None:
    """Scatter tokens into output_tokens [num_permuted_tokens, hidden_size]
    (moe_permute.cpp:108-204)."""
    _check(num_permuted_tokens >= 0, "num_permuted_token must be >= 0")
    if num_permuted_tokens == 0:
        return
    _check(probs_stride >= 0, "probs_stride must be >= 0")
    _check(tokens.is_cuda and output_tokens.is_cuda, "permute: tokens / output_tokens must be CUDA")
    _check(tokens.is_contiguous() and output_tokens.is_contiguous(),
           "permute: tokens / output_tokens must be contiguous")
    _check(tokens.dim() == 2 and output_tokens.dim() == 2, "permute: tokens / output_tokens must be 2D")
    _check(tokens.shape[1] == hidden_size, "permute: tokens.shape[1] must equal hidden_size")
    _check(tuple(output_tokens.shape) == (num_permuted_tokens, hidden_size),
           "permute: output_tokens shape must be [num_permuted_token, hidden_size]")
    _check(row_id_map.is_cuda and row_id_map.dtype == torch.int32 and row_id_map.is_contiguous(),
           "permute: row_id_map must be contiguous int32 CUDA tensor")
    _check(num_dispatched_tokens.is_cuda and num_dispatched_tokens.dtype == torch.int32
           and num_dispatched_tokens.is_contiguous() and num_dispatched_tokens.numel() == 1,
           "permute: num_dispatched_token_tensor must be contiguous int32 CUDA tensor with exactly one element")
    esz = 1 if use_fp8 else 2
    _check(tokens.element_size() == esz and output_tokens.element_size() == esz,
           "permute (fp8): tokens / output_tokens must have 1-byte elements" if use_fp8
           else "permute (16-bit): tokens / output_tokens must have 2-byte elements")
    _check(hidden_size % (16 // esz) == 0,
           f"permute ({'fp8' if use_fp8 else '16-bit'}): hidden_size must be a multiple of {16 // esz}")
    _f32_opt(scaling_factor, "scaling_factor")
    _f32_opt(output_scaling_factor, "output_scaling_factor")
    _f32_opt(probs, "probs")
    _f32_opt(output_probs, "output_probs")
    eff = probs_stride if probs_stride > 0 else num_local_experts
    if probs is not None and with_probs:
        _check(probs.dim() == 2, "permute: probs must be 2D ([T, probs_stride])")
        _check(probs.shape[1] == eff,
               "permute: probs.size(1) must equal probs_stride (or num_local_experts when probs_stride == 0)")
    # the reference ignores scaling factors on the 16-bit path (moe_permute.cpp:194-203)
    sf = scaling_factor if use_fp8 and output_scaling_factor is not None else None
    osf = output_scaling_factor if sf is not None else None
    pr = probs if with_probs and output_probs is not None else None
    opr = output_probs if pr is not None else None
    if sf is not None:
        _check(sf.numel() == tokens.shape[0] * scales_per_token and osf.numel() >= num_permuted_tokens * scales_per_token,
               "permute: scaling factor shapes do not match scales_per_token")
    if pr is not None:
        _check(opr.numel() >= num_permuted_tokens, "permute: output_probs too small")
    _C.call(
        "pta_moe_permute", _C.ptr(tokens), tokens.shape[0], esz, int(hidden_size), _C.ptr(output_tokens),
        int(num_permuted_tokens), _C.ptr(row_id_map), row_id_map.shape[0], _C.ptr(num_dispatched_tokens),
        int(pad_multiple), int(num_local_experts), _C.ptr(sf), _C.ptr(osf), int(scales_per_token) if sf is not None else 0,
        _C.ptr(pr), _C.ptr(opr), int(probs_stride), _C.stream(tokens.device),
    )


def unpermute_impl(
    permuted_tokens: torch.Tensor,
    output_tokens: torch.Tensor,
    permuted_probs: Optional[torch.Tensor],
    output_probs: Optional[torch.Tensor],
    row_id_map: torch.Tensor,
    num_dispatched_tokens: torch.Tensor,
    num_local_experts: int,
    hidden_size: int,
    with_probs: bool,
    probs_stride: int,
) -> None:
    """Reduce permuted bf16/fp16 rows back into output_tokens [T, hidden_size]
    (moe_permute.cpp:214-276)."""
    _check(probs_stride >= 0, "probs_stride must be >= 0")
    _check(permuted_tokens.is_cuda and output_tokens.is_cuda, "unpermute: tensors must be CUDA")
    _check(permuted_tokens.dtype in (torch.bfloat16, torch.float16),
           "unpermute: permuted_tokens must be bfloat16 or float16")
    _check(output_tokens.dtype == permuted_tokens.dtype, "unpermute: output_tokens dtype must match permuted_tokens")
    _check(hidden_size % 8 == 0, "unpermute: hidden_size must be a multiple of 8")
    _check(row_id_map.is_cuda and row_id_map.dtype == torch.int32,
           "unpermute: row_id_map must be int32 CUDA tensor")
    _check(num_dispatched_tokens.is_cuda and num_dispatched_tokens.dtype == torch.int32,
           "unpermute_launcher: num_dispatched_tokens_tensor must be int32 CUDA tensor")
    _check(permuted_tokens.is_contiguous() and output_tokens.is_contiguous() and row_id_map.is_contiguous(),
           "unpermute: tensors must be contiguous")
    _check(permuted_tokens.dim() == 2 and permuted_tokens.shape[1] == hidden_size
           and output_tokens.dim() == 2 and output_tokens.shape[1] == hidden_size,
           "unpermute: token tensors must be [rows, hidden_size]")
    eff = probs_stride if probs_stride > 0 else num_local_experts
    if with_probs:
        _check(permuted_probs is not None, "unpermute_launcher: with_probs but permuted_probs is empty")
        _check(permuted_probs.dtype == torch.float32, "unpermute_launcher: permuted_probs must be float32")
        _check(output_probs is not None, "unpermute_launcher: with_probs but output_probs is empty")
        _check(output_probs.dtype == torch.float32, "unpermute_launcher: output_probs must be float32")
        _check(output_probs.dim() == 2, "unpermute: output_probs must be 2D ([T, probs_stride])")
        _check(output_probs.shape[1] == eff,
               "unpermute: output_probs.size(1) must equal probs_stride (or num_local_experts when probs_stride == 0)")
        _check(permuted_probs.is_contiguous() and output_probs.is_contiguous()
               and permuted_probs.numel() >= permuted_tokens.shape[0],
               "unpermute: probs must be contiguous with one value per permuted row")
    pp = permuted_probs if with_probs else None
    op = output_probs if with_probs else None
    _C.call(
        "pta_moe_unpermute", _C.ptr(permuted_tokens), permuted_tokens.shape[0], _C.in_dtype_code(permuted_tokens.dtype),
        int(hidden_size), _C.ptr(output_tokens), output_tokens.shape[0], _C.ptr(row_id_map),
        _C.ptr(num_dispatched_tokens), int(num_local_experts), _C.ptr(pp), _C.ptr(op), int(probs_stride),
        _C.stream(permuted_tokens.device),
    )
