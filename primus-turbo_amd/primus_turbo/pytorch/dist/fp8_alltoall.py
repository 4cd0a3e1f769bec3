"""FP8AllToAll: an all-to-all(-v) whose payload travels as FP8 bytes
(drop-in for primus_turbo/pytorch/dist/fp8_alltoall.py:25-194).

One direction of the exchange is the same in forward and backward, with the
split lists swapped, so both run through ``_fp8_exchange``:

1. tensorwise quantize of the local rows (``quantize_fp8``, the gfx950
   tensorwise kernel);
2. all-reduce(MIN) of the 4-byte ``scale_inv`` over the group;
3. ``all_to_all_single`` of the uint8 bytes (1 byte per element instead of
   2 or 4);
4. dequantize of the received bytes with the reduced ``scale_inv``
   (``dequantize_fp8``).

The order is the reference's (fp8_alltoall.py:82-116): each sender quantizes
with its own scale and every receiver dequantizes with the group's minimum
``scale_inv``, so a sender's rows come back exactly scaled only when its amax
equals the group's smallest amax; otherwise they come back scaled by
amax_min / amax_sender, as in the reference.  Steps 2 and 3 are RCCL
collectives (the group's backend); steps 1 and 4 are this build's kernels.
With one rank the function returns its input unchanged in both directions
(the reference's forward bypass; its backward bypass returns a bare tensor
where autograd needs one gradient per input, which this one does not repeat).
"""

from __future__ import annotations

from typing import List, Optional, Tuple, Union

import torch
import torch.distributed as dist

from primus_turbo.pytorch.core.low_precision import (
    Float8QuantConfig,
    Format,
    ScalingGranularity,
    ScalingStrategy,
    float8_e4m3,
    float8_e5m2,
)
from primus_turbo.pytorch.ops.quantization import dequantize_fp8, quantize_fp8

__all__ = ["FP8AllToAll"]


def _fp8_dtype(fmt: Format, forward: bool) -> torch.dtype:
    """E4M3 both ways; HYBRID: E4M3 forward, E5M2 backward (fp8_alltoall.py:67-72,134-139)."""
    if fmt == Format.E4M3:
        return float8_e4m3
    if fmt == Format.HYBRID:
        return float8_e4m3 if forward else float8_e5m2
    raise ValueError("FP8AlltoAll only support E4M3 and HYBRID format.")


def _quantize_payload(x: torch.Tensor, fp8_dtype: torch.dtype, granularity: ScalingGranularity,
                      group) -> Tuple[torch.Tensor, torch.Tensor]:
    """Steps 1-2: the local rows as uint8 FP8 bytes and the group-reduced scale_inv."""
    q, scale_inv = quantize_fp8(x, fp8_dtype, granularity)
    if group is not None:
        dist.all_reduce(scale_inv, op=dist.ReduceOp.MIN, group=group)
    return q.view(torch.uint8), scale_inv


def _dequantize_payload(received: torch.Tensor, fp8_dtype: torch.dtype, orig_dtype: torch.dtype,
                        granularity: ScalingGranularity, scale_inv: torch.Tensor) -> torch.Tensor:
    """Step 4: received uint8 bytes back to ``orig_dtype`` with the reduced scale_inv."""
    if received.nelement() == 0:
        return torch.empty_like(received, dtype=orig_dtype)
    return dequantize_fp8(received.view(fp8_dtype), orig_dtype, granularity, scale_inv=scale_inv)


def _fp8_exchange(x: torch.Tensor, quant: bool, fp8_dtype: torch.dtype, granularity: ScalingGranularity, group,
                  out_splits: Optional[List[int]], in_splits: Optional[List[int]]) -> torch.Tensor:
    """One all-to-all(-v) along dim 0: rows ``in_splits[r]`` go to rank r and
    ``out_splits[r]`` rows arrive from it (equal splits when None)."""
    orig_dtype = x.dtype
    x = x.contiguous()
    if quant:
        payload, scale_inv = _quantize_payload(x, fp8_dtype, granularity, group)
    else:
        payload, scale_inv = x, None
    rows = payload.shape[0] if out_splits is None else sum(out_splits)
    received = torch.empty((rows, *payload.shape[1:]), dtype=payload.dtype, device=payload.device)
    dist.all_to_all_single(received, payload, output_split_sizes=out_splits, input_split_sizes=in_splits,
                           group=group)
    if received.nelement() == 0:
        return torch.empty_like(received, dtype=orig_dtype)
    if not quant:
        return received
    return _dequantize_payload(received, fp8_dtype, orig_dtype, granularity, scale_inv)


class FP8AllToAll(torch.autograd.Function):
    """All-to-all of ``input_`` along dim 0 over ``group`` with FP8 payloads.

    Args (fp8_alltoall.py:25-50): group, input_, output_split_sizes,
    input_split_sizes (None: dim 0 divides equally by the world size),
    fwd_quant / bwd_quant (FP8 payload in forward / backward), config
    (``ScalingStrategy.DYNAMIC`` and ``ScalingGranularity.TENSORWISE`` only;
    format E4M3 or HYBRID).
    """

    @staticmethod
    def forward(ctx, group, input_: torch.Tensor, output_split_sizes: Union[List, None],
                input_split_sizes: Union[List, None], fwd_quant: bool, bwd_quant: bool,
                config: Float8QuantConfig) -> torch.Tensor:
        assert group is not None, "group should not be None."
        assert config.strategy == ScalingStrategy.DYNAMIC
        assert config.granularity == ScalingGranularity.TENSORWISE
        fp8_dtype = _fp8_dtype(config.format, True)
        ctx.group, ctx.config, ctx.bwd_quant = group, config, bwd_quant
        ctx.output_split_sizes, ctx.input_split_sizes = output_split_sizes, input_split_sizes
        if dist.get_world_size(group=group) == 1:
            return input_
        return _fp8_exchange(input_, fwd_quant, fp8_dtype, config.granularity, group, output_split_sizes,
                             input_split_sizes)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        fp8_dtype = _fp8_dtype(ctx.config.format, False)
        if dist.get_world_size(group=ctx.group) == 1:
            dgrad = grad_output
        else:
            # the reverse exchange: what arrived from rank r goes back to it
            dgrad = _fp8_exchange(grad_output, ctx.bwd_quant, fp8_dtype, ctx.config.granularity, ctx.group,
                                  ctx.input_split_sizes, ctx.output_split_sizes)
        return None, dgrad, None, None, None, None, None
