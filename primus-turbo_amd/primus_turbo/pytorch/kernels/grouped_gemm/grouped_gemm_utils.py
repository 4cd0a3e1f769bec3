"""Group offset helpers (primus_turbo/pytorch/kernels/grouped_gemm/grouped_gemm_utils.py:28-34)."""

from __future__ import annotations

import torch

from primus_turbo.pytorch import _C


def group_offs_from_lens(group_lens: torch.Tensor) -> torch.Tensor:
    """int64 exclusive prefix sum [G+1] of group_lens, computed on the device."""
    assert group_lens.is_cuda, "group_lens must be on CUDA"
    lens = group_lens.to(torch.int64).contiguous()
    G = lens.numel()
    offs = torch.empty(G + 1, dtype=torch.int64, device=lens.device)
    _C.call("pta_grouped_compute_offs", _C.ptr(lens), _C.ptr(offs), G, _C.stream(lens.device))
    return offs
