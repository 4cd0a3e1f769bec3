"""Device capability helpers (primus_turbo/pytorch/core/utils.py:13-36 in the reference)."""

from __future__ import annotations

import functools

import torch


@functools.lru_cache(maxsize=None)
def get_device_compute_capability():
    """(major, minor) of the current device, e.g. (9, 5) for gfx950; (0, 0) without a GPU."""
    if not torch.cuda.is_available():
        return (0, 0)
    return torch.cuda.get_device_capability()


def is_gfx950() -> bool:
    return get_device_compute_capability() == (9, 5)


def is_gfx942() -> bool:
    return get_device_compute_capability() == (9, 4)


@functools.lru_cache(maxsize=None)
def get_num_cus() -> int:
    if not torch.cuda.is_available():
        return 0
    return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
