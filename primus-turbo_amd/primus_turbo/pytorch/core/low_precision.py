"""FP8 dtypes and quantization config types.

Same names, values and validation as the reference's
primus_turbo/pytorch/core/low_precision.py:77-186.  This build targets gfx950
only, where FP8 is the OCP encoding (float8_e4m3fn / float8_e5m2).
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum, auto
from typing import NamedTuple, Optional, Tuple

import torch

from primus_turbo.pytorch.core.utils import get_device_compute_capability

__all__ = ["float8_e4m3", "float8_e5m2"]

float8_e4m3 = torch.float8_e4m3fn
float8_e5m2 = torch.float8_e5m2
float8_e8m0 = torch.float8_e8m0fnu
float4_e2m1fn_x2 = getattr(torch, "float4_e2m1fn_x2", None)


def is_fp8_dtype(dtype) -> bool:
    return dtype in (torch.float8_e4m3fn, torch.float8_e4m3fnuz, torch.float8_e5m2, torch.float8_e5m2fnuz)


def check_fp8_support() -> Tuple[bool, str]:
    if get_device_compute_capability() >= (9, 4):
        return True, ""
    return False, "Device compute capability gfx942 or higher required for FP8 execution."


def check_fp8_ocp_support() -> Tuple[bool, str]:
    if get_device_compute_capability() >= (9, 5):
        return True, ""
    return False, "Device compute capability gfx950 or higher required for FP8 OCP format."


def check_mxfp8_support() -> Tuple[bool, str]:
    if get_device_compute_capability() >= (9, 5):
        return True, ""
    return False, "Device compute capability gfx950 or higher required for MXFP8 execution."


MXFP8_BLOCK_SIZE = 32
MXFP8_PADDING_ALIGN_SIZE = 128
DEFAULT_BLOCK_SIZE = 128


class Format(Enum):
    E4M3 = auto()
    E5M2 = auto()
    E2M1_X2 = auto()
    HYBRID = auto()


class ScaleDtype(Enum):
    FP32 = auto()
    E8M0 = auto()


class ScalingGranularity(Enum):
    TENSORWISE = auto()
    ROWWISE = auto()
    BLOCKWISE = auto()
    MX_BLOCKWISE = auto()


class ScalingStrategy(Enum):
    DYNAMIC = auto()


class ScalingRecipe(NamedTuple):
    """use_2d_block selects 128x128 (blockwise) or 32x32 (MX) weight blocks.

    use_sr / use_rht / shuffle_scale / shuffle_out belong to layouts this build
    does not implement; quantizers reject them with NotImplementedError.
    """

    use_2d_block: bool = False
    use_sr: bool = False
    use_rht: bool = False
    shuffle_scale: bool = False
    shuffle_out: bool = False


@dataclass
class Float8QuantConfig:
    format: Format = Format.E4M3
    granularity: ScalingGranularity = ScalingGranularity.TENSORWISE
    strategy: ScalingStrategy = ScalingStrategy.DYNAMIC
    scale_dtype: ScaleDtype = ScaleDtype.FP32
    block_size: Optional[int] = None  # only used by BLOCKWISE / MX_BLOCKWISE

    def __post_init__(self):
        if self.granularity == ScalingGranularity.BLOCKWISE:
            assert self.block_size is not None, "block_size must be set when granularity is BLOCKWISE"
        if self.granularity == ScalingGranularity.MX_BLOCKWISE:
            assert self.block_size in [MXFP8_BLOCK_SIZE], (
                f"block_size should be {[MXFP8_BLOCK_SIZE]} when granularity is MX_BLOCKWISE"
            )
            assert self.scale_dtype == ScaleDtype.E8M0, (
                f"scale_dtype should be {ScaleDtype.E8M0} when granularity is MX_BLOCKWISE"
            )
