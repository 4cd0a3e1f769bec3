"""Backend selection surface of the reference (primus_turbo/pytorch/core/backend.py:59-270).

The reference dispatches each FP8 op between hipBLASLt, CK, Triton, FlyDSL and
a hand-written kernel.  This build has exactly one implementation per op (the
gfx950 HIP kernels), so the manager only keeps the API: the environment
variables and setters are parsed and validated, and every backend name maps
to the native kernels.
"""

from __future__ import annotations

import os
from enum import Enum
from typing import Dict, Optional


class BackendType(Enum):
    CK = 1
    HIPBLASLT = 2
    TRITON = 3
    AITER = 4
    TURBO = 5
    FLYDSL = 6


class PrecisionType(Enum):
    BF16_FP16_FP32 = 1
    FP8 = 2
    FP4 = 3


ENV_GEMM_BACKEND = "PRIMUS_TURBO_GEMM_BACKEND"
ENV_GROUPED_GEMM_BACKEND = "PRIMUS_TURBO_GROUPED_GEMM_BACKEND"
ENV_AUTO_TUNE = "PRIMUS_TURBO_AUTO_TUNE"

_PRECISION_KEYS = {"BF16": PrecisionType.BF16_FP16_FP32, "FP16": PrecisionType.BF16_FP16_FP32,
                   "FP32": PrecisionType.BF16_FP16_FP32, "FP8": PrecisionType.FP8, "FP4": PrecisionType.FP4}


def _parse_backend_env(value: Optional[str]) -> Dict[PrecisionType, BackendType]:
    """'TRITON' or 'FP8:TRITON,BF16:CK' -> {precision: backend}."""
    out: Dict[PrecisionType, BackendType] = {}
    if not value:
        return out
    for item in value.split(","):
        item = item.strip()
        if not item:
            continue
        if ":" in item:
            key, name = (s.strip().upper() for s in item.split(":", 1))
            if key not in _PRECISION_KEYS:
                raise ValueError(f"unknown precision '{key}' in backend spec '{value}'")
            out[_PRECISION_KEYS[key]] = BackendType[name]
        else:
            b = BackendType[item.upper()]
            for p in PrecisionType:
                out.setdefault(p, b)
    return out


class GlobalBackendManager:
    _gemm_backend: Dict[PrecisionType, BackendType] = {}
    _grouped_gemm_backend: Dict[PrecisionType, BackendType] = {}
    _auto_tune: Optional[bool] = None

    @classmethod
    def set_gemm_backend(cls, backend: Optional[BackendType], precision: PrecisionType = PrecisionType.FP8):
        if backend is None:
            cls._gemm_backend.pop(precision, None)
        else:
            cls._gemm_backend[precision] = backend

    @classmethod
    def get_gemm_backend(cls, precision: PrecisionType) -> Optional[BackendType]:
        if precision in cls._gemm_backend:
            return cls._gemm_backend[precision]
        return _parse_backend_env(os.environ.get(ENV_GEMM_BACKEND)).get(precision)

    @classmethod
    def set_grouped_gemm_backend(cls, backend: Optional[BackendType], precision: PrecisionType = PrecisionType.FP8):
        if backend is None:
            cls._grouped_gemm_backend.pop(precision, None)
        else:
            cls._grouped_gemm_backend[precision] = backend

    @classmethod
    def get_grouped_gemm_backend(cls, precision: PrecisionType) -> Optional[BackendType]:
        if precision in cls._grouped_gemm_backend:
            return cls._grouped_gemm_backend[precision]
        return _parse_backend_env(os.environ.get(ENV_GROUPED_GEMM_BACKEND)).get(precision)

    @classmethod
    def set_auto_tune(cls, enable: Optional[bool]):
        cls._auto_tune = enable

    @classmethod
    def auto_tune_enabled(cls) -> bool:
        if cls._auto_tune is not None:
            return cls._auto_tune
        return os.environ.get(ENV_AUTO_TUNE, "0") not in ("0", "", "false", "False")

    @classmethod
    def reset(cls):
        cls._gemm_backend = {}
        cls._grouped_gemm_backend = {}
        cls._auto_tune = None
