"""PyTorch front end: ``import primus_turbo.pytorch as turbo``.

Mirrors the reference's primus_turbo/pytorch/__init__.py for the FP8 linear
path: ``turbo.ops`` (quantize_fp8, gemm_fp8, grouped_gemm_fp8, ...),
``turbo.modules`` (Float8Linear), ``turbo.dist`` (FP8AllToAll), ``turbo.float8_e4m3`` / ``turbo.float8_e5m2``
and the core config types.
"""

from primus_turbo.pytorch import core, dist, modules, ops  # noqa: F401
from primus_turbo.pytorch.core.low_precision import float8_e4m3, float8_e5m2  # noqa: F401
