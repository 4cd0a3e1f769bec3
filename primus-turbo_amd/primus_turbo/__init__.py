"""MI355X-native FP8 linear path with the Primus-Turbo Python operator surface.

``import primus_turbo.pytorch as turbo`` exposes ``turbo.ops.quantize_fp8``,
``turbo.ops.gemm_fp8``, ``turbo.ops.grouped_gemm_fp8`` and the
``Float8QuantConfig`` types, backed by hand-written gfx950 HIP kernels in
``lib/libprimus_turbo_amd.so``.
"""

__version__ = "0.1.0"
