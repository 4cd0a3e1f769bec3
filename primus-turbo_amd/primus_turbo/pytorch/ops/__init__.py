from primus_turbo.pytorch.ops.gemm_fp8 import gemm_fp8  # noqa: F401
from primus_turbo.pytorch.ops.grouped_gemm_fp8 import grouped_gemm_fp8  # noqa: F401
from primus_turbo.pytorch.ops.quantization import (  # noqa: F401
    dequantize_fp8,
    grouped_dequantize_fp8,
    grouped_quantize_fp8,
    grouped_quantize_fp8_with_trans,
    quantize_fp8,
    quantize_fp8_with_trans,
)
from primus_turbo.pytorch.ops.moe import moe_permute, moe_unpermute  # noqa: F401
