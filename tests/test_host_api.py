"""Host-side API behaviour that needs no GPU (config validation, backend
selection parsing, error behaviour of the op surface without a device)."""

import pytest
import torch


def test_quant_config_validation():
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, ScaleDtype, ScalingGranularity

    with pytest.raises(AssertionError):
        Float8QuantConfig(granularity=ScalingGranularity.BLOCKWISE)
    with pytest.raises(AssertionError):
        Float8QuantConfig(granularity=ScalingGranularity.MX_BLOCKWISE, block_size=32)  # scale dtype FP32
    with pytest.raises(AssertionError):
        Float8QuantConfig(granularity=ScalingGranularity.MX_BLOCKWISE, block_size=64, scale_dtype=ScaleDtype.E8M0)
    Float8QuantConfig(granularity=ScalingGranularity.MX_BLOCKWISE, block_size=32, scale_dtype=ScaleDtype.E8M0)
    c = Float8QuantConfig()
    assert c.granularity == ScalingGranularity.TENSORWISE


def test_granularity_codes_match_c_abi():
    from primus_turbo.pytorch import _C
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG

    assert (SG.TENSORWISE.value, SG.ROWWISE.value, SG.BLOCKWISE.value, SG.MX_BLOCKWISE.value) == (
        _C.PTA_TENSORWISE, _C.PTA_ROWWISE, _C.PTA_BLOCKWISE, _C.PTA_MX_BLOCKWISE)


def test_dtypes():
    import primus_turbo.pytorch as turbo

    assert turbo.float8_e4m3 == torch.float8_e4m3fn and turbo.float8_e5m2 == torch.float8_e5m2


def test_backend_env_parsing(monkeypatch):
    from primus_turbo.pytorch.core.backend import BackendType, GlobalBackendManager, PrecisionType

    GlobalBackendManager.reset()
    monkeypatch.setenv("PRIMUS_TURBO_GEMM_BACKEND", "FP8:TRITON,BF16:CK")
    assert GlobalBackendManager.get_gemm_backend(PrecisionType.FP8) == BackendType.TRITON
    assert GlobalBackendManager.get_gemm_backend(PrecisionType.BF16_FP16_FP32) == BackendType.CK
    monkeypatch.setenv("PRIMUS_TURBO_GEMM_BACKEND", "HIPBLASLT")
    assert GlobalBackendManager.get_gemm_backend(PrecisionType.FP8) == BackendType.HIPBLASLT
    GlobalBackendManager.set_gemm_backend(BackendType.TURBO)
    assert GlobalBackendManager.get_gemm_backend(PrecisionType.FP8) == BackendType.TURBO
    monkeypatch.setenv("PRIMUS_TURBO_GEMM_BACKEND", "FP9:TRITON")
    GlobalBackendManager.reset()
    with pytest.raises(ValueError):
        GlobalBackendManager.get_gemm_backend(PrecisionType.FP8)
    GlobalBackendManager.reset()


def test_ops_fail_loudly_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity

    x = torch.randn(4, 4, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="GPU"):
        turbo.ops.quantize_fp8(x, torch.float8_e4m3fn, ScalingGranularity.TENSORWISE)


def test_gemm_fp8_shape_asserts():
    import primus_turbo.pytorch as turbo

    with pytest.raises(AssertionError, match="2D"):
        turbo.ops.gemm_fp8(torch.zeros(2, 2, 2), torch.zeros(2, 2))


def test_float8_linear_conversion():
    """Float8Linear.from_float keeps the parameters (in place) or copies them."""
    import torch

    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, ScalingGranularity

    lin = torch.nn.Linear(64, 32, bias=True)
    w = lin.weight.detach().clone()
    cfg = Float8QuantConfig(granularity=ScalingGranularity.BLOCKWISE, block_size=128)
    new = turbo.modules.Float8Linear.from_float(lin, cfg, inplace=False)
    assert isinstance(new, turbo.modules.Float8Linear) and new.config is cfg
    assert torch.equal(new.weight, w) and torch.equal(new.bias, lin.bias)
    assert type(lin) is torch.nn.Linear
    same = turbo.modules.Float8Linear.from_float(lin)
    assert same is lin and isinstance(lin, turbo.modules.Float8Linear)
    assert lin.config.granularity == ScalingGranularity.TENSORWISE
    assert "config=" in repr(lin)
