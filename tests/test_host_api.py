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


def _qt_host(shape, data_shape, gran, scale, **kw):
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor

    g = torch.Generator().manual_seed(3)
    data = torch.randint(0, 120, data_shape, dtype=torch.uint8, generator=g).view(torch.float8_e4m3fn)
    return QuantizedTensor(data, scale, shape=torch.Size(shape), orig_dtype=torch.bfloat16,
                           dest_dtype=torch.float8_e4m3fn, granularity=gran, **kw)


def test_quantized_tensor_is_a_tensor_wrapper():
    """QuantizedTensor behaves as the reference's wrapper subclass: outer
    shape / dtype of the high-precision tensor, views without dequantizing
    (quantized_tensor.py:148-836)."""
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor

    qt = _qt_host((64, 256), (64, 256), SG.TENSORWISE, torch.ones(()))
    assert isinstance(qt, torch.Tensor) and isinstance(qt, QuantizedTensor)
    assert qt.shape == (64, 256) and qt.dtype == torch.bfloat16 and qt.real_dtype == torch.float8_e4m3fn
    assert qt.dim() == 2 and qt.size(-1) == 256 and qt.device.type == "cpu"
    v = qt.view(32, 512)
    assert isinstance(v, QuantizedTensor) and v.shape == (32, 512)
    assert v.qdata.shape == (32, 512) and v.qdata.data_ptr() == qt.qdata.data_ptr()
    r = qt.reshape(-1, 128)
    assert r.shape == (128, 128) and r.qdata.shape == (128, 128)
    d = qt.detach()
    assert isinstance(d, QuantizedTensor) and d.granularity == SG.TENSORWISE and not d.requires_grad
    row = qt[3]
    assert not isinstance(row, QuantizedTensor) and torch.equal(row.view(torch.uint8), qt.qdata[3].view(torch.uint8))
    names, meta = qt.__tensor_flatten__()
    back = QuantizedTensor.__tensor_unflatten__({n: getattr(qt, n) for n in names}, meta, qt.shape, qt.stride())
    assert back.shape == qt.shape and back.granularity == qt.granularity and back.qdata is qt.qdata
    with pytest.raises(NotImplementedError):
        qt + 1  # arithmetic is not defined on quantized data


def test_quantized_tensor_mx_view_keeps_padding():
    """MX data is stored with the inner dim padded to 128 and one exponent per
    32 elements; a view re-pads the target shape the same way."""
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG, ScalingRecipe
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor

    e = torch.zeros((64, 4), dtype=torch.uint8)
    qt = _qt_host((64, 100), (64, 128), SG.MX_BLOCKWISE, e, block_size=32, scaling_recipe=ScalingRecipe(),
                  quantized_axis=-1)
    v = qt.view(32, 200)
    assert v.shape == (32, 200) and v.qdata.shape == (32, 256) and v.scale_inv.shape == (32, 8)
    assert v.quantized_axis == 1


def test_quantized_tensor_view_autograd():
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG

    qt = _qt_host((64, 256), (64, 256), SG.TENSORWISE, torch.ones(()), requires_grad=True)
    v = qt.view(128, 128)
    assert v.requires_grad
    g = torch.ones((128, 128), dtype=torch.bfloat16)
    (gin,) = torch.autograd.grad(v, qt, g)
    assert gin.shape == (64, 256)


@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
def test_dense_gemm_fp8_refuses_graph_capture(monkeypatch, gran):
    """Dense gemm_fp8 raises RuntimeError under HIP graph capture before it
    touches the device (the capture state is forced from the host here)."""
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, ScaleDtype, ScalingGranularity

    g = getattr(ScalingGranularity, gran)
    kw = {}
    if g == ScalingGranularity.BLOCKWISE:
        kw = dict(block_size=128)
    elif g == ScalingGranularity.MX_BLOCKWISE:
        kw = dict(block_size=32, scale_dtype=ScaleDtype.E8M0)
    cfg = Float8QuantConfig(granularity=g, **kw)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    a = torch.zeros(128, 128, dtype=torch.bfloat16)
    b = torch.zeros(128, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="graph capture"):
        turbo.ops.gemm_fp8(a, b, trans_b=True, config=cfg)
