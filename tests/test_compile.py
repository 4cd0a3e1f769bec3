"""torch.compile support of the public quantize / dequantize ops.

The reference registers its quantization impls as custom ops with fake
implementations (quantization_impl.py:74-486) and tests quantize_fp8 under
torch.compile(fullgraph=True) (tests/pytorch/ops/test_quantization.py:34-50,
103-120).  CPU part: the ops trace without graph breaks on meta tensors and the
fake outputs have the reference's shapes.  GPU part: compiled == eager, bit
for bit, and Float8Linear under torch.compile (test_linear_fp8.py:33-70).
"""

import pytest
import torch


def _mods():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity, ScalingRecipe

    return turbo, ScalingGranularity, ScalingRecipe


def _cases(SG, SR):
    return [
        ("tensorwise", SG.TENSORWISE, {}),
        ("rowwise_last", SG.ROWWISE, {"axis": -1}),
        ("rowwise_first", SG.ROWWISE, {"axis": 0}),
        ("block_1x128", SG.BLOCKWISE, {"axis": 1, "block_size": 128}),
        ("block_128x1", SG.BLOCKWISE, {"axis": 0, "block_size": 128}),
        ("block_weight", SG.BLOCKWISE, {"block_size": 128, "scaling_recipe": SR(use_2d_block=True)}),
        ("mx_row", SG.MX_BLOCKWISE, {"axis": 1, "block_size": 32}),
        ("mx_col", SG.MX_BLOCKWISE, {"axis": 0, "block_size": 32}),
    ]


EXPECTED = {  # (q shape, scale shape) for a [96, 160] input
    "tensorwise": ((96, 160), ()),
    "rowwise_last": ((96, 160), (96, 1)),
    "rowwise_first": ((96, 160), (1, 160)),
    "block_1x128": ((96, 160), (96, 2)),
    "block_128x1": ((96, 160), (1, 160)),
    "block_weight": ((96, 160), (1, 2)),
    "mx_row": ((96, 256), (96, 8)),
    "mx_col": ((160, 128), (160, 4)),
}


@pytest.mark.parametrize("name", list(EXPECTED))
def test_quantize_traces_fullgraph_on_meta(name):
    turbo, SG, SR = _mods()
    gran, kw = {c[0]: (c[1], c[2]) for c in _cases(SG, SR)}[name]
    torch._dynamo.reset()
    x = torch.empty(96, 160, dtype=torch.bfloat16, device="meta")
    q, s = torch.compile(lambda t: turbo.ops.quantize_fp8(t, torch.float8_e4m3fn, gran, **kw), fullgraph=True,
                         backend="aot_eager")(x)
    assert (tuple(q.shape), tuple(s.shape)) == EXPECTED[name]
    assert q.dtype == torch.float8_e4m3fn
    assert s.dtype == (torch.float8_e8m0fnu if gran == SG.MX_BLOCKWISE else torch.float32)
    d = torch.compile(lambda a, b: turbo.ops.dequantize_fp8(a, torch.bfloat16, gran, scale_inv=b, **kw),
                      fullgraph=True, backend="aot_eager")(q, s)
    assert d.dtype == torch.bfloat16


def test_with_trans_traces_fullgraph_on_meta():
    turbo, SG, SR = _mods()
    x = torch.empty(96, 256, dtype=torch.bfloat16, device="meta")
    torch._dynamo.reset()
    out = torch.compile(lambda t: turbo.ops.quantize_fp8_with_trans(t, torch.float8_e4m3fn, SG.BLOCKWISE,
                                                                    block_size=128),
                        fullgraph=True, backend="aot_eager")(x)
    assert [tuple(t.shape) for t in out] == [(96, 256), (96, 2), (96, 256), (1, 256)]
    torch._dynamo.reset()
    out = torch.compile(lambda t: turbo.ops.quantize_fp8_with_trans(t, torch.float8_e4m3fn, SG.MX_BLOCKWISE,
                                                                    block_size=32,
                                                                    scaling_recipe=SR(shuffle_scale=True)),
                        fullgraph=True, backend="aot_eager")(x)
    assert [tuple(t.shape) for t in out] == [(96, 256), (256, 8), (256, 128), (256, 4)]


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(EXPECTED))
def test_compiled_quantize_equals_eager(name):
    turbo, SG, SR = _mods()
    gran, kw = {c[0]: (c[1], c[2]) for c in _cases(SG, SR)}[name]
    g = torch.Generator().manual_seed(3)
    x = torch.randn((96, 160), generator=g).bfloat16().cuda()
    q0, s0 = turbo.ops.quantize_fp8(x, torch.float8_e4m3fn, gran, **kw)
    torch._dynamo.reset()
    q1, s1 = torch.compile(lambda t: turbo.ops.quantize_fp8(t, torch.float8_e4m3fn, gran, **kw), fullgraph=True)(x)
    assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8))
    assert q0.shape == q1.shape and s0.shape == s1.shape
    assert torch.equal(s0.view(torch.uint8) if s0.dtype == torch.float8_e8m0fnu else s0,
                       s1.view(torch.uint8) if s1.dtype == torch.float8_e8m0fnu else s1)
    d0 = turbo.ops.dequantize_fp8(q0, torch.bfloat16, gran, scale_inv=s0, **kw)
    d1 = torch.compile(lambda a, b: turbo.ops.dequantize_fp8(a, torch.bfloat16, gran, scale_inv=b, **kw),
                       fullgraph=True)(q0, s0)
    assert torch.equal(d0, d1)


@pytest.mark.gpu
def test_float8linear_under_torch_compile():
    turbo, SG, SR = _mods()
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format
    from primus_turbo.pytorch.modules import Float8Linear

    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 256, bias=True).cuda().bfloat16()
    cfg = Float8QuantConfig(granularity=SG.BLOCKWISE, format=Format.E4M3, block_size=128)
    m0 = Float8Linear.from_float(lin, cfg)
    x = torch.randn(128, 512, device="cuda", dtype=torch.bfloat16)
    x0 = x.clone().requires_grad_(True)
    y0 = m0(x0)
    gy = torch.randn_like(y0)
    y0.backward(gy)
    gw0 = m0.weight.grad.clone()
    m0.weight.grad = None
    m0.bias.grad = None
    torch._dynamo.reset()
    m1 = torch.compile(m0, fullgraph=False)
    x1 = x.clone().requires_grad_(True)
    y1 = m1(x1)
    y1.backward(gy)
    assert torch.equal(y0, y1)
    assert torch.equal(x0.grad, x1.grad)
    assert torch.equal(gw0, m0.weight.grad)
