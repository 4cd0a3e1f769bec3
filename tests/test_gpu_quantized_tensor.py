"""GPU parity of QuantizedTensor: quantize / dequantize against the oracle,
transposes, grouped MX, and gemm_fp8 fed with pre-quantized operands."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import FMT, assert_bytes_equal, assert_f32_bitexact, f32, randn, u8

pytestmark = pytest.mark.gpu


def _mods():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScalingGranularity, ScalingRecipe
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor, create_quantized_weight

    return turbo, Float8QuantConfig, Format, ScalingGranularity, ScalingRecipe, QuantizedTensor, create_quantized_weight


def _bf16(x: np.ndarray) -> np.ndarray:
    return f32(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16))


@pytest.mark.parametrize("qdt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_quantize_dequantize_vs_oracle(qdt):
    _, _, _, SG, SR, QT, _ = _mods()
    x = randn((256, 384), seed=11)
    xc = x.cuda()
    fmt = FMT[qdt]
    # tensorwise
    q = QT.quantize(xc, qdt, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, fmt)
    assert_bytes_equal(u8(q.qdata), qo, "tensorwise bytes")
    assert np.array_equal(f32(q.dequantize()), _bf16(O.dequant_tensorwise(qo, fmt, so)))
    # rowwise along K
    q = QT.quantize(xc, qdt, SG.ROWWISE, axis=-1)
    qo, so = O.quant_rowwise(x, fmt, -1)
    assert_bytes_equal(u8(q.qdata), qo, "rowwise bytes")
    assert np.array_equal(f32(q.dequantize()), _bf16(O.dequant_rowwise(qo, fmt, so)))
    # blockwise 1x128 activation and 128x128 weight
    q = QT.quantize(xc, qdt, SG.BLOCKWISE, axis=-1, block_size=128)
    qo, so = O.quant_block1d(x, fmt, 1)
    assert_bytes_equal(u8(q.qdata), qo, "blockwise bytes")
    assert_f32_bitexact(f32(q.scale_inv), so, "blockwise scales")
    assert np.array_equal(f32(q.dequantize()), _bf16(O.dequant_block1d(qo, fmt, so, 1)))
    q = QT.quantize(xc, qdt, SG.BLOCKWISE, axis=-1, block_size=128, scaling_recipe=SR(use_2d_block=True))
    qo, so = O.quant_block_weight(x, fmt)
    assert_bytes_equal(u8(q.qdata), qo, "weight bytes")
    assert np.array_equal(f32(q.dequantize()), _bf16(O.dequant_block2d(qo, fmt, so)))
    # MX rowwise, inner dim not a multiple of 128 (stored padded, dequantized back to the shape)
    xm = randn((96, 160), seed=12)
    q = QT.quantize(xm.cuda(), qdt, SG.MX_BLOCKWISE, axis=-1, block_size=32, scaling_recipe=SR())
    qo, eo = O.quant_mx(xm, fmt, 1)
    assert_bytes_equal(u8(q.qdata), qo, "mx bytes")
    d = f32(q.dequantize())
    assert d.shape == (96, 160)
    assert np.array_equal(d, _bf16(O.dequant_mx(qo, fmt, eo))[:, :160])


def test_transposes():
    _, _, _, SG, _, QT, _ = _mods()
    x = randn((128, 320), seed=13).cuda()
    qdt = torch.float8_e4m3fn
    q = QT.quantize(x, qdt, SG.TENSORWISE)
    t = q.t()
    assert isinstance(t, QT) and t.shape == (320, 128)
    assert_bytes_equal(u8(t.qdata), u8(q.qdata).T, "tensorwise transpose is a byte transpose")
    assert torch.equal(t.scale_inv, q.scale_inv)
    assert torch.equal(q.transpose(-2, -1).qdata.view(torch.uint8), t.qdata.view(torch.uint8))
    # rowwise: dequantize, transpose, re-quantize along axis -2
    q = QT.quantize(x, qdt, SG.ROWWISE, axis=-1)
    t = q.t()
    ref = QT.quantize(q.dequantize().t().contiguous(), qdt, SG.ROWWISE, axis=-2)
    assert t.quantized_axis == 0
    assert torch.equal(t.qdata.view(torch.uint8), ref.qdata.view(torch.uint8))
    assert torch.equal(t.scale_inv, ref.scale_inv)


def test_batched_colwise_mx_quantized_tensor():
    """3-D MX along the middle axis: dequantize() gives the original [B, M, N]
    back (the op itself returns the stored [B, N, M_pad] layout)."""
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG, ScalingRecipe as SR
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor as QT

    x = torch.randn((2, 96, 64), generator=torch.Generator().manual_seed(4)).bfloat16().cuda()
    q = QT.quantize(x, torch.float8_e4m3fn, SG.MX_BLOCKWISE, axis=-2, block_size=32, scaling_recipe=SR())
    y = q.dequantize()
    assert y.shape == x.shape
    torch.testing.assert_close(y, x, rtol=0.1, atol=0.1)


@pytest.mark.parametrize("axis", [-1, -2])
def test_grouped_mx_quantized_tensor(axis):
    """Grouped MX QuantizedTensor: padded groups in, packed rows back out of
    dequantize (grouped_dequantize_mxfp8 in the reference)."""
    _, _, _, SG, SR, QT, _ = _mods()
    lens = [100, 0, 37, 200]
    M, N = sum(lens), 256
    x = randn((M, N), seed=14)
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    q = QT.quantize(x.cuda(), torch.float8_e4m3fn, SG.MX_BLOCKWISE, axis=axis, group_lens=gl, block_size=32,
                    scaling_recipe=SR())
    q_row, e_row, offs_row, q_col, e_col, offs_col = O.quant_mx_grouped(x, 0, lens)
    d = f32(q.dequantize())
    assert d.shape == (M, N)
    if axis == -1:
        assert np.array_equal(q.group_offs.cpu().numpy(), offs_row)
        deq = O.dequant_mx(q_row, 0, e_row)
        rows = np.concatenate([np.arange(offs_row[g], offs_row[g] + L) for g, L in enumerate(lens)])
        ref = deq[rows, :N]
    else:
        assert np.array_equal(q.group_offs.cpu().numpy(), offs_col)
        deq = O.dequant_mx(q_col, 0, e_col)  # [N, padded M]
        cols = np.concatenate([np.arange(offs_col[g], offs_col[g] + L) for g, L in enumerate(lens)])
        ref = deq[:, cols].T
    assert np.array_equal(d, _bf16(ref))


@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
def test_gemm_fp8_with_quantized_inputs(gran):
    """gemm_fp8 on QuantizedTensor operands gives the same output as on the
    high-precision tensors it quantizes internally."""
    turbo, Cfg, Fmt, SG, SR, QT, create_w = _mods()
    g = getattr(SG, gran)
    from primus_turbo.pytorch.core.low_precision import ScaleDtype

    bs = {"BLOCKWISE": 128, "MX_BLOCKWISE": 32}.get(gran)
    kw = {"block_size": bs} if bs else {}
    if g == SG.MX_BLOCKWISE:
        kw["scale_dtype"] = ScaleDtype.E8M0
    cfg = Cfg(granularity=g, format=Fmt.E4M3, **kw)
    a = randn((256, 512), seed=15).cuda()
    w = randn((384, 512), seed=16, scale=0.05).cuda()
    ref = turbo.ops.gemm_fp8(a, w, False, True, torch.bfloat16, cfg)
    recipe = SR() if g == SG.MX_BLOCKWISE else None
    qa = QT.quantize(a, torch.float8_e4m3fn, g, axis=-1, block_size=bs, scaling_recipe=recipe)
    qw, _ = create_w(w, torch.float8_e4m3fn, cfg)
    out = turbo.ops.gemm_fp8(qa, qw, False, True, torch.bfloat16, cfg)
    assert torch.equal(out, ref), f"{gran}: max diff {(out.float() - ref.float()).abs().max().item()}"


@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
@pytest.mark.parametrize("layout", ["NT", "NN"])
def test_gemm_fp8_quantized_pair_fwd_bwd(gran, layout):
    """The reference's QuantizedTensor gemm test (tests/pytorch/ops/test_gemm_fp8.py:349-466):
    inputs quantized outside gemm_fp8 and passed as QuantizedTensorPair(data, None);
    the gradients reach the QuantizedTensor leaves with the high-precision shapes,
    and forward / both gradients hold the reference's SNR bound (> 25 dB, e4m3)."""
    turbo, Cfg, Fmt, SG, SR, QT, _ = _mods()
    from primus_turbo.pytorch.core.low_precision import ScaleDtype
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensorPair

    g = getattr(SG, gran)
    if layout == "NN" and g == SG.MX_BLOCKWISE:
        pytest.skip("MX gemm_fp8 is NT only (gemm_fp8.py:525)")
    trans_b = layout == "NT"
    m, n, k = 256, 384, 512
    bs = {"BLOCKWISE": 128, "MX_BLOCKWISE": 32}.get(gran)
    kw = {"block_size": bs} if bs else {}
    if g == SG.MX_BLOCKWISE:
        kw["scale_dtype"] = ScaleDtype.E8M0
    cfg = Cfg(granularity=g, format=Fmt.E4M3, **kw)
    gen = torch.Generator().manual_seed(42)
    a = torch.randn((m, k), generator=gen).bfloat16().cuda().requires_grad_(True)
    b = torch.randn((n, k) if trans_b else (k, n), generator=gen).bfloat16().cuda().requires_grad_(True)
    a_ref = a.detach().float().requires_grad_(True)
    b_ref = b.detach().float().requires_grad_(True)
    qa = QT.quantize(a, torch.float8_e4m3fn, g, block_size=bs, axis=-1,
                     scaling_recipe=SR() if g == SG.MX_BLOCKWISE else None)
    qb = QT.quantize(b, torch.float8_e4m3fn, g, block_size=bs, axis=-1 if trans_b else -2,
                     scaling_recipe=SR(use_2d_block=True) if g in (SG.MX_BLOCKWISE, SG.BLOCKWISE) else None)
    c_ref = a_ref @ (b_ref.T if trans_b else b_ref)
    gc = torch.randn(c_ref.shape, generator=gen).cuda()
    c_ref.backward(gc)
    c = turbo.ops.gemm_fp8(QuantizedTensorPair(data=qa, data_t=None), QuantizedTensorPair(data=qb, data_t=None),
                           False, trans_b, torch.bfloat16, cfg)
    c.backward(gc.bfloat16())
    assert c.shape == c_ref.shape
    assert qa.grad is not None and qa.grad.shape == a.shape
    assert qb.grad is not None and qb.grad.shape == b.shape
    for name, x, r in (("C", c, c_ref), ("dA", qa.grad, a_ref.grad), ("dB", qb.grad, b_ref.grad)):
        s = O.snr_db(f32(r), f32(x))
        assert s > 25, f"{gran} {layout} {name}: SNR {s:.1f} dB"
