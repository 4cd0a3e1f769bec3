"""Quantizers on inputs holding NaN (quiet and signalling, both signs), infinities,
signed zeros, subnormals and the largest finite values: FP8 bytes and scale bits
against the CPU oracle, whose amax drops NaN (fmaxf) and whose clamp sends NaN to
+max (fminf / fmaxf), as the reference's kernels do
(csrc/include/primus_turbo/device/reduce.cuh:100-116, quant_utils.cuh:31-38)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import FMT, assert_bytes_equal, assert_f32_bitexact, f32, randn, u8

pytestmark = pytest.mark.gpu

FP8 = [torch.float8_e4m3fn, torch.float8_e5m2]

# bf16 bit patterns: qNaN, -qNaN, sNaN, -sNaN, +inf, -inf, +0, -0, largest finite
# of both signs, smallest subnormal of both signs, smallest normal
SPECIAL = [0x7FC0, 0xFFC0, 0x7F81, 0xFF81, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x7F7F, 0xFF7F, 0x0001, 0x8001, 0x0080]


def _special_input(shape, seed, with_inf=True):
    """Seeded N(0,1) bf16 with special values planted in several 128-blocks: all of
    SPECIAL in row 0; single NaNs; a column run of sNaN; a 1 x 128 block of NaN
    only; the largest finite value; -inf in the last element."""
    x = randn(shape, seed=seed, outliers=0.001)
    M, N = x.shape[-2], x.shape[-1]
    v = x.view(torch.int16)
    pats = SPECIAL if with_inf else [p for p in SPECIAL if p not in (0x7F80, 0xFF80)]
    for j, p in enumerate(pats[: min(len(pats), N)]):
        v[..., 0, j] = torch.tensor(p, dtype=torch.int32).to(torch.int16)
    nan = torch.tensor(0x7FC0, dtype=torch.int32).to(torch.int16)
    snan = torch.tensor(0x7F81, dtype=torch.int32).to(torch.int16)
    if M > 5 and N > 200:
        v[..., 5, 200] = nan
    if M > 135 and N > 300:
        v[..., 130:135, 300] = snan
    if M > 200 and N >= 512:
        v[..., 200, 384:512] = nan
    if M > 64 and N > 130:
        v[..., 64, 130] = torch.tensor(0x7F7F, dtype=torch.int32).to(torch.int16)
    if with_inf:
        v[..., M - 1, N - 1] = torch.tensor(0xFF80, dtype=torch.int32).to(torch.int16)
    return x


def _turbo():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity, ScalingRecipe

    return turbo, ScalingGranularity, ScalingRecipe


@pytest.mark.parametrize("with_inf", [True, False])
@pytest.mark.parametrize("qdt", FP8)
def test_tensorwise_special(qdt, with_inf):
    turbo, SG, _ = _turbo()
    x = _special_input((256, 512), seed=21, with_inf=with_inf)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, FMT[qdt])
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s).reshape(()), so, "scale")


@pytest.mark.parametrize("qdt", FP8)
def test_rowwise_special(qdt):
    turbo, SG, _ = _turbo()
    x = _special_input((256, 512), seed=22)
    for axis in (-1, 0):
        q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.ROWWISE, axis=axis)
        qo, so = O.quant_rowwise(x, FMT[qdt], axis)
        assert_bytes_equal(u8(q), qo, f"fp8 bytes (axis {axis})")
        assert_f32_bitexact(f32(s), so, f"scales (axis {axis})")


@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_1d_and_dual_special(qdt):
    turbo, SG, _ = _turbo()
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_dual_impl

    x = _special_input((256, 512), seed=23)
    for axis in (0, 1):
        q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.BLOCKWISE, block_size=128, axis=axis)
        qo, so = O.quant_block1d(x, FMT[qdt], axis)
        assert_bytes_equal(u8(q), qo, f"fp8 bytes (axis {axis})")
        assert_f32_bitexact(f32(s), so, f"scales (axis {axis})")
    o = O.quant_block_dual(x, FMT[qdt])
    qr, sr, qc, sc = quant_fp8_blockwise_dual_impl(x.cuda(), qdt, 128)
    assert_bytes_equal(u8(qr), o[0], "row bytes")
    assert_f32_bitexact(f32(sr), o[1], "row scales")
    assert_bytes_equal(u8(qc), o[2], "col bytes")
    assert_f32_bitexact(f32(sc), o[3], "col scales")
    _, _, qct, _ = quant_fp8_blockwise_dual_impl(x.cuda(), qdt, 128, col_transposed=True)
    assert_bytes_equal(u8(qct)[:, :256], o[2].T, "transposed col bytes")


@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_weight_special(qdt):
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_for_weight_impl

    w = _special_input((2, 256, 512), seed=24)
    q, s, qt = quant_fp8_blockwise_for_weight_impl(w.cuda(), qdt, 128, with_transpose=True)
    qo, so = O.quant_block_weight(w, FMT[qdt])
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scales")
    assert_bytes_equal(u8(qt), np.ascontiguousarray(np.swapaxes(qo, -1, -2)), "transposed bytes")


@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_segment_special(qdt):
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_segment_m_row_col_impl

    x = _special_input((384, 512), seed=25)
    lens = torch.tensor([100, 0, 156, 128], dtype=torch.int64)
    offs = group_offs_from_lens(lens.cuda())
    qr, qc, sr, sc, vk_lens, vk_offs = quant_fp8_blockwise_segment_m_row_col_impl(
        x.cuda(), qdt, 128, lens.cuda(), offs)
    o = O.quant_block_segment(x, FMT[qdt], lens.numpy())
    P = int(o[5][-1])
    assert_bytes_equal(u8(qr), o[0], "row bytes")
    assert_f32_bitexact(f32(sr), o[2], "row scales")
    assert_bytes_equal(u8(qc)[:P], o[1][:P], "padded col bytes")
    assert_f32_bitexact(f32(sc)[: P // 128], o[3][: P // 128], "col scales")
