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


@pytest.mark.parametrize("width", [1040, 2064, 3088, 4096, 6160, 14336])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("qdt", FP8)
def test_rowwise_packed_rows_special(width, dtype, qdt):
    """Last-axis rowwise on 16-bit rows of 1040-14336 elements: the wave-per-row
    (up to 4096) and workgroup-per-row kernels hold them packed two per
    register, with lanes whose 16-element chunk lies past the row's end
    (widths that are not a multiple of the chunk span).
    Rows carry NaN, +-inf, the largest finite value and NaN in the last
    element; the others are plain N(0,1) with outliers."""
    turbo, SG, _ = _turbo()
    x = randn((67, width), dtype=dtype, seed=23, outliers=0.001)
    big = torch.finfo(dtype).max
    x[1, 5] = float("nan")
    x[2, width - 1] = float("inf")
    x[3, 1000] = float("-inf")
    x[4, 7] = big
    x[4, width - 2] = -big
    x[5, width - 1] = float("nan")
    x[6, :] = 0.0
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.ROWWISE, axis=-1)
    qo, so = O.quant_rowwise(x, FMT[qdt], -1)
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scales")


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


@pytest.mark.parametrize("use_2d", [False, True])
@pytest.mark.parametrize("qdt", FP8)
def test_mxfp8_special(qdt, use_2d):
    """MX: exponents and bytes against the oracle's restatement of the rule
    (NaN-dropping amax, an infinite amax gives exponent 255 - emax, the cast
    clamped to +-max with NaN to +max), rowwise, colwise and dual."""
    turbo, SG, SR = _turbo()
    x = _special_input((256, 512), seed=26)
    r = SR(use_2d_block=use_2d)
    for direction, axis in ((1, 1), (0, 0)):
        q, e = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.MX_BLOCKWISE, block_size=32, axis=axis, scaling_recipe=r)
        qo, eo = O.quant_mx(x, FMT[qdt], direction, use_2d)
        assert_bytes_equal(u8(q), qo, f"mx bytes (direction {direction})")
        assert_bytes_equal(u8(e), eo, f"e8m0 (direction {direction})")
    qr, er, qc, ec = turbo.ops.quantize_fp8_with_trans(x.cuda(), qdt, SG.MX_BLOCKWISE, block_size=32,
                                                      scaling_recipe=r, scaling_recipe_for_trans=r)
    for (qk, ek), direction in (((qr, er), 1), ((qc, ec), 0)):
        qo, eo = O.quant_mx(x, FMT[qdt], direction, use_2d)
        assert_bytes_equal(u8(qk), qo, f"dual mx bytes (direction {direction})")
        assert_bytes_equal(u8(ek), eo, f"dual e8m0 (direction {direction})")


def _snan_dense(shape, seed, dtype=torch.bfloat16):
    """N(0,1) with 6% signalling NaN (both signs) and 4% values x100 at seeded
    positions, in bf16, fp16 or fp32: every 16-value lane chunk and every
    4-row column run is likely to hold a block maximum ahead of a signalling
    NaN, where a max that turned the NaN into a running NaN would lose the
    maximum before it."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    big = torch.rand(shape, generator=g) < 0.04
    x = torch.where(big, x * 100.0, x).to(dtype)
    snan = torch.rand(shape, generator=g) < 0.06
    neg = torch.rand(shape, generator=g) < 0.5
    if dtype == torch.float32:
        v = x.view(torch.int32)
        pos_bits = torch.tensor(0x7F800001, dtype=torch.int64).to(torch.int32)
        neg_bits = torch.tensor(0xFF800001, dtype=torch.int64).to(torch.int32)
    else:  # bf16: 0x7F81; fp16: exponent 11111, quiet bit clear, 0x7D00
        v = x.view(torch.int16)
        p, n = (0x7F81, 0xFF81) if dtype == torch.bfloat16 else (0x7D00, 0xFD00)
        pos_bits = torch.tensor(p, dtype=torch.int32).to(torch.int16)
        neg_bits = torch.tensor(n, dtype=torch.int32).to(torch.int16)
    v[snan & ~neg] = pos_bits
    v[snan & neg] = neg_bits
    return x


@pytest.mark.parametrize("in_dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("qdt", FP8)
def test_snan_every_quantizer(qdt, in_dt):
    """Signalling NaN scattered through the input: amax drops it wherever it
    falls in a lane's chain (tensorwise, rowwise on both axes, blockwise 1-D,
    dual, weight, segment and MX in both directions)."""
    turbo, SG, SR = _turbo()
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl, quant_fp8_blockwise_for_weight_impl,
        quant_fp8_blockwise_segment_m_row_col_impl)

    x = _snan_dense((384, 512), seed=31, dtype=in_dt)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, FMT[qdt])
    assert_bytes_equal(u8(q), qo, "tensorwise bytes")
    assert_f32_bitexact(f32(s).reshape(()), so, "tensorwise scale")
    for axis in (-1, 0):
        q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.ROWWISE, axis=axis)
        qo, so = O.quant_rowwise(x, FMT[qdt], axis)
        assert_bytes_equal(u8(q), qo, f"rowwise bytes (axis {axis})")
        assert_f32_bitexact(f32(s), so, f"rowwise scales (axis {axis})")
    for axis in (0, 1):
        q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.BLOCKWISE, block_size=128, axis=axis)
        qo, so = O.quant_block1d(x, FMT[qdt], axis)
        assert_bytes_equal(u8(q), qo, f"blockwise bytes (axis {axis})")
        assert_f32_bitexact(f32(s), so, f"blockwise scales (axis {axis})")
    o = O.quant_block_dual(x, FMT[qdt])
    qr, sr, qc, sc = quant_fp8_blockwise_dual_impl(x.cuda(), qdt, 128)
    assert_bytes_equal(u8(qr), o[0], "dual row bytes")
    assert_f32_bitexact(f32(sr), o[1], "dual row scales")
    assert_bytes_equal(u8(qc), o[2], "dual col bytes")
    assert_f32_bitexact(f32(sc), o[3], "dual col scales")
    w = x.reshape(3, 128, 512)
    q, s, qt = quant_fp8_blockwise_for_weight_impl(w.cuda(), qdt, 128, with_transpose=True)
    qo, so = O.quant_block_weight(w, FMT[qdt])
    assert_bytes_equal(u8(q), qo, "weight bytes")
    assert_f32_bitexact(f32(s), so, "weight scales")
    assert_bytes_equal(u8(qt), np.ascontiguousarray(np.swapaxes(qo, -1, -2)), "weight transposed bytes")
    lens = torch.tensor([100, 0, 156, 128], dtype=torch.int64)
    offs = group_offs_from_lens(lens.cuda())
    for col_t in (False, True):
        qr, qc, sr, sc, _, _ = quant_fp8_blockwise_segment_m_row_col_impl(
            x.cuda(), qdt, 128, lens.cuda(), offs, col_transposed=col_t)
        o = O.quant_block_segment(x, FMT[qdt], lens.numpy())
        P = int(o[5][-1])
        assert_bytes_equal(u8(qr), o[0], "segment row bytes")
        assert_f32_bitexact(f32(sr), o[2], "segment row scales")
        qcol = u8(qc)[:, :P].T if col_t else u8(qc)[:P]
        assert_bytes_equal(np.ascontiguousarray(qcol), o[1][:P], f"segment col bytes (transposed {col_t})")
        assert_f32_bitexact(f32(sc)[: P // 128], o[3][: P // 128], "segment col scales")
    if in_dt == torch.float32:
        return  # MX takes bf16 / fp16 inputs only, as the reference asserts
    for use_2d in (False, True):
        r = SR(use_2d_block=use_2d)
        for direction, axis in ((1, 1), (0, 0)):
            q, e = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.MX_BLOCKWISE, block_size=32, axis=axis,
                                          scaling_recipe=r)
            qo, eo = O.quant_mx(x, FMT[qdt], direction, use_2d)
            assert_bytes_equal(u8(q), qo, f"mx bytes (direction {direction}, 2-D {use_2d})")
            assert_bytes_equal(u8(e), eo, f"e8m0 (direction {direction}, 2-D {use_2d})")


@pytest.mark.parametrize("qdt", FP8)
def test_snan_grouped_mx(qdt):
    """Grouped MX quantize (rows split by group, padded per group) with
    scattered signalling NaN, against the oracle."""
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import grouped_quantize_mxfp8_impl

    lens = [300, 0, 513, 128, 59]
    x = _snan_dense((sum(lens), 256), seed=32)
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    go = group_offs_from_lens(gl)
    q_row, e_row, q_col, e_col, _, orw, _, oc = grouped_quantize_mxfp8_impl(x.cuda(), qdt, None, 32, gl, go, True)
    rq, re, rorw, cq, ce, roc = O.quant_mx_grouped(x, FMT[qdt], lens)
    assert np.array_equal(orw.cpu().numpy(), rorw) and np.array_equal(oc.cpu().numpy(), roc)
    R, C = int(rorw[-1]), int(roc[-1])
    assert_bytes_equal(u8(q_row)[:R], rq[:R], "grouped mx row bytes")
    assert_bytes_equal(u8(e_row)[:R], re[:R], "grouped mx row exponents")
    assert_bytes_equal(u8(q_col)[:, :C], cq[:, :C], "grouped mx col bytes")
    assert_bytes_equal(u8(e_col)[:, : C // 32], ce[:, : C // 32], "grouped mx col exponents")


@pytest.mark.parametrize("out", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("qdt", FP8)
def test_dequant_every_byte(qdt, out):
    """Every fp8 byte, the NaN codes (and e5m2's infinities) included, through
    the tensorwise, rowwise and blockwise (1-D both axes, 2-D) dequantizers,
    against the oracle's exact decode and float64 product; NaN must come out
    where the oracle has NaN."""
    turbo, SG, SR = _turbo()
    M, N = 256, 512
    q8 = (torch.arange(M * N, dtype=torch.int64) % 256).to(torch.uint8).view(M, N)
    q8 = q8[torch.randperm(M, generator=torch.Generator().manual_seed(4))].contiguous()
    q = q8.view(qdt)
    g = torch.Generator().manual_seed(5)

    def sc(*shape):
        return (torch.rand(shape, generator=g) * 3 + 0.01).float()

    def check(y, ref, what):
        # the reference multiplies in fp32 and then casts (quantization_tensorwise.cu:36-42):
        # the exact float64 product rounds to fp32 first, then to the output type
        np.testing.assert_array_equal(f32(y), torch.from_numpy(ref).float().to(out).float().numpy(), err_msg=what)

    s = sc()
    y = turbo.ops.dequantize_fp8(q.cuda(), out, SG.TENSORWISE, scale_inv=s.cuda())
    check(y, O.dequant_tensorwise(u8(q), FMT[qdt], s.numpy()), "tensorwise")
    s = sc(M, 1)
    y = turbo.ops.dequantize_fp8(q.cuda(), out, SG.ROWWISE, axis=-1, scale_inv=s.cuda())
    check(y, O.dequant_rowwise(u8(q), FMT[qdt], s.numpy()), "rowwise")
    for axis, shape in ((1, (M, N // 128)), (0, (M // 128, N))):
        s = sc(*shape)
        y = turbo.ops.dequantize_fp8(q.cuda(), out, SG.BLOCKWISE, block_size=128, axis=axis, scale_inv=s.cuda())
        check(y, O.dequant_block1d(u8(q), FMT[qdt], s.numpy(), axis), f"blockwise axis {axis}")
    s = sc(M // 128, N // 128)
    y = turbo.ops.dequantize_fp8(q.cuda(), out, SG.BLOCKWISE, block_size=128, scale_inv=s.cuda(),
                                 scaling_recipe=SR(use_2d_block=True))
    check(y, O.dequant_block2d(u8(q), FMT[qdt], s.numpy()), "blockwise 2-D")


@pytest.mark.parametrize("qdt", FP8)
def test_streamed_paired_tiles_special(qdt):
    """Inputs of 192 MiB or more are quantized two neighbouring 128 x 128 tiles
    per workgroup (neighbours along a tile row, or along a tile column for the
    modes that write a transposed copy of a non-grouped tensor).  NaN, sNaN and
    infinities sit in one tile of a pair whose neighbour is clean in either
    order: the weight mode's recomputation branch (taken by both tiles when
    either needs it) and the dual kernel's per-wave paths must give the
    oracle's bytes and scales for both tiles."""
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
    )

    M, N = 8192, 12288  # 192 MiB of bf16: the streamed, paired launch
    x = randn((M, N), seed=31, outliers=0.001)
    v = x.view(torch.int16)
    planted = {(3, 5): 0x7FC0, (100, 7): 0x7F80, (5 * 128 + 1, 11 * 128 + 2): 0x7F81,
               (M - 1, N - 1): 0xFF80, (40 * 128 + 9, 31 * 128 + 127): 0xFFC0}
    for (r, c), p in planted.items():
        v[r, c] = torch.tensor(p, dtype=torch.int32).to(torch.int16)
    xd = x.cuda()
    f = FMT[qdt]
    qo, so = O.quant_block_weight(x, f)
    q, s, qt = quant_fp8_blockwise_for_weight_impl(xd, qdt, 128, with_transpose=True)
    assert_bytes_equal(u8(q), qo, "weight bytes (pairs along a tile column)")
    assert_f32_bitexact(f32(s), so, "weight scales (pairs along a tile column)")
    assert_bytes_equal(u8(qt), np.ascontiguousarray(qo.T), "weight transposed bytes")
    del q, s, qt
    q, s = quant_fp8_blockwise_for_weight_impl(xd, qdt, 128)
    assert_bytes_equal(u8(q), qo, "weight bytes (pairs along a tile row)")
    assert_f32_bitexact(f32(s), so, "weight scales (pairs along a tile row)")
    del q, s, qo, so
    o = O.quant_block_dual(x, f)
    qr, sr, qc, sc = quant_fp8_blockwise_dual_impl(xd, qdt, 128)
    assert_bytes_equal(u8(qr), o[0], "dual row bytes")
    assert_f32_bitexact(f32(sr), o[1], "dual row scales")
    assert_bytes_equal(u8(qc), o[2], "dual col bytes")
    assert_f32_bitexact(f32(sc), o[3], "dual col scales")
    del qr, sr, qc, sc
    _, _, qct, _ = quant_fp8_blockwise_dual_impl(xd, qdt, 128, col_transposed=True)
    assert_bytes_equal(u8(qct), np.ascontiguousarray(o[2].T), "dual transposed col bytes")
