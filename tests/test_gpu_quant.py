"""GPU parity of the quantization kernels: FP8 bytes and scales must be
bit-identical to (a) the CPU oracle and (b) where the reference's own HIP
kernels build (oracle/_ref), to the reference's kernels run on the same GPU."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (
    FMT,
    assert_bytes_equal,
    assert_f32_bitexact,
    f32,
    randn,
    ref_lib,
    stream,
    u8,
)

pytestmark = pytest.mark.gpu

FP8 = [torch.float8_e4m3fn, torch.float8_e5m2]


def _turbo():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity, ScalingRecipe

    return turbo, ScalingGranularity, ScalingRecipe


def _input(shape, dtype=torch.bfloat16, seed=0, special=True):
    x = randn(shape, dtype=dtype, seed=seed, outliers=0.001)
    if special and x.numel() >= 8:
        flat = x.view(-1)
        flat[0] = 0.0
        flat[1] = -0.0
        flat[2] = 1e-6
        flat[3] = -3.0e2
    return x


# ---------------------------------------------------------------------------
# tensorwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(512, 1024), (1000, 37), (3, 5, 7), (4096, 1536)])
@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_tensorwise_vs_oracle(shape, qdt, dtype):
    turbo, SG, _ = _turbo()
    x = _input(shape, dtype)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, FMT[qdt])
    assert q.shape == x.shape and s.shape == () and q.dtype == qdt
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scale_inv")


@pytest.mark.parametrize("qdt", FP8)
def test_tensorwise_every_bf16_value(qdt):
    """All finite bf16 values within +-max with amax == max (scale exactly 1):
    the bytes are the RNE encodings of the inputs themselves."""
    turbo, SG, _ = _turbo()
    u = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    mx = O.FP8_MAX[FMT[qdt]]
    vals = u[np.isfinite(u) & (np.abs(u) <= mx)]
    vals = np.concatenate([vals, [mx]]).astype(np.float32)
    x = torch.from_numpy(vals).to(torch.bfloat16)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.TENSORWISE)
    assert float(s) == 1.0
    exp = np.array([O.fp8_encode_scalar(float(v), FMT[qdt]) for v in vals], dtype=np.uint8)
    assert_bytes_equal(u8(q), exp, "rne bytes")


@pytest.mark.parametrize("n", [(1 << 19) + 5, (1 << 20) + 5, (1 << 21) - 7, 1 << 21, (1 << 21) + 16])
@pytest.mark.parametrize("spike", [0, -1, "mid"])
def test_tensorwise_single_launch_sizes(n, spike):
    """Sizes around the single-launch form's limits (16, 32 and 64 elements per
    thread, and the first size that takes the two-launch form): one spike
    anywhere, including the last workgroup's last element, sets the scale."""
    turbo, SG, _ = _turbo()
    x = _input((n,), seed=11)
    pos = n // 2 + 3 if spike == "mid" else spike
    x[pos] = -1000.0
    q, s = turbo.ops.quantize_fp8(x.cuda(), torch.float8_e4m3fn, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, FMT[torch.float8_e4m3fn])
    assert_f32_bitexact(f32(s), so, "scale_inv")
    assert_bytes_equal(u8(q), qo, "fp8 bytes")


def test_tensorwise_single_launch_workspace_reuse():
    """One workspace for consecutive single-launch calls on different inputs,
    enqueued back to back (a larger amax first, then a smaller one, then a
    smaller n): each call's per-call tag keeps it from reading the partial
    maxima an earlier call left in the workspace."""
    from primus_turbo.pytorch import _C

    n = (1 << 20) + 5
    ws_n = _C.query("pta_quantize_fp8_tensorwise_workspace_size", n)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    cases = []
    for seed, spike, m in ((31, 900.0, n), (32, 3.0, n), (33, 40.0, n // 3)):
        x = _input((m,), seed=seed, special=False)
        x[m // 2] = spike
        cases.append((x, x.cuda(), torch.empty(m, dtype=torch.uint8, device="cuda"),
                      torch.empty((), dtype=torch.float32, device="cuda")))
    for _, xd, q, s in cases:
        _C.call("pta_quantize_fp8_tensorwise", _C.ptr(xd), _C.PTA_BF16, xd.numel(), None, _C.ptr(q), _C.PTA_E4M3,
                _C.ptr(s), _C.ptr(ws), ws_n, _C.stream(xd.device))
    torch.cuda.synchronize()
    for i, (x, _, q, s) in enumerate(cases):
        qo, so = O.quant_tensorwise(x, FMT[torch.float8_e4m3fn])
        assert_f32_bitexact(f32(s), so, f"scale_inv of call {i}")
        assert_bytes_equal(u8(q), qo, f"fp8 bytes of call {i}")


@pytest.mark.parametrize("n", [1, 4096, 1 << 20, (1 << 20) + 13])
@pytest.mark.parametrize("qdt", FP8)
def test_tensorwise_vs_reference_kernels(n, qdt):
    L = ref_lib()
    if L is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    turbo, SG, _ = _turbo()
    x = _input((n,), seed=3).cuda()
    q, s = turbo.ops.quantize_fp8(x, qdt, SG.TENSORWISE)
    qr = torch.empty_like(q)
    sr = torch.empty((), dtype=torch.float32, device="cuda")
    ws = torch.empty(L.ref_tensorwise_ws_bytes(n), dtype=torch.uint8, device="cuda")
    assert L.ref_quant_tensorwise(x.data_ptr(), n, FMT[qdt], qr.data_ptr(), sr.data_ptr(), ws.data_ptr(), stream()) == 0
    torch.cuda.synchronize()
    assert_bytes_equal(u8(q), u8(qr), "fp8 bytes vs reference kernel")
    assert_f32_bitexact(f32(s), f32(sr), "scale_inv vs reference kernel")


# ---------------------------------------------------------------------------
# rowwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "shape,axis",
    [((256, 4096), -1), ((33, 100), -1), ((7, 5000), 1), ((3, 20000), -1), ((300, 96), 0), ((4, 300, 96), 1),
     ((2, 3, 64), 0)],
)
@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rowwise_vs_oracle(shape, axis, qdt, dtype):
    turbo, SG, _ = _turbo()
    x = _input(shape, dtype, seed=1)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.ROWWISE, axis=axis)
    qo, so = O.quant_rowwise(x, FMT[qdt], axis)
    assert tuple(s.shape) == so.shape
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scale_inv")


@pytest.mark.parametrize("shape,axis", [((256, 4096), -1), ((33, 100), -1), ((300, 96), 0), ((4, 300, 96), 1)])
@pytest.mark.parametrize("qdt", FP8)
def test_rowwise_vs_reference_kernels(shape, axis, qdt):
    L = ref_lib()
    if L is None:
        pytest.skip("oracle/_ref not built")
    turbo, SG, _ = _turbo()
    x = _input(shape, seed=2).cuda()
    q, s = turbo.ops.quantize_fp8(x, qdt, SG.ROWWISE, axis=axis)
    qr = torch.empty_like(q)
    ax = axis % x.dim()
    B = int(np.prod(shape[:ax])) if ax > 0 else 1
    M = shape[ax]
    N = int(np.prod(shape[ax + 1:])) if ax + 1 < len(shape) else 1
    sc = torch.empty(B * N, dtype=torch.float32, device="cuda")
    sr = torch.empty(B * N, dtype=torch.float32, device="cuda")
    if N == 1:
        assert L.ref_quant_rowwise_last(x.data_ptr(), B, M, FMT[qdt], qr.data_ptr(), sc.data_ptr(), sr.data_ptr(),
                                        stream()) == 0
    else:
        ws = torch.empty(L.ref_rowwise_col_ws_bytes(B, M, N), dtype=torch.uint8, device="cuda")
        assert L.ref_quant_rowwise_col(x.data_ptr(), B, M, N, FMT[qdt], qr.data_ptr(), sc.data_ptr(), sr.data_ptr(),
                                       ws.data_ptr(), stream()) == 0
    torch.cuda.synchronize()
    assert_bytes_equal(u8(q), u8(qr), "fp8 bytes vs reference kernel")
    assert_f32_bitexact(f32(s).reshape(-1), f32(sr), "scale_inv vs reference kernel")


# ---------------------------------------------------------------------------
# blockwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(256, 512), (300, 200), (128, 128), (1, 1000), (640, 7168)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_1d_vs_oracle(shape, axis, qdt):
    turbo, SG, _ = _turbo()
    x = _input(shape, seed=4)
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.BLOCKWISE, block_size=128, axis=axis)
    qo, so = O.quant_block1d(x, FMT[qdt], axis)
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scales")


@pytest.mark.parametrize("shape", [(256, 512), (300, 200), (4096, 2048)])
@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_dual_vs_oracle(shape, qdt):
    turbo, SG, _ = _turbo()
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_dual_impl

    x = _input(shape, seed=5)
    qr, sr, qc, sc = turbo.ops.quantize_fp8_with_trans(x.cuda(), qdt, SG.BLOCKWISE, block_size=128)
    o = O.quant_block_dual(x, FMT[qdt])
    assert_bytes_equal(u8(qr), o[0], "row bytes")
    assert_f32_bitexact(f32(sr), o[1], "row scales")
    assert_bytes_equal(u8(qc), o[2], "col bytes")
    assert_f32_bitexact(f32(sc), o[3], "col scales")
    # transposed column output: same bytes, [N, roundup(M,128)] with zero padding
    _, _, qct, sct = quant_fp8_blockwise_dual_impl(x.cuda(), qdt, 128, col_transposed=True)
    M, N = shape
    qct = u8(qct)
    assert_bytes_equal(qct[:, :M], o[2].T, "transposed col bytes")
    assert not qct[:, M:].any(), "padding must be zero"
    assert_f32_bitexact(f32(sct), o[3], "col scales (transposed path)")
    # K-block-major row scales: same values, storage [N/128, M]
    qrk, srk, _, _ = quant_fp8_blockwise_dual_impl(x.cuda(), qdt, 128, col_transposed=True, row_scale_kmajor=True)
    assert srk.shape == (M, -(-N // 128)) and srk.stride() == (1, M)
    assert_bytes_equal(u8(qrk), o[0], "row bytes (k-major scales)")
    assert_f32_bitexact(f32(srk), o[1], "row scales (k-major storage)")
    assert_f32_bitexact(f32(srk.t().contiguous()).T, o[1], "k-major storage order")


@pytest.mark.parametrize("shape", [(512, 384), (300, 260), (2, 300, 260), (4, 256, 640)])
@pytest.mark.parametrize("qdt", FP8)
def test_blockwise_weight_vs_oracle_and_reference(shape, qdt):
    turbo, SG, SR = _turbo()
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_for_weight_impl

    w = _input(shape, seed=6)
    q, s = turbo.ops.quantize_fp8(w.cuda(), qdt, SG.BLOCKWISE, block_size=128, scaling_recipe=SR(use_2d_block=True))
    qo, so = O.quant_block_weight(w, FMT[qdt])
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scales")
    _, _, qt = quant_fp8_blockwise_for_weight_impl(w.cuda(), qdt, 128, with_transpose=True)
    M = shape[-2]
    qt = u8(qt)
    assert_bytes_equal(qt[..., :M], np.swapaxes(qo, -1, -2), "transposed copy")
    assert not qt[..., M:].any()
    L = ref_lib()
    if L is not None:
        wc = w.cuda().contiguous()
        B = shape[0] if len(shape) == 3 else 1
        qr = torch.empty_like(q)
        sr = torch.empty_like(s)
        assert L.ref_quant_weight(wc.data_ptr(), B, shape[-2], shape[-1], FMT[qdt], qr.data_ptr(), sr.data_ptr(),
                                  stream()) == 0
        torch.cuda.synchronize()
        assert_bytes_equal(u8(q), u8(qr), "fp8 bytes vs reference kernel")
        assert_f32_bitexact(f32(s), f32(sr), "scales vs reference kernel")


@pytest.mark.parametrize("lens", [[100, 0, 300, 128, 5], [0, 0, 64], [1000], [256, 256, 0, 0]])
@pytest.mark.parametrize("qdt", FP8)
def test_segment_vs_oracle_and_reference(lens, qdt):
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_segment_m_row_col_impl

    M, N = sum(lens), 384
    x = _input((max(M, 1), N), seed=7)[:M].contiguous()
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    go = group_offs_from_lens(gl)
    qr, qc, sr, sc, vl, vo = quant_fp8_blockwise_segment_m_row_col_impl(x.cuda(), qdt, 128, gl, go)
    o = O.quant_block_segment(x, FMT[qdt], lens)
    np.testing.assert_array_equal(vl.cpu().numpy(), o[4])
    np.testing.assert_array_equal(vo.cpu().numpy(), o[5])
    P = int(o[5][-1])
    assert_bytes_equal(u8(qr), o[0], "row bytes")
    assert_f32_bitexact(f32(sr), o[2], "row scales (transposed)")
    assert_bytes_equal(u8(qc)[:P], o[1][:P], "padded col bytes")
    assert_f32_bitexact(f32(sc)[: P // 128], o[3][: P // 128], "col scales")
    L = ref_lib()
    if L is not None and M > 0:
        xc = x.cuda().contiguous()
        G = len(lens)
        qr2, qc2 = torch.empty_like(qr), torch.zeros_like(qc)
        sr2, sc2 = torch.empty_like(sr), torch.zeros_like(sc)
        vl2, vo2 = torch.empty_like(vl), torch.empty_like(vo)
        assert L.ref_quant_segment(xc.data_ptr(), M, N, G, gl.data_ptr(), go.data_ptr(), FMT[qdt], qr2.data_ptr(),
                                   qc2.data_ptr(), sr2.data_ptr(), sc2.data_ptr(), vl2.data_ptr(), vo2.data_ptr(),
                                   stream()) == 0
        torch.cuda.synchronize()
        assert_bytes_equal(u8(qr), u8(qr2), "row bytes vs reference kernel")
        assert_f32_bitexact(f32(sr), f32(sr2), "row scales vs reference kernel")
        assert_bytes_equal(u8(qc)[:P], u8(qc2)[:P], "col bytes vs reference kernel")
        assert_f32_bitexact(f32(sc)[: P // 128], f32(sc2)[: P // 128], "col scales vs reference kernel")


@pytest.mark.parametrize("lens", [[100, 0, 300, 128, 5], [0, 0, 64], [1000]])
@pytest.mark.parametrize("N", [384, 200])
def test_segment_col_transposed_vs_oracle(lens, N):
    """The transposed column copy [N, roundup(M,128) + 128 G] holds the padded
    column layout's rows as columns (the wgrad operand layout)."""
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quant_fp8_blockwise_segment_m_row_col_impl

    qdt = torch.float8_e4m3fn
    M = sum(lens)
    x = _input((max(M, 1), N), seed=11)[:M].contiguous()
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    go = group_offs_from_lens(gl)
    qr, qcT, sr, sc, vl, vo = quant_fp8_blockwise_segment_m_row_col_impl(x.cuda(), qdt, 128, gl, go,
                                                                         col_transposed=True)
    o = O.quant_block_segment(x, FMT[qdt], lens)
    P = int(o[5][-1])
    assert tuple(qcT.shape) == (N, (M + 127) // 128 * 128 + 128 * len(lens))
    np.testing.assert_array_equal(vo.cpu().numpy(), o[5])
    assert_bytes_equal(u8(qr), o[0], "row bytes")
    assert_f32_bitexact(f32(sr), o[2], "row scales (transposed)")
    assert_bytes_equal(u8(qcT)[:, :P], np.ascontiguousarray(o[1][:P].T), "transposed col bytes")
    assert_f32_bitexact(f32(sc)[: P // 128], o[3][: P // 128], "col scales")


# ---------------------------------------------------------------------------
# MXFP8 (rule restated from the OCP MX spec; the reference kernel is absent)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(256, 512), (176, 160), (64, 32), (2, 96, 256)])
@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("use_2d", [False, True])
def test_mxfp8_vs_oracle(shape, qdt, use_2d):
    turbo, SG, SR = _turbo()
    g = torch.Generator().manual_seed(8)
    mag = torch.exp(torch.randn(shape, generator=g) * 1.5)
    sign = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0)
    x = (mag * sign).to(torch.bfloat16)
    r = SR(use_2d_block=use_2d)
    nd = len(shape)
    for direction, axis in ((1, nd - 1), (0, nd - 2)):
        q, e = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.MX_BLOCKWISE, block_size=32, axis=axis, scaling_recipe=r)
        qo, eo = O.quant_mx(x, FMT[qdt], direction, use_2d)
        assert e.dtype == torch.float8_e8m0fnu
        assert_bytes_equal(u8(q), qo, f"mx bytes dir={direction}")
        assert_bytes_equal(u8(e), eo, f"e8m0 dir={direction}")
    if nd == 2:
        qr, er, qc, ec = turbo.ops.quantize_fp8_with_trans(x.cuda(), qdt, SG.MX_BLOCKWISE, block_size=32,
                                                          scaling_recipe=r, scaling_recipe_for_trans=r)
        assert_bytes_equal(u8(qr), O.quant_mx(x, FMT[qdt], 1, use_2d)[0], "dual row bytes")
        assert_bytes_equal(u8(qc), O.quant_mx(x, FMT[qdt], 0, use_2d)[0], "dual col bytes")
        # K-block-major exponents: same bytes, stored [cols_pad/128, rows, 4]
        from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_mxfp8_impl

        qrk, erk, qck, eck = quantize_mxfp8_impl(x.cuda(), qdt, None, 32, with_trans=True, scaling_recipe=r,
                                                 scaling_recipe_for_trans=r, exp_kmajor=True)
        assert_bytes_equal(u8(qrk), u8(qr), "dual row bytes (k-major exponents)")
        assert_bytes_equal(u8(qck), u8(qc), "dual col bytes (k-major exponents)")
        for ek, e_ref, what in ((erk, er, "row"), (eck, ec, "col")):
            nb, rows, four = ek.shape
            assert four == 4 and rows == e_ref.shape[0] and nb * 4 == e_ref.shape[1]
            back = u8(ek).transpose(1, 0, 2).reshape(rows, nb * 4)
            assert_bytes_equal(back, u8(e_ref), f"k-major {what} exponents")


@pytest.mark.parametrize("B", [1, 4])
@pytest.mark.parametrize("M,N", [(32, 32), (64, 256), (256, 1024), (1024, 64), (176, 160)])
@pytest.mark.parametrize("use_2d", [False, True])
def test_mxfp8_scale_shuffle(B, M, N, use_2d):
    """shuffle_scale recipes give the 16 x 16 shuffle of the plain exponents
    (the reference's test_quantize_mxfp8_shuffle); the shuffle matches the
    oracle and, where it builds, the reference's own shuffle kernel."""
    turbo, SG, SR = _turbo()
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_mxfp8_impl, shuffle_scale_impl

    g = torch.Generator().manual_seed(21)
    x = torch.randn((B, M, N), generator=g).to(torch.bfloat16).cuda()
    x2 = x.view(-1, N)
    r = SR(use_2d_block=use_2d)
    rs = SR(use_2d_block=use_2d, shuffle_scale=True)
    _, er, _, ec = turbo.ops.quantize_fp8_with_trans(x2, torch.float8_e4m3fn, SG.MX_BLOCKWISE, block_size=32,
                                                    scaling_recipe=r, scaling_recipe_for_trans=r)
    _, ers, _, ecs = turbo.ops.quantize_fp8_with_trans(x2, torch.float8_e4m3fn, SG.MX_BLOCKWISE, block_size=32,
                                                      scaling_recipe=rs, scaling_recipe_for_trans=rs)
    L = ref_lib()
    for plain, shuffled, what in ((er, ers, "row"), (ec, ecs, "col")):
        mine = shuffle_scale_impl(plain, [16, 16])
        assert_bytes_equal(u8(shuffled), u8(mine), f"quantize shuffle_scale {what}")
        assert_bytes_equal(u8(mine), O.shuffle_e8m0(u8(plain)), f"shuffle vs oracle {what}")
        if L is not None and L.ref_shuffle_e8m0 is not None:
            ref = torch.empty_like(mine).view(torch.uint8)
            pl = plain.contiguous().view(torch.uint8)
            assert L.ref_shuffle_e8m0(pl.data_ptr(), pl.shape[0], pl.shape[1], ref.data_ptr(), stream()) == 0
            torch.cuda.synchronize()
            assert_bytes_equal(u8(mine), u8(ref), f"shuffle vs reference kernel {what}")
    # 3-D input: one padded block per batch
    q3, e3 = quantize_mxfp8_impl(x, torch.float8_e4m3fn, 2, 32, scaling_recipe=rs)
    _, e3p = quantize_mxfp8_impl(x, torch.float8_e4m3fn, 2, 32, scaling_recipe=r)
    assert e3.shape[0] == B
    for b in range(B):
        assert_bytes_equal(u8(e3[b]), O.shuffle_e8m0(u8(e3p[b])), f"batched shuffle {b}")


# ---------------------------------------------------------------------------
# dequantization
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_dequant_vs_oracle(qdt, out):
    turbo, SG, SR = _turbo()
    x = _input((300, 260), seed=9)
    xc = x.cuda()
    # tensorwise
    q, s = turbo.ops.quantize_fp8(xc, qdt, SG.TENSORWISE)
    y = turbo.ops.dequantize_fp8(q, out, SG.TENSORWISE, scale_inv=s)
    ref = O.dequant_tensorwise(u8(q), FMT[qdt], f32(s))
    np.testing.assert_array_equal(f32(y), torch.from_numpy(ref).float().to(out).float().numpy())
    # blockwise 1-D both axes and 2-D
    for axis in (0, 1):
        q, s = turbo.ops.quantize_fp8(xc, qdt, SG.BLOCKWISE, block_size=128, axis=axis)
        y = turbo.ops.dequantize_fp8(q, out, SG.BLOCKWISE, block_size=128, axis=axis, scale_inv=s)
        ref = O.dequant_block1d(u8(q), FMT[qdt], f32(s), axis)
        np.testing.assert_array_equal(f32(y), torch.from_numpy(ref).float().to(out).float().numpy())
    r = SR(use_2d_block=True)
    q, s = turbo.ops.quantize_fp8(xc, qdt, SG.BLOCKWISE, block_size=128, scaling_recipe=r)
    y = turbo.ops.dequantize_fp8(q, out, SG.BLOCKWISE, block_size=128, scale_inv=s, scaling_recipe=r)
    ref = O.dequant_block2d(u8(q), FMT[qdt], f32(s))
    np.testing.assert_array_equal(f32(y), torch.from_numpy(ref).float().to(out).float().numpy())
    # rowwise
    q, s = turbo.ops.quantize_fp8(xc, qdt, SG.ROWWISE, axis=-1)
    y = turbo.ops.dequantize_fp8(q, out, SG.ROWWISE, axis=-1, scale_inv=s)
    ref = O.dequant_rowwise(u8(q), FMT[qdt], f32(s))
    np.testing.assert_array_equal(f32(y), torch.from_numpy(ref).float().to(out).float().numpy())


def test_reference_roundtrip_tolerance():
    """The reference's own quantize->dequantize criterion (tests/pytorch/ops/
    test_quantization.py with tests/pytorch/test_utils.py:17-31: rtol = atol = 0.1)."""
    turbo, SG, SR = _turbo()
    x = randn((512, 1024), seed=10).cuda()
    for g, kw in ((SG.TENSORWISE, {}), (SG.ROWWISE, {"axis": -1}), (SG.BLOCKWISE, {"block_size": 128, "axis": 1})):
        q, s = turbo.ops.quantize_fp8(x, torch.float8_e4m3fn, g, **kw)
        y = turbo.ops.dequantize_fp8(q, torch.bfloat16, g, scale_inv=s, **kw)
        torch.testing.assert_close(y, x, rtol=0.1, atol=0.1)


def _fp8_bytes_no_nan(shape, fmt, seed):
    """Random fp8 bytes covering every finite encoding (NaN / Inf codes
    replaced by zero)."""
    g = torch.Generator().manual_seed(seed)
    b = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    bad = (b & 0x7F) == 0x7F if fmt == 0 else (b & 0x7C) == 0x7C
    b[bad] = 0
    return b


def _equal_or_both_nan(got, exp, what):
    g, e = got.float().cpu(), exp.float().cpu()
    both_nan = torch.isnan(g) & torch.isnan(e)
    same = (g.view(torch.int32) == e.view(torch.int32)) | both_nan
    assert bool(same.all()), f"{what}: {int((~same).sum())} mismatches"


@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("rowwise", [True, False])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("RC", [(64, 256), (300, 128), (1024, 1024), (7, 32)])
def test_mx_dequant_vs_reference_kernel(qdt, rowwise, out, RC):
    """MX dequantize against the reference's own kernel
    (csrc/kernels/quantization/dequantization_mxfp8.cu, built into
    oracle/_ref) on every finite fp8 byte and every E8M0 exponent 0..255:
    the e = 0 -> 0.0 and e = 255 -> +Inf decode (utils.cuh:117-120) included.
    Output bits equal (NaN, from 0 x Inf, matched as NaN)."""
    from primus_turbo.pytorch import _C

    L = ref_lib()
    if L is None or L.ref_dequant_mxfp8 is None:
        pytest.skip("oracle/_ref not built")
    R, C = RC
    fmt = FMT[qdt]
    q = _fp8_bytes_no_nan((R, C), fmt, seed=R + C).cuda()
    e = (torch.arange(R * (C // 32), dtype=torch.int64) % 256).to(torch.uint8).view(R, C // 32)
    e = e[torch.randperm(R, generator=torch.Generator().manual_seed(3))].contiguous().cuda()
    shape = (R, C) if rowwise else (C, R)
    y = torch.empty(shape, dtype=out, device="cuda")
    yr = torch.empty(shape, dtype=out, device="cuda")
    oc = _C.PTA_BF16 if out == torch.bfloat16 else _C.PTA_F32
    _C.call("pta_dequantize_mxfp8", q.data_ptr(), fmt, R, C, e.data_ptr(), 0 if rowwise else 1, y.data_ptr(), oc,
            stream())
    assert L.ref_dequant_mxfp8(q.data_ptr(), fmt, R, C, e.data_ptr(), R, C // 32, 1 if rowwise else 0,
                               yr.data_ptr(), 2 if out == torch.bfloat16 else 0, stream()) == 0
    torch.cuda.synchronize()
    _equal_or_both_nan(y, yr, "mx dequant vs reference kernel")


@pytest.mark.parametrize("BMN", [(1, 128, 256), (1, 4096, 7168), (3, 77, 1000), (2, 1, 33), (1, 1000, 1)])
def test_transpose_u8_vs_reference_kernel(BMN):
    """The fp8 byte transpose against the reference's transpose_2d kernel
    (csrc/kernels/transpose/transpose_2d.cu, built into oracle/_ref)."""
    from primus_turbo.pytorch import _C

    L = ref_lib()
    if L is None or L.ref_transpose_2d is None:
        pytest.skip("oracle/_ref not built")
    B, M, N = BMN
    x = torch.randint(0, 256, (B, M, N), generator=torch.Generator().manual_seed(9), dtype=torch.int32)
    x = x.to(torch.uint8).cuda()
    y = torch.empty((B, N, M), dtype=torch.uint8, device="cuda")
    yr = torch.empty_like(y)
    _C.call("pta_transpose_u8", x.data_ptr(), B, M, N, y.data_ptr(), stream())
    assert L.ref_transpose_2d(x.data_ptr(), yr.data_ptr(), B, M, N, 1, stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, yr)
    assert torch.equal(y.cpu(), x.cpu().transpose(1, 2))


def _mx_padded_ref(x, axis, align=128):
    """Zero-padded input in the layout MX dequantize returns (the reference's
    mxfp8_padded_ref, tests/pytorch/ops/test_quantization.py:252-275)."""
    pad = lambda n: (align - n % align) % align  # noqa: E731
    if x.dim() == 2:
        if axis == 0:
            return torch.cat([x, torch.zeros(pad(x.size(0)), x.size(1), dtype=x.dtype, device=x.device)], 0)
        return torch.cat([x, torch.zeros(x.size(0), pad(x.size(1)), dtype=x.dtype, device=x.device)], 1)
    if axis == 1:
        xt = x.transpose(1, 2).contiguous()
        return torch.cat([xt, torch.zeros(xt.size(0), xt.size(1), pad(xt.size(2)), dtype=x.dtype, device=x.device)], 2)
    return torch.cat([x, torch.zeros(x.size(0), x.size(1), pad(x.size(2)), dtype=x.dtype, device=x.device)], 2)


@pytest.mark.parametrize("orig_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dest_dtype", FP8)
@pytest.mark.parametrize("batched", [False, True])
@pytest.mark.parametrize("B", [1, 4])
@pytest.mark.parametrize("M", [32, 64, 256, 1024])
@pytest.mark.parametrize("N", [32, 64, 256, 1024])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("use_2d_block", [True, False])
def test_reference_mx_roundtrip(orig_dtype, dest_dtype, batched, B, M, N, axis, use_2d_block):
    """The reference's MXFP8 criterion, with its grid unchanged
    (tests/pytorch/ops/test_quantization.py:304-359): quantize along `axis`,
    dequantize, and compare the zero-padded input with the result at the fp8
    tolerance of tests/pytorch/test_utils.py:17-31 (rtol = atol = 0.1,
    measured against the dequantized value)."""
    turbo, SG, SR = _turbo()
    torch.manual_seed(42)
    x = torch.randn((B, M, N) if batched else (M, N), device="cuda", dtype=orig_dtype)
    qaxis = axis + 1 if batched else axis
    rec = SR(use_2d_block=use_2d_block)
    q, s = turbo.ops.quantize_fp8(x, dest_dtype, SG.MX_BLOCKWISE, axis=qaxis, block_size=32, scaling_recipe=rec)
    y = turbo.ops.dequantize_fp8(q, orig_dtype, SG.MX_BLOCKWISE, block_size=32, axis=qaxis, scale_inv=s,
                                 scaling_recipe=rec)
    torch.testing.assert_close(_mx_padded_ref(x, qaxis), y, rtol=0.1, atol=0.1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("qdt", FP8)
@pytest.mark.parametrize("shape,spike_pos", [((1, 100), -1), ((1, 8193), -1), ((512, 3072), 8300), ((512, 3072), -1),
                                             ((1024, 4096), -1)])
def test_tensorwise_spike_amax(dtype, qdt, shape, spike_pos):
    """The reference's partial-tile amax regression case (test_quantization.py:
    66-95): one spike of 100 in a field of 0.5 sets the scale, bit for bit
    against the oracle."""
    turbo, SG, _ = _turbo()
    x = torch.full(shape, 0.5, dtype=dtype)
    x.view(-1)[spike_pos] = 100.0
    q, s = turbo.ops.quantize_fp8(x.cuda(), qdt, SG.TENSORWISE)
    qo, so = O.quant_tensorwise(x, FMT[qdt])
    assert_f32_bitexact(f32(s), so, "scale_inv")
    assert_bytes_equal(u8(q), qo, "fp8 bytes")


@pytest.mark.parametrize("orig_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dest_dtype", FP8)
@pytest.mark.parametrize("B", [1, 4])
@pytest.mark.parametrize("M", [32, 64, 256, 1024])
@pytest.mark.parametrize("N", [32, 64, 256, 1024])
@pytest.mark.parametrize("use_2d_block", [True, False])
def test_reference_mx_with_trans_roundtrip(orig_dtype, dest_dtype, B, M, N, use_2d_block):
    """The reference's dual MXFP8 criterion, with its grid unchanged
    (tests/pytorch/ops/test_quantization.py:362-460): the rowwise copy
    dequantizes to [B*M, N_pad] and the transposed copy (axis 0) to
    [M_pad, N], each equal to the zero-padded input at rtol = atol = 0.1.
    No element is exempt: the shared exponent is bumped wherever the block
    maximum would saturate, so nothing is clamped."""
    turbo, SG, SR = _turbo()
    torch.manual_seed(42)
    x = torch.randn((B, M, N), device="cuda", dtype=orig_dtype).view(-1, N)
    rec = SR(use_2d_block=use_2d_block)
    qr, sr, qt, st = turbo.ops.quantize_fp8_with_trans(x, dest_dtype, SG.MX_BLOCKWISE, block_size=32,
                                                       scaling_recipe=rec, scaling_recipe_for_trans=rec)
    yr = turbo.ops.dequantize_fp8(qr, orig_dtype, SG.MX_BLOCKWISE, block_size=32, axis=1, scale_inv=sr,
                                  scaling_recipe=rec)
    yc = turbo.ops.dequantize_fp8(qt, orig_dtype, SG.MX_BLOCKWISE, block_size=32, axis=0, scale_inv=st,
                                  scaling_recipe=rec)
    torch.testing.assert_close(_mx_padded_ref(x, 1), yr, rtol=0.1, atol=0.1)
    torch.testing.assert_close(_mx_padded_ref(x, 0), yc, rtol=0.1, atol=0.1)


@pytest.mark.parametrize("BMN", [(4, 111, 1), (1, 1, 4096), (4, 7168, 111), (1, 111, 4096)])
@pytest.mark.parametrize("axis", [-1, -2, -3, 0, 1, 2])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rowwise_reference_axes_vs_oracle(BMN, axis, dtype):
    """The reference's rowwise parametrization (test_quantization.py:98-140:
    every axis of a [B, M, N] input, sizes 1 / 111 / 4096 / 7168), held to
    bit-exact bytes and scales against the oracle instead of a tolerance."""
    turbo, SG, _ = _turbo()
    x = _input(BMN, dtype, seed=12, special=False)
    q, s = turbo.ops.quantize_fp8(x.cuda(), torch.float8_e4m3fn, SG.ROWWISE, axis=axis)
    qo, so = O.quant_rowwise(x, FMT[torch.float8_e4m3fn], axis)
    assert tuple(s.shape) == so.shape
    assert_bytes_equal(u8(q), qo, "fp8 bytes")
    assert_f32_bitexact(f32(s), so, "scale_inv")
