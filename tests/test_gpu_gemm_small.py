"""The 64 x 64-tile GEMM path (problems with few 256 x 256 tiles) against the
256 x 256-tile kernel, bit for bit.

Both kernels feed the same K permutation of each 128-deep block to the same
MFMA, in the same K-block order, and scale in the same order, so every output
must be identical.  ``gemm_fp8_impl`` takes the small-tile path for these
shapes (reading K-major operands in place); the reference output comes from
``gemm_fp8_nt`` (always the large-tile kernel) on operands transposed to NT in
torch.  Operands are random fp8 bytes (NaN / Inf patterns replaced) with random
scales, so every bit of the inputs takes part.  The oracle-based parity of the
same path is in test_gpu_gemm.py, whose small shapes take this path too."""

import pytest
import torch

pytestmark = pytest.mark.gpu

E4, E5 = torch.float8_e4m3fn, torch.float8_e5m2


def _fp8(shape, dt, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
    if dt == E4:
        bad = (x & 0x7F) == 0x7F
    else:
        bad = ((x >> 2) & 0x1F) == 0x1F
    x[bad] = 0x38
    return x.view(dt).cuda()


def _scales(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(shape, generator=g) * 1.5 + 0.5).float().cuda()


def _exps(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(118, 134, shape, generator=g, dtype=torch.uint8).cuda()


def _cd(a, b):
    return -(-a // b)


def _case(M, N, K, layout, trans_c, gran_name, fa=E4, fb=E4, out_dtype=torch.bfloat16):
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_impl, gemm_fp8_nt

    g = getattr(SG, gran_name)
    ta, tb = layout[0] == "T", layout[1] == "T"
    qa = _fp8((K, M) if ta else (M, K), fa, 1)
    qb = _fp8((N, K) if tb else (K, N), fb, 2)
    a_nt = qa.t().contiguous() if ta else qa
    b_nt = qb if tb else qb.t().contiguous()
    kb = _cd(K, 128)
    if g == SG.TENSORWISE:
        sa, sb = _scales((1,), 3), _scales((1,), 4)
        nt = dict(a_scale=sa, b_scale=sb)
    elif g == SG.ROWWISE:
        sa, sb = _scales((M,), 3), _scales((N,), 4)
        nt = dict(a_scale=sa, b_scale=sb)
    elif g == SG.BLOCKWISE:
        # scale layouts of the reference's wrapper for each layout
        if not ta:
            sa = _scales((M, kb), 3)
            sa_nt = (sa, (kb, 1), False)
        else:
            sa = _scales((kb, M), 3)
            sa_nt = (sa, (1, M), False)
        if tb:
            sb = _scales((_cd(N, 128), kb), 4)
            sb_nt = (sb, (kb, 1), True)
        elif not ta:
            sb = _scales((kb, _cd(N, 128)), 4)
            sb_nt = (sb, (1, _cd(N, 128)), True)
        else:
            sb = _scales((kb, N), 4)
            sb_nt = (sb, (1, N), False)
        nt = dict(a_scale=sa_nt[0], sa_strides=sa_nt[1], a_scale_2d=sa_nt[2],
                  b_scale=sb_nt[0], sb_strides=sb_nt[1], b_scale_2d=sb_nt[2])
    else:
        sa, sb = _exps((M, K // 32), 3), _exps((N, K // 32), 4)
        nt = dict(a_scale=sa, sa_strides=(K // 32, 4), b_scale=sb, sb_strides=(K // 32, 4))
    out = gemm_fp8_impl(qa, sa, ta, qb, sb, tb, out_dtype, trans_c, g.value)
    if not trans_c:
        ref = gemm_fp8_nt(a_nt, b_nt, out_dtype, g, **nt, large_tiles_only=True)
    else:  # C^T = B' A'^T: exchange the operands and their scale addressing
        other = {"a_scale": "b_scale", "sa_strides": "sb_strides", "a_scale_2d": "b_scale_2d"}
        other.update({v: k for k, v in other.items()})
        sw = {other[k]: v for k, v in nt.items()}
        ref = gemm_fp8_nt(b_nt, a_nt, out_dtype, g, **sw, large_tiles_only=True)
    torch.cuda.synchronize()
    assert out.shape == ref.shape
    diff = (out.view(torch.int16 if out.element_size() == 2 else torch.int32)
            != ref.view(torch.int16 if ref.element_size() == 2 else torch.int32))
    assert not bool(diff.any()), f"{int(diff.sum())} of {diff.numel()} outputs differ, first at {diff.nonzero()[0].tolist()}"


# 32 x 64 tiles for the first six, 64 x 64 for (1024, 1024) and (1000, 1040),
# 128 x 128 for (1904, 2000) (ragged in both dimensions)
SHAPES = [(512, 1024, 1024), (255, 512, 576), (64, 128, 128), (200, 136, 1040), (8, 24, 16), (1000, 520, 2048),
          (1024, 1024, 256), (1000, 1040, 384), (1904, 2000, 256)]


@pytest.mark.parametrize("mnk", SHAPES)
@pytest.mark.parametrize("layout", ["NT", "NN", "TN"])
@pytest.mark.parametrize("trans_c", [False, True])
@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE"])
def test_small_path_matches_large_tile_kernel(mnk, layout, trans_c, gran):
    M, N, K = mnk
    if layout == "TN" and M % 8:
        pytest.skip("K-major A with M % 8 != 0 takes the transpose path")
    _case(M, N, K, layout, trans_c, gran)


@pytest.mark.parametrize("mnk", [(512, 1024, 1024), (255, 512, 640), (64, 128, 128), (200, 136, 1024),
                                 (1000, 1040, 512), (1904, 2000, 256)])
@pytest.mark.parametrize("trans_c", [False, True])
def test_small_path_mx_matches_large_tile_kernel(mnk, trans_c):
    M, N, K = mnk
    _case(M, N, K, "NT", trans_c, "MX_BLOCKWISE")


@pytest.mark.parametrize("fmts", [(E4, E5), (E5, E4), (E5, E5)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("gran", ["TENSORWISE", "BLOCKWISE", "MX_BLOCKWISE"])
@pytest.mark.parametrize("mnk", [(320, 200, 384), (1904, 2000, 256)])
def test_small_path_formats_and_outputs(fmts, out_dtype, gran, mnk):
    layout = "NT" if gran == "MX_BLOCKWISE" else "NN"
    _case(*mnk, layout, False, gran, fmts[0], fmts[1], out_dtype)


def _strided_args(M, N, K, scales, seed):
    """Operands as row-strided views (row stride K + 64) with scales in one of
    the layouts the autograd functions hand to gemm_fp8_nt."""
    from primus_turbo.pytorch.core.low_precision import ScalingGranularity as SG

    qa = _fp8((M, K + 64), E4, seed)[:, :K]
    qb = _fp8((N, K + 64), E4, seed + 1)[:, :K]
    kb = _cd(K, 128)
    if scales == "TENSORWISE":
        return qa, qb, SG.TENSORWISE, dict(a_scale=_scales((1,), seed + 2), b_scale=_scales((1,), seed + 3))
    if scales == "ROWWISE":
        return qa, qb, SG.ROWWISE, dict(a_scale=_scales((M,), seed + 2), b_scale=_scales((N,), seed + 3))
    if scales == "BLOCK_1Dx2D":  # forward: A [M, K/128], B [N/128, K/128]
        return qa, qb, SG.BLOCKWISE, dict(a_scale=_scales((M, kb), seed + 2), sa_strides=(kb, 1),
                                          b_scale=_scales((_cd(N, 128), kb), seed + 3), sb_strides=(kb, 1),
                                          b_scale_2d=True)
    if scales == "BLOCK_1Dx1D":  # wgrad: both K-block major [K/128, rows]
        return qa, qb, SG.BLOCKWISE, dict(a_scale=_scales((kb, M), seed + 2), sa_strides=(1, M),
                                          b_scale=_scales((kb, N), seed + 3), sb_strides=(1, N))
    if scales == "MX_ROWMAJOR":  # [rows, K/32] bytes
        return qa, qb, SG.MX_BLOCKWISE, dict(a_scale=_exps((M, K // 32), seed + 2), sa_strides=(K // 32, 4),
                                             b_scale=_exps((N, K // 32), seed + 3), sb_strides=(K // 32, 4))
    # MX_KMAJOR: [K/128, rows, 4] bytes
    return qa, qb, SG.MX_BLOCKWISE, dict(a_scale=_exps((K // 128, M, 4), seed + 2), sa_strides=(4, 4 * M),
                                         b_scale=_exps((K // 128, N, 4), seed + 3), sb_strides=(4, 4 * N))


@pytest.mark.parametrize("scales", ["TENSORWISE", "ROWWISE", "BLOCK_1Dx2D", "BLOCK_1Dx1D", "MX_ROWMAJOR", "MX_KMAJOR"])
@pytest.mark.parametrize("mnk", [(512, 1024, 1024), (200, 136, 1024), (1904, 2000, 256)])
def test_strided_entry_small_kernel_matches_large(scales, mnk):
    """gemm_fp8_nt (the autograd functions' NT entry) takes the small-tile kernel
    for few 256 x 256 tiles (blockwise ones it would run on 128 x 128 tiles
    excepted): row-strided operands, a row-strided output and each scale
    layout give the same bits as the 256 x 256 kernel."""
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt

    M, N, K = mnk
    qa, qb, g, nt = _strided_args(M, N, K, scales, 40)
    wide = torch.zeros((M, N + 24), dtype=torch.bfloat16, device="cuda")
    out = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt, out=wide[:, :N])
    ref = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt, large_tiles_only=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"{int((out != ref).sum())} outputs differ"
    assert not wide[:, N:].float().any(), "columns past N of the output rows were written"


@pytest.mark.parametrize("scales", ["TENSORWISE", "BLOCK_1Dx2D", "BLOCK_1Dx1D", "MX_KMAJOR"])
def test_strided_entry_k_split(scales):
    """108 tiles of 256 x 256 with K = 4096: gemm_fp8_nt runs the K split
    through its workspace; the result matches the unsplit kernel to within fp32
    summation order and repeats bit for bit."""
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt

    M, N, K = 2300, 3000, 4096
    qa, qb, g, nt = _strided_args(M, N, K, scales, 50)
    out = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt)
    again = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt)
    ref = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt, large_tiles_only=True)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "split GEMM is not deterministic"
    o, r = out.double(), ref.double()
    assert torch.isfinite(o).all()
    assert float((o - r).abs().max()) <= 2.0 ** -6 * float(r.abs().max()), "split and whole results differ beyond rounding"
