"""GPU parity of the FP8 GEMMs against the fp64 oracle on the same quantized
operands.  Tolerance (bf16 / fp16 output): SNR >= 40 dB and
max|out - ref| / max|ref| <= 1e-2, where ref is the exact product of the
dequantized operands.  The reference's own end-to-end criterion (SNR vs an
unquantized matmul > 25 dB e4m3, > 20 dB e5m2, tests/pytorch/ops/
test_gemm_fp8.py:101-114) is checked on the autograd path."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import FMT, f32, randn, u8

pytestmark = pytest.mark.gpu

SNR_MIN = 40.0
REL_MAX = 1e-2


def _mods():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import (
        Float8QuantConfig,
        Format,
        ScaleDtype,
        ScalingGranularity,
        ScalingRecipe,
    )
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_impl

    return turbo, Float8QuantConfig, Format, ScaleDtype, ScalingGranularity, ScalingRecipe, gemm_fp8_impl


def _check(out, ref, what):
    o = f32(out).astype(np.float64)
    snr = O.snr_db(ref, o)
    rel = O.max_rel_err(ref, o)
    assert snr >= SNR_MIN and rel <= REL_MAX, f"{what}: SNR {snr:.1f} dB, max rel err {rel:.2e}"
    return snr, rel


@pytest.mark.parametrize("mnk", [(512, 1024, 1024), (255, 512, 576), (1024, 768, 2048), (64, 128, 128), (2304, 4096, 256)])
@pytest.mark.parametrize("layout", ["NT", "NN", "TN"])
@pytest.mark.parametrize("trans_c", [False, True])
@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE"])
def test_gemm_tensor_row_vs_oracle(mnk, layout, trans_c, gran):
    turbo, _, _, _, SG, _, gemm_fp8_impl = _mods()
    g = getattr(SG, gran)
    M, N, K = mnk
    ta, tb = layout[0] == "T", layout[1] == "T"
    if K % 16 and (ta or not tb):
        pytest.skip("odd K exercised through the autograd path")
    a = randn((K, M) if ta else (M, K), seed=1).cuda()
    b = randn((N, K) if tb else (K, N), seed=2).cuda()
    qdt = torch.float8_e4m3fn
    if g == SG.TENSORWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g)
        da = O.dequant_tensorwise(u8(qa), 0, f32(sa))
        db = O.dequant_tensorwise(u8(qb), 0, f32(sb))
    else:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, axis=0 if ta else -1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, axis=-1 if tb else 0)
        da = O.dequant_rowwise(u8(qa), 0, f32(sa))
        db = O.dequant_rowwise(u8(qb), 0, f32(sb))
    out = gemm_fp8_impl(qa, sa, ta, qb, sb, tb, torch.bfloat16, trans_c, g.value)
    ref = O.gemm_ref(da, db, ta, tb, trans_c)
    assert tuple(out.shape) == ref.shape
    _check(out, ref, f"{gran} {layout} trans_c={trans_c}")


@pytest.mark.parametrize("mnk", [(512, 1024, 1024), (256, 384, 512), (4096, 2048, 7168), (300, 256, 384)])
@pytest.mark.parametrize("layout", ["NT", "NN", "TN"])
@pytest.mark.parametrize("qdt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_gemm_blockwise_vs_oracle(mnk, layout, qdt):
    """Blockwise scale layouts of the reference's Triton wrapper (gemm_fp8_kernel.py:1013-1154)."""
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    g = SG.BLOCKWISE
    M, N, K = mnk
    f = FMT[qdt]
    if layout == "NT":
        a = randn((M, K), seed=3, outliers=0.001).cuda()
        w = randn((N, K), seed=4, outliers=0.001).cuda()
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=1)
        qw, sw = turbo.ops.quantize_fp8(w, qdt, g, block_size=128, scaling_recipe=SR(use_2d_block=True))
        da = O.dequant_block1d(u8(qa), f, f32(sa), 1)
        dw = O.dequant_block2d(u8(qw), f, f32(sw))
        out = gemm_fp8_impl(qa, sa, False, qw, sw, True, torch.bfloat16, False, g.value)
        ref = O.gemm_ref(da, dw, False, True)
    elif layout == "NN":  # dgrad: A = grad [M, K], B = weight [K, N] stored as the forward weight [K, N]
        a = randn((M, K), seed=5).cuda()
        w = randn((K, N), seed=6).cuda()
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=1)
        qw, sw = turbo.ops.quantize_fp8(w, qdt, g, block_size=128, scaling_recipe=SR(use_2d_block=True))
        da = O.dequant_block1d(u8(qa), f, f32(sa), 1)
        dw = O.dequant_block2d(u8(qw), f, f32(sw))
        out = gemm_fp8_impl(qa, sa, False, qw, sw, False, torch.bfloat16, False, g.value)
        ref = O.gemm_ref(da, dw, False, False)
    else:  # TN (wgrad): A [K, M] col scales [K/128, M], B [K, N] col scales [K/128, N], output trans_c
        a = randn((K, M), seed=7).cuda()
        b = randn((K, N), seed=8).cuda()
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=0)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=128, axis=0)
        da = O.dequant_block1d(u8(qa), f, f32(sa), 0)
        db = O.dequant_block1d(u8(qb), f, f32(sb), 0)
        out = gemm_fp8_impl(qa, sa, True, qb, sb, False, torch.bfloat16, True, g.value)
        ref = O.gemm_ref(da, db, True, False, True)
    assert tuple(out.shape) == ref.shape
    _check(out, ref, f"BLOCKWISE {layout}")


@pytest.mark.parametrize("mnk", [(2304, 3072, 4096), (2300, 3000, 4096), (4096, 2048, 7168), (2048, 4352, 4224), (1024, 4096, 4096), (1000, 4000, 3072)])
@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
def test_gemm_k_split_vs_oracle(mnk, gran):
    """Problems of 48-128 tiles of 256 x 256 with K >= 4096, or up to 64 tiles
    with K >= 3072 (blockwise; the others take the small-tile kernel there),
    K-contiguous operands, an odd count of K blocks included, run every tile as two half-K
    workgroups (fp32 partials handed over through the workspace), including
    partial edge tiles: the result meets the oracle criterion and
    matches the unsplit strided entry (same operands) to within fp32 summation
    order, and a repeated call gives the same bits."""
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt
    from primus_turbo.pytorch.ops.gemm_fp8 import _mx_strides

    g = getattr(SG, gran)
    M, N, K = mnk
    qdt = torch.float8_e4m3fn
    a = randn((M, K), seed=21, outliers=0.001).cuda()
    b = randn((N, K), seed=22, outliers=0.001).cuda()
    kb = (K + 127) // 128
    if g == SG.TENSORWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g)
        da, db = O.dequant_tensorwise(u8(qa), 0, f32(sa)), O.dequant_tensorwise(u8(qb), 0, f32(sb))
        nt = dict(a_scale=sa, b_scale=sb)
    elif g == SG.ROWWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, axis=-1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, axis=-1)
        da, db = O.dequant_rowwise(u8(qa), 0, f32(sa)), O.dequant_rowwise(u8(qb), 0, f32(sb))
        nt = dict(a_scale=sa, b_scale=sb)
    elif g == SG.BLOCKWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=128, scaling_recipe=SR(use_2d_block=True))
        da, db = O.dequant_block1d(u8(qa), 0, f32(sa), 1), O.dequant_block2d(u8(qb), 0, f32(sb))
        nt = dict(a_scale=sa, sa_strides=(kb, 1), b_scale=sb, sb_strides=(kb, 1), b_scale_2d=True)
    else:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=32, axis=1, scaling_recipe=SR())
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=32, axis=1, scaling_recipe=SR(use_2d_block=True))
        da, db = O.dequant_mx(u8(qa), 0, u8(sa)), O.dequant_mx(u8(qb), 0, u8(sb))
        nt = dict(a_scale=sa, sa_strides=_mx_strides(sa), b_scale=sb, sb_strides=_mx_strides(sb))
    out = gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, g.value)
    again = gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, g.value)
    whole = gemm_fp8_nt(qa, qb, torch.bfloat16, g, **nt, large_tiles_only=True)[:, :N]
    ref = O.gemm_ref(da, db, False, True)
    _check(out, ref, f"{gran} split")
    assert torch.equal(out, again), "split GEMM is not deterministic"
    o, w = f32(out).astype(np.float64), f32(whole).astype(np.float64)
    assert np.max(np.abs(o - w)) <= 2.0 ** -6 * np.max(np.abs(w)), "split and whole results differ beyond rounding"


def test_gemm_k_split_workspace_reuse():
    """One workspace for consecutive K-split calls on different activations,
    enqueued back to back: each call's tag keeps its second halves from
    adding a partial tile an earlier call left in the workspace, so every
    output matches the unsplit kernel on its own operands."""
    turbo, _, _, _, SG, _, _ = _mods()
    from primus_turbo.pytorch import _C
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt

    g = SG.TENSORWISE
    M, N, K = 1024, 4096, 4096  # 64 tiles, K >= 4096: split
    ws_n = _C.query("pta_gemm_fp8_workspace_size", M, N, K, 0, 1, g.value)
    assert ws_n >= 64 * 256 * 256 * 4
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    b = randn((N, K), seed=40).cuda()
    qb, sb = turbo.ops.quantize_fp8(b, torch.float8_e4m3fn, g)
    calls = []
    for seed, amp in ((41, 30.0), (42, 0.01), (43, 1.0)):
        a = (randn((M, K), seed=seed).float() * amp).bfloat16().cuda()
        qa, sa = turbo.ops.quantize_fp8(a, torch.float8_e4m3fn, g)
        calls.append((qa, sa, torch.empty((M, N), dtype=torch.bfloat16, device="cuda")))
    for qa, sa, out in calls:
        _C.call("pta_gemm_fp8", _C.ptr(qa), _C.PTA_E4M3, _C.ptr(sa), 0, _C.ptr(qb), _C.PTA_E4M3, _C.ptr(sb), 1,
                _C.ptr(out), _C.PTA_BF16, 0, M, N, K, g.value, _C.ptr(ws), ws_n, _C.stream(qa.device))
    torch.cuda.synchronize()
    for i, (qa, sa, out) in enumerate(calls):
        whole = gemm_fp8_nt(qa, qb, torch.bfloat16, g, a_scale=sa, b_scale=sb, large_tiles_only=True)
        o, w = out.double(), whole.double()
        assert torch.isfinite(o).all(), f"call {i}: non-finite output"
        assert float((o - w).abs().max()) <= 2.0 ** -6 * float(w.abs().max()), f"call {i} differs from its own product"


@pytest.mark.parametrize("gran", ["TENSORWISE", "BLOCKWISE"])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("trans_c", [False, True])
def test_gemm_k_split_out_dtype_trans_c(gran, out_dtype, trans_c):
    """The K-split finisher writes through the same epilogue as a whole tile:
    fp32 and fp16 outputs and the transposed output (operands exchanged) meet
    the oracle criterion on a 108-tile problem with a partial edge tile."""
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    g = getattr(SG, gran)
    M, N, K = 2300, 3000, 4096
    qdt = torch.float8_e4m3fn
    a = randn((M, K), seed=31, outliers=0.001).cuda()
    b = randn((N, K), seed=32, outliers=0.001).cuda()
    if g == SG.TENSORWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g)
        da, db = O.dequant_tensorwise(u8(qa), 0, f32(sa)), O.dequant_tensorwise(u8(qb), 0, f32(sb))
    else:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=128, scaling_recipe=SR(use_2d_block=True))
        da, db = O.dequant_block1d(u8(qa), 0, f32(sa), 1), O.dequant_block2d(u8(qb), 0, f32(sb))
    out = gemm_fp8_impl(qa, sa, False, qb, sb, True, out_dtype, trans_c, g.value)
    ref = O.gemm_ref(da, db, False, True, trans_c)
    assert out.dtype == out_dtype and tuple(out.shape) == ref.shape
    _check(out, ref, f"{gran} split {out_dtype} trans_c={trans_c}")


@pytest.mark.parametrize("mnk", [(256, 512, 512), (176, 352, 160), (1024, 1024, 1024)])
@pytest.mark.parametrize("fmts", [(torch.float8_e4m3fn, torch.float8_e4m3fn), (torch.float8_e5m2, torch.float8_e4m3fn)])
def test_gemm_mx_vs_oracle(mnk, fmts):
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    g = SG.MX_BLOCKWISE
    M, N, K = mnk
    gen = torch.Generator().manual_seed(11)
    a = (torch.exp(torch.randn((M, K), generator=gen) * 1.5) * torch.sign(torch.randn((M, K), generator=gen))).bfloat16()
    b = torch.randn((N, K), generator=gen).bfloat16()
    qa, ea = turbo.ops.quantize_fp8(a.cuda(), fmts[0], g, block_size=32, axis=1, scaling_recipe=SR())
    qb, eb = turbo.ops.quantize_fp8(b.cuda(), fmts[1], g, block_size=32, axis=1, scaling_recipe=SR(use_2d_block=True))
    da = O.dequant_mx(u8(qa), FMT[fmts[0]], u8(ea))
    db = O.dequant_mx(u8(qb), FMT[fmts[1]], u8(eb))
    out = gemm_fp8_impl(qa, ea, False, qb, eb, True, torch.bfloat16, False, g.value)
    ref = O.gemm_ref(da, db, False, True)
    _check(out, ref, "MX")
    # the same operands with K-block-major exponents give the same output bits
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_mxfp8_impl
    from primus_turbo.pytorch.ops.gemm_fp8 import _mx_strides
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt

    qak, eak = quantize_mxfp8_impl(a.cuda(), fmts[0], 1, 32, scaling_recipe=SR(), exp_kmajor=True)
    qbk, ebk = quantize_mxfp8_impl(b.cuda(), fmts[1], 1, 32, scaling_recipe=SR(use_2d_block=True), exp_kmajor=True)
    outk = gemm_fp8_nt(qak, qbk, torch.bfloat16, g, eak, _mx_strides(eak), False, ebk, _mx_strides(ebk), False)
    assert torch.equal(outk[:, :N], out), "k-major exponents change the MX GEMM result"


def _autograd_case(m, n, k, layout, fmt_name, gran_name, block_size=None, dtype=torch.bfloat16):
    turbo, Cfg, Format, ScaleDtype, SG, _, _ = _mods()
    fmt = getattr(Format, fmt_name)
    gran = getattr(SG, gran_name)
    ta, tb = layout[0] == "T", layout[1] == "T"
    gen = torch.Generator().manual_seed(42)
    a = torch.randn((k, m) if ta else (m, k), generator=gen).to(dtype).cuda().requires_grad_()
    b = torch.randn((n, k) if tb else (k, n), generator=gen).to(dtype).cuda().requires_grad_()
    a_ref = a.detach().float().requires_grad_()
    b_ref = b.detach().float().requires_grad_()
    c_ref = (a_ref.T if ta else a_ref) @ (b_ref.T if tb else b_ref)
    grad = torch.randn(c_ref.shape, generator=gen).cuda()
    c_ref.backward(grad)
    if block_size is not None:
        sd = ScaleDtype.E8M0 if gran == SG.MX_BLOCKWISE else ScaleDtype.FP32
        cfg = Cfg(granularity=gran, format=fmt, block_size=block_size, scale_dtype=sd)
    else:
        cfg = Cfg(granularity=gran, format=fmt)
    c = turbo.ops.gemm_fp8(a, b, ta, tb, dtype, cfg)
    c.backward(grad.to(dtype))
    assert c.shape == c_ref.shape and a.grad.shape == a.shape and b.grad.shape == b.shape
    thr = 25 if fmt == Format.E4M3 else 20
    for name, x, r in (("C", c, c_ref), ("dA", a.grad, a_ref.grad), ("dB", b.grad, b_ref.grad)):
        s = O.snr_db(f32(r), f32(x))
        assert s > thr, f"{name} SNR {s:.1f} dB <= {thr}"


@pytest.mark.parametrize("mnk", [(1024, 4096, 4096), (2272, 3008, 4096)])
@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
def test_gemm_fp8_autograd_k_split_shapes(mnk, gran):
    """A layer whose forward and dgrad GEMMs take the K split (64 / 108 tiles
    of 256 x 256, K = 4096; the second with partial edge tiles) meets the
    reference's end-to-end criterion for C, dA and dB."""
    bs = {"BLOCKWISE": 128, "MX_BLOCKWISE": 32}.get(gran)
    _autograd_case(*mnk, "NT", "E4M3", gran, block_size=bs)


@pytest.mark.parametrize("m", [255, 512])
@pytest.mark.parametrize("n,k", [(512, 576), (1024, 256)])
@pytest.mark.parametrize("layout", ["NT", "NN"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2", "HYBRID"])
def test_gemm_fp8_tensorwise_autograd(m, n, k, layout, fmt):
    _autograd_case(m, n, k, layout, fmt, "TENSORWISE")


@pytest.mark.parametrize("m", [255, 512])
@pytest.mark.parametrize("n,k", [(512, 576), (1024, 256)])
@pytest.mark.parametrize("layout", ["NT", "NN"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2"])
def test_gemm_fp8_rowwise_autograd(m, n, k, layout, fmt):
    _autograd_case(m, n, k, layout, fmt, "ROWWISE")


@pytest.mark.parametrize("m", [512, 1024])
@pytest.mark.parametrize("n,k", [(1024, 256), (4096, 1024)])
@pytest.mark.parametrize("layout", ["NT", "NN"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2"])
def test_gemm_fp8_blockwise_autograd(m, n, k, layout, fmt):
    _autograd_case(m, n, k, layout, fmt, "BLOCKWISE", block_size=128)


@pytest.mark.parametrize("m,n,k", [(176, 352, 160), (256, 256, 512), (1024, 1024, 1024)])
@pytest.mark.parametrize("fmt", ["E4M3", "HYBRID"])
def test_gemm_fp8_mx_autograd(m, n, k, fmt):
    _autograd_case(m, n, k, "NT", fmt, "MX_BLOCKWISE", block_size=32)


def test_gemm_blockwise_deterministic():
    turbo, Cfg, Format, _, SG, _, _ = _mods()
    cfg = Cfg(granularity=SG.BLOCKWISE, format=Format.E4M3, block_size=128)
    a = randn((512, 1024), seed=1).cuda()
    b = randn((768, 1024), seed=2).cuda()
    outs = [turbo.ops.gemm_fp8(a, b, False, True, torch.bfloat16, cfg) for _ in range(5)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])



@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
@pytest.mark.parametrize("n", [4352, 4300])
def test_gemm_multi_round_vs_oracle(gran, n):
    """272 tiles (more than one round on 256 CUs); n = 4300 leaves a partial last
    tile column and a C row stride that is not 16-byte aligned."""
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    g = getattr(SG, gran)
    M, K = 4096, 256
    qdt = torch.float8_e4m3fn
    a = randn((M, K), seed=21).cuda()
    b = randn((n, K), seed=22).cuda()
    if g == SG.TENSORWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g)
        da, db = O.dequant_tensorwise(u8(qa), 0, f32(sa)), O.dequant_tensorwise(u8(qb), 0, f32(sb))
    elif g == SG.ROWWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, axis=-1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, axis=-1)
        da, db = O.dequant_rowwise(u8(qa), 0, f32(sa)), O.dequant_rowwise(u8(qb), 0, f32(sb))
    elif g == SG.BLOCKWISE:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=128, axis=1)
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=128, scaling_recipe=SR(use_2d_block=True))
        da, db = O.dequant_block1d(u8(qa), 0, f32(sa), 1), O.dequant_block2d(u8(qb), 0, f32(sb))
    else:
        qa, sa = turbo.ops.quantize_fp8(a, qdt, g, block_size=32, axis=1, scaling_recipe=SR())
        qb, sb = turbo.ops.quantize_fp8(b, qdt, g, block_size=32, axis=1, scaling_recipe=SR())
        da, db = O.dequant_mx(u8(qa), 0, u8(sa)), O.dequant_mx(u8(qb), 0, u8(sb))
    out = gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, g.value)
    _check(out, O.gemm_ref(da, db, False, True), f"{gran} n={n}")


def test_gemm_multi_round_wgrad_1d_scales():
    """1-D x 1-D blockwise (TN, column scales staged through LDS) over 272 tiles."""
    turbo, _, _, _, SG, SR, gemm_fp8_impl = _mods()
    g = SG.BLOCKWISE
    M, N, K = 4096, 4352, 256
    a = randn((K, M), seed=23).cuda()
    b = randn((K, N), seed=24).cuda()
    qa, sa = turbo.ops.quantize_fp8(a, torch.float8_e4m3fn, g, block_size=128, axis=0)
    qb, sb = turbo.ops.quantize_fp8(b, torch.float8_e4m3fn, g, block_size=128, axis=0)
    da = O.dequant_block1d(u8(qa), 0, f32(sa), 0)
    db = O.dequant_block1d(u8(qb), 0, f32(sb), 0)
    out = gemm_fp8_impl(qa, sa, True, qb, sb, False, torch.bfloat16, False, g.value)
    _check(out, O.gemm_ref(da, db, True, False), "TN multi-round")


@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE", "MX_BLOCKWISE"])
def test_float8_linear_fwd_bwd(gran):
    """Float8Linear on a [2, 96, 512] input against an fp32 Linear (reference's
    SNR criterion, > 25 dB for e4m3), bias and leading dims included."""
    turbo, Cfg, Format, ScaleDtype, SG, _, _ = _mods()
    g = getattr(SG, gran)
    kw = {}
    if g == SG.BLOCKWISE:
        kw = dict(block_size=128)
    elif g == SG.MX_BLOCKWISE:
        kw = dict(block_size=32, scale_dtype=ScaleDtype.E8M0)
    cfg = Cfg(granularity=g, format=Format.E4M3, **kw)
    torch.manual_seed(3)
    ref = torch.nn.Linear(512, 256, bias=True).cuda()
    lin = turbo.modules.Float8Linear.from_float(ref, cfg, inplace=False).to(torch.bfloat16)
    x = torch.randn(2, 96, 512, device="cuda")
    xb = x.bfloat16().requires_grad_()
    y = lin(xb)
    assert y.shape == (2, 96, 256) and y.dtype == torch.bfloat16
    dy = torch.randn_like(y)
    y.backward(dy)
    xr = xb.detach().float().requires_grad_()
    yr = torch.nn.functional.linear(xr, lin.weight.detach().float(), lin.bias.detach().float())
    yr.backward(dy.float())
    for name, a, r in (("y", y, yr), ("dx", xb.grad, xr.grad)):
        s = O.snr_db(f32(r), f32(a))
        assert s > 25, f"{name} SNR {s:.1f} dB"
    assert lin.weight.grad is not None and lin.weight.grad.shape == lin.weight.shape


@pytest.mark.skip(reason="its one GPU run ended in a segmentation fault inside torch.cuda.graph's capture_end; "
                         "no cause found in the captured path, so dense gemm_fp8 now raises RuntimeError under "
                         "capture (tests/test_host_api.py) and this case stays off the GPU")
def test_tensorwise_layer_graph_replay():
    """Forward + backward of the tensorwise gemm_fp8 layer recorded once into a
    HIP graph, at a size where eager calls take the single-launch tensorwise
    quantize (x and dy hold 2^21 elements), which hands partial maxima over
    between workgroups under per-call tags that a replayed graph would repeat;
    under capture the two-pass quantize runs instead.  The GEMMs (32-64 tiles)
    take the small-tile kernel.  Every replay, with eager work and
    synchronisations between replays, gives the same bits, and matches the
    eager result to within fp32 summation order."""
    turbo, Cfg, Format, _, SG, _, _ = _mods()
    M, K, N = 1024, 2048, 2048
    gen = torch.Generator().manual_seed(9)
    x = torch.randn((M, K), generator=gen).bfloat16().cuda().requires_grad_()
    w = torch.randn((N, K), generator=gen).bfloat16().cuda().requires_grad_()
    dy = torch.randn((M, N), generator=gen).bfloat16().cuda()
    cfg = Cfg(format=Format.E4M3, granularity=SG.TENSORWISE)

    y = turbo.ops.gemm_fp8(x, w, trans_b=True, config=cfg)
    y.backward(dy)
    eager = (y.detach().clone(), x.grad.clone(), w.grad.clone())
    x.grad = torch.zeros_like(x)
    w.grad = torch.zeros_like(w)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = turbo.ops.gemm_fp8(x, w, trans_b=True, config=cfg)
        out.backward(dy)
    first = None
    for _ in range(3):
        x.grad.zero_()
        w.grad.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = (out.clone(), x.grad.clone(), w.grad.clone())
        if first is None:
            first = got
            for name, g_, e in zip(("y", "dx", "dw"), got, eager):
                gv, ev = f32(g_).astype(np.float64), f32(e).astype(np.float64)
                assert np.max(np.abs(gv - ev)) <= 2.0 ** -6 * np.max(np.abs(ev)), f"{name}: graph and eager differ"
        else:
            for name, g_, f in zip(("y", "dx", "dw"), got, first):
                assert torch.equal(g_, f), f"{name}: replays differ"
        _ = (x.detach() * 2).sum().item()  # eager work between replays
    del graph
    torch.cuda.synchronize()


def test_empty_k_writes_zeros():
    """K = 0: the product is a zero matrix, written by a fill kernel (no memset,
    so the call can be recorded into a graph)."""
    from primus_turbo.pytorch import _C

    M, N = 300, 200
    a = torch.empty((M, 16), dtype=torch.float8_e4m3fn, device="cuda")
    b = torch.empty((N, 16), dtype=torch.float8_e4m3fn, device="cuda")
    s = torch.ones((), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    _C.call("pta_gemm_fp8", _C.ptr(a), _C.fp8_code(a.dtype), _C.ptr(s), 0, _C.ptr(b), _C.fp8_code(b.dtype),
            _C.ptr(s), 1, _C.ptr(out), _C.out_dtype_code(out.dtype), 0, M, N, 0, _C.PTA_TENSORWISE, None, 0,
            _C.stream(a.device))
    torch.cuda.synchronize()
    assert not out.float().any()


@pytest.mark.parametrize("gran", ["TENSORWISE", "ROWWISE", "BLOCKWISE"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2", "HYBRID"])
@pytest.mark.parametrize("bias", [True, False])
def test_reference_float8linear_criterion(gran, dtype, fmt, bias):
    """The reference's Float8Linear test (tests/pytorch/modules/
    test_linear_fp8.py:14-102) at M=128, N=256, K=512: output, input and weight
    gradients above 20 dB against nn.Linear in the same dtype, bias gradient at
    its dtype tolerance; HYBRID with TENSORWISE only, as there."""
    turbo, Cfg, Format, ScaleDtype, SG, _, _ = _mods()
    if fmt == "HYBRID" and gran != "TENSORWISE":
        pytest.skip("Format.HYBRID is only supported for TENSORWISE granularity (as in the reference)")
    cfg = Cfg(granularity=getattr(SG, gran), format=getattr(Format, fmt),
              **({"block_size": 128} if gran == "BLOCKWISE" else {}))
    torch.manual_seed(0)
    M, N, K = 128, 256, 512
    x1 = torch.randn((M, K), dtype=dtype, device="cuda", requires_grad=True)
    x2 = x1.detach().clone().requires_grad_()
    model = torch.nn.Linear(K, N, bias=bias).to("cuda", dtype=dtype)
    out_ref = model(x1)
    grad_out = torch.randn_like(out_ref)
    out_ref.backward(grad_out)
    xg_ref, wg_ref = x1.grad.clone(), model.weight.grad.clone()
    bg_ref = model.bias.grad.clone() if bias else None
    model.weight.grad = None
    if bias:
        model.bias.grad = None
    lin = turbo.modules.Float8Linear.from_float(model, cfg)
    out = lin(x2)
    out.backward(grad_out)
    for name, r, a in (("out", out_ref, out), ("dx", xg_ref, x2.grad), ("dw", wg_ref, lin.weight.grad)):
        s = O.snr_db(f32(r), f32(a))
        assert s > 20, f"{name} SNR {s:.1f} dB"
    if bias:
        torch.testing.assert_close(lin.bias.grad, bg_ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("m", [176, 512])
@pytest.mark.parametrize("n", [256, 352])
@pytest.mark.parametrize("k", [128, 160])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2", "HYBRID"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fp8_mx_reference_grid(m, n, k, fmt, dtype):
    """The reference's MX gemm_fp8 grid (test_gemm_fp8.py:293-330: ragged m/n,
    k = 128 / 160, all three formats, bf16 and fp16 outputs), its SNR criterion."""
    _autograd_case(m, n, k, "NT", fmt, "MX_BLOCKWISE", block_size=32, dtype=dtype)
