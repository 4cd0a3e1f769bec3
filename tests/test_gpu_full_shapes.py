"""Parity at the full shapes of every BASELINE.json configuration.

Each test quantizes the configuration's seeded inputs on the GPU the way the
autograd functions do, checks the FP8 bytes and scales bit for bit against
the CPU oracle over the whole tensors (oracle calls split over row ranges on
a thread pool; the C oracle releases the GIL), then runs the public op
forward and backward and compares the results with the fp64 products of the
dequantized operands over the whole outputs:

* tolerance (bf16 outputs): SNR >= 40 dB and max|out - ref| / max|ref| <= 1e-2;
* where the backward re-quantizes a dequantized operand (rowwise, config 2),
  the oracle restates that re-quantization too: the GPU's re-quantized bytes
  and scales are checked bit for bit, then the gradients against the fp64
  products at the same tolerance.

Inputs follow BASELINE.json: N(0,1) activations, N(0, 0.02) weights where the
config says so, 0.1% outliers x50 for config 3, a seeded Zipf(1.1) 32-expert
split with 4 empty experts for config 4, sign x lognormal magnitudes for
config 5."""

from __future__ import annotations

import concurrent.futures as cf
import gc

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bitexact, f32, randn, u8

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

SNR_MIN = 40.0
REL_MAX = 1e-2
_POOL = cf.ThreadPoolExecutor(16)
E4 = torch.float8_e4m3fn
E5 = torch.float8_e5m2


def _mods():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import (
        Float8QuantConfig,
        Format,
        ScaleDtype,
        ScalingGranularity,
        ScalingRecipe,
    )

    return turbo, Float8QuantConfig, Format, ScaleDtype, ScalingGranularity, ScalingRecipe


def _check(out, ref, what):
    o = out if isinstance(out, np.ndarray) else f32(out)
    snr = O.snr_db(ref, o)
    rel = O.max_rel_err(ref, o)
    print(f"{what}: SNR {snr:.1f} dB, max rel {rel:.2e}", flush=True)
    assert snr >= SNR_MIN and rel <= REL_MAX, f"{what}: SNR {snr:.1f} dB, max rel err {rel:.2e}"


def _chunks(n, step):
    """About 16 row ranges covering [0, n), each a multiple of `step` rows
    (the last one may be shorter)."""
    per = -(-n // 16)
    c = max(step, -(-per // step) * step)
    return [(r0, min(n, r0 + c)) for r0 in range(0, n, c)]


def _par(fn, spans):
    for f in [_POOL.submit(fn, r0, r1) for r0, r1 in spans]:
        f.result()


# ---- oracle quantizers over row ranges --------------------------------------
def _o_rowwise_last(x, fmt):
    M, N = x.shape
    q, s = np.empty((M, N), np.uint8), np.empty((M, 1), np.float32)

    def one(r0, r1):
        q[r0:r1], s[r0:r1] = O.quant_rowwise(x[r0:r1], fmt, -1)

    _par(one, _chunks(M, 1))
    return q, s


def _o_rowwise_cols(x, fmt):
    """Rowwise along axis 0 (one scale per column, over all rows), over column ranges."""
    M, N = x.shape
    q, s = np.empty((M, N), np.uint8), np.empty((1, N), np.float32)

    def one(c0, c1):
        q[:, c0:c1], s[:, c0:c1] = O.quant_rowwise(np.ascontiguousarray(x[:, c0:c1]), fmt, 0)

    _par(one, _chunks(N, 16))
    return q, s


def _deq16(q, fmt, s, dtype=torch.float32):
    """The product's dequantize: dtype(float(q) * scale_inv), one fp32 product,
    returned as fp32 values of `dtype` (numpy)."""
    v = torch.from_numpy(O.fp8_to_float(q, fmt))
    return (v * torch.from_numpy(np.asarray(s, np.float32))).to(dtype).float().numpy()


def _o_block1d(x, fmt, axis):
    M, N = x.shape
    q = np.empty((M, N), np.uint8)
    s = np.empty((M, -(-N // 128)) if axis == 1 else (-(-M // 128), N), np.float32)

    def one(r0, r1):
        qq, ss = O.quant_block1d(x[r0:r1], fmt, axis)
        q[r0:r1] = qq
        if axis == 1:
            s[r0:r1] = ss
        else:
            s[r0 // 128:r0 // 128 + ss.shape[0]] = ss

    _par(one, _chunks(M, 128))
    return q, s


def _o_weight(x, fmt):
    M, N = x.shape
    q = np.empty((M, N), np.uint8)
    s = np.empty((-(-M // 128), -(-N // 128)), np.float32)

    def one(r0, r1):
        qq, ss = O.quant_block_weight(x[r0:r1], fmt)
        q[r0:r1] = qq
        s[r0 // 128:r0 // 128 + ss.shape[0]] = ss

    _par(one, _chunks(M, 128))
    return q, s


def _o_mx(x, fmt, direction, use_2d):
    """quant_mx of x[M, N] over 128-row ranges: rowwise q[M, N_pad], e[M, N_pad/32];
    colwise (transposed) q[N, M_pad], e[N, M_pad/32]."""
    M, N = x.shape
    Mp, Np = -(-M // 128) * 128, -(-N // 128) * 128
    if direction == 1:
        q, e = np.empty((M, Np), np.uint8), np.empty((M, Np // 32), np.uint8)
    else:
        q, e = np.empty((N, Mp), np.uint8), np.empty((N, Mp // 32), np.uint8)

    def one(r0, r1):
        qq, ee = O.quant_mx(x[r0:r1], fmt, direction, use_2d)
        if direction == 1:
            q[r0:r1], e[r0:r1] = qq, ee
        else:
            q[:, r0:r0 + qq.shape[1]] = qq
            e[:, r0 // 32:r0 // 32 + ee.shape[1]] = ee

    _par(one, _chunks(M, 128))
    return q, e


def _deq_mx_rows(q, e, fmt, rows, cols):
    return O.dequant_mx(q[:rows], fmt, e[:rows])[:, :cols]


def _outliers(shape, seed, scale=1.0):
    return randn(shape, seed=seed, scale=scale, outliers=0.001)


# ---------------------------------------------------------------------------
# config 2: rowwise e4m3, Llama-3-8B up-proj, NT
# ---------------------------------------------------------------------------
def test_cfg2_rowwise_8192x14336x4096():
    turbo, QC, Fmt, _, SG, _ = _mods()
    M, N, K = 8192, 14336, 4096
    print(f"cfg2 rowwise {M}x{N}x{K}", flush=True)
    a = randn((M, K), seed=201)
    w = randn((N, K), seed=202, scale=0.02)
    g = randn((M, N), seed=203)
    qa, sa = turbo.ops.quantize_fp8(a.cuda(), E4, SG.ROWWISE, axis=-1)
    qw, sw = turbo.ops.quantize_fp8(w.cuda(), E4, SG.ROWWISE, axis=-1)
    oqa, osa = _o_rowwise_last(a, 0)
    oqw, osw = _o_rowwise_last(w, 0)
    assert_bytes_equal(u8(qa), oqa, "A bytes")
    assert_f32_bitexact(f32(sa), osa, "A scales")
    assert_bytes_equal(u8(qw), oqw, "W bytes")
    assert_f32_bitexact(f32(sw), osw, "W scales")
    del qa, qw, sa, sw
    cfg = QC(granularity=SG.ROWWISE, format=Fmt.E4M3)
    ad = a.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    out = turbo.ops.gemm_fp8(ad, wd, trans_b=True, config=cfg)
    out.backward(g.cuda())
    torch.cuda.synchronize()
    _check(out, O.gemm_ref(O.dequant_rowwise(oqa, 0, osa), O.dequant_rowwise(oqw, 0, osw), False, True),
           "cfg2 forward vs fp64 oracle")
    # backward (gemm_fp8.py:231-379), restated on the oracle: grad rowwise
    # along N (dgrad) and along M (wgrad); the weight and activation copies
    # re-quantized along the other axis from their bf16 dequantized forward
    # bytes.  The GPU's re-quantized copies are checked bit for bit first.
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor as QT

    # (fp32 arrays holding the bf16 values: the quantizers widen bf16 to fp32
    # exactly before any arithmetic, so the bytes and scales are the same)
    oqw_t, osw_t = _o_rowwise_cols(_deq16(oqw, 0, osw, torch.bfloat16), 0)
    oqa_t, osa_t = _o_rowwise_cols(_deq16(oqa, 0, osa, torch.bfloat16), 0)
    oqg, osg = _o_rowwise_last(g, 0)
    oqg_t, osg_t = _o_rowwise_cols(g.float().numpy(), 0)
    for name, x, q, s in (("W_t", wd, oqw_t, osw_t), ("A_t", ad, oqa_t, osa_t)):
        t = QT.quantize(QT.quantize(x.detach(), E4, SG.ROWWISE, axis=-1).dequantize(), E4, SG.ROWWISE, axis=-2)
        assert_bytes_equal(u8(t.qdata), q, f"{name} re-quantized bytes")
        assert_f32_bitexact(f32(t.scale_inv).reshape(s.shape), s, f"{name} re-quantized scales")
        del t
    t = QT.quantize(g.cuda(), E4, SG.ROWWISE, axis=-2)
    assert_bytes_equal(u8(t.qdata), oqg_t, "grad column bytes")
    assert_f32_bitexact(f32(t.scale_inv).reshape(osg_t.shape), osg_t, "grad column scales")
    del t
    _check(ad.grad, O.gemm_ref(O.dequant_rowwise(oqg, 0, osg), O.dequant_rowwise(oqw_t, 0, osw_t), False, False),
           "cfg2 dA vs fp64 oracle")
    _check(wd.grad, O.gemm_ref(O.dequant_rowwise(oqg_t, 0, osg_t), O.dequant_rowwise(oqa_t, 0, osa_t), True, False),
           "cfg2 dW vs fp64 oracle")


# ---------------------------------------------------------------------------
# config 3: blockwise 1x128 / 128x128 e4m3, fwd NT + dgrad + wgrad
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("MNK", [(4096, 18432, 7168), (4096, 7168, 2048)], ids=["S1", "S2"])
def test_cfg3_blockwise_fwd_dgrad_wgrad(MNK):
    turbo, QC, Fmt, _, SG, SR = _mods()
    M, N, K = MNK
    print(f"cfg3 blockwise {M}x{N}x{K}", flush=True)
    a = _outliers((M, K), 301)
    w = _outliers((N, K), 302)
    g = _outliers((M, N), 303)
    # the quantizers of the autograd path, in the reference layouts
    qar, sar, qac, sac = turbo.ops.quantize_fp8_with_trans(a.cuda(), E4, SG.BLOCKWISE, block_size=128)
    qw, sw = turbo.ops.quantize_fp8(w.cuda(), E4, SG.BLOCKWISE, block_size=128, scaling_recipe=SR(use_2d_block=True))
    qgr, sgr, qgc, sgc = turbo.ops.quantize_fp8_with_trans(g.cuda(), E4, SG.BLOCKWISE, block_size=128)
    for (gq, gs), x, axis, what in (((qar, sar), a, 1, "A rows"), ((qac, sac), a, 0, "A cols"),
                                    ((qgr, sgr), g, 1, "G rows"), ((qgc, sgc), g, 0, "G cols")):
        oq, os_ = _o_block1d(x, 0, axis)
        assert_bytes_equal(u8(gq), oq, f"{what} bytes")
        assert_f32_bitexact(f32(gs), os_, f"{what} scales")
    oqw, osw = _o_weight(w, 0)
    assert_bytes_equal(u8(qw), oqw, "W bytes")
    assert_f32_bitexact(f32(sw), osw, "W scales")
    da_r = O.dequant_block1d(u8(qar), 0, f32(sar), 1)
    da_c = O.dequant_block1d(u8(qac), 0, f32(sac), 0)
    dg_r = O.dequant_block1d(u8(qgr), 0, f32(sgr), 1)
    dg_c = O.dequant_block1d(u8(qgc), 0, f32(sgc), 0)
    dw = O.dequant_block2d(oqw, 0, osw)
    del qar, sar, qac, sac, qw, sw, qgr, sgr, qgc, sgc
    cfg = QC(granularity=SG.BLOCKWISE, format=Fmt.E4M3, block_size=128)
    ad = a.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    out = turbo.ops.gemm_fp8(ad, wd, trans_b=True, config=cfg)
    out.backward(g.cuda())
    torch.cuda.synchronize()
    _check(out, O.gemm_ref(da_r, dw, False, True), "cfg3 forward NT vs fp64 oracle")
    _check(ad.grad, O.gemm_ref(dg_r, dw, False, False), "cfg3 dgrad vs fp64 oracle")
    _check(wd.grad, O.gemm_ref(dg_c, da_c, True, False), "cfg3 wgrad vs fp64 oracle")


# ---------------------------------------------------------------------------
# config 4: grouped blockwise MoE, 32 experts, Zipf split with 4 empty groups
# ---------------------------------------------------------------------------
def _zipf_lens(total=65536, experts=32, nonempty=28, seed=0):
    gen = torch.Generator().manual_seed(seed)
    wts = torch.tensor([r ** -1.1 for r in range(1, nonempty + 1)], dtype=torch.float64)
    cnt = torch.floor(total * wts / wts.sum()).to(torch.int64)
    cnt[0] += total - int(cnt.sum())
    full = torch.zeros(experts, dtype=torch.int64)
    full[:nonempty] = cnt
    return full[torch.randperm(experts, generator=gen)]


def test_cfg4_grouped_blockwise_zipf_fwd_dgrad_wgrad():
    turbo, QC, Fmt, _, SG, SR = _mods()
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_segment_m_row_col_impl,
    )

    G, Mt, N, K = 32, 65536, 2048, 7168
    lens = _zipf_lens()
    assert int(lens.sum()) == Mt and int((lens == 0).sum()) == 4
    print(f"cfg4 grouped {G}x{N}x{K}, M {Mt}, lens {lens.tolist()}", flush=True)
    a = randn((Mt, K), seed=401)
    w = randn((G, N, K), seed=402, scale=0.02)
    gout = randn((Mt, N), seed=403)
    gl = lens.cuda()
    go = group_offs_from_lens(gl)
    offs = [0] + np.cumsum(lens.numpy()).tolist()

    # the autograd path's quantizers: segment row + 128-padded column copies, 128 x 128 weights
    def seg(x):
        r = quant_fp8_blockwise_segment_m_row_col_impl(x.cuda(), E4, 128, gl, go)
        return u8(r[0]), f32(r[2]), u8(r[1]), f32(r[3]), r[5].cpu().numpy()

    a_row, a_srt, a_col, a_sc, vo = seg(a)
    g_row, g_srt, g_col, g_sc, vo2 = seg(gout)
    assert np.array_equal(vo, vo2)
    qw, sw = turbo.ops.quantize_fp8(w.cuda(), E4, SG.BLOCKWISE, block_size=128, scaling_recipe=SR(use_2d_block=True))
    qw, sw = u8(qw), f32(sw)
    # bytes and scales against the oracle: rows (group-independent), per-group
    # 128-padded column blocks, per-expert 128 x 128 weight tiles
    for gq, gs, x, what in ((a_row, a_srt, a, "A"), (g_row, g_srt, gout, "G")):
        oq, os_ = _o_block1d(x, 0, 1)
        assert_bytes_equal(gq, oq, f"{what} row bytes")
        assert_f32_bitexact(gs.T, os_, f"{what} row scales")

    def col_group(gi):
        s0, L = offs[gi], int(lens[gi])
        P = -(-L // 128) * 128
        p0 = int(vo[gi])
        assert int(vo[gi + 1]) - p0 == P
        if L == 0:
            return
        for gc, gsc, x, what in ((a_col, a_sc, a, "A"), (g_col, g_sc, gout, "G")):
            pad = torch.zeros((P, x.shape[1]), dtype=x.dtype)
            pad[:L] = x[s0:s0 + L]
            oq, os_ = O.quant_block1d(pad, 0, 0)
            assert_bytes_equal(gc[p0:p0 + P], oq, f"{what} col bytes, group {gi}")
            assert_f32_bitexact(gsc[p0 // 128:(p0 + P) // 128], os_, f"{what} col scales, group {gi}")

    def w_group(gi):
        oq, os_ = O.quant_block_weight(w[gi], 0)
        assert_bytes_equal(qw[gi], oq, f"W bytes, expert {gi}")
        assert_f32_bitexact(sw[gi], os_, f"W scales, expert {gi}")

    for f in [_POOL.submit(col_group, gi) for gi in range(G)] + [_POOL.submit(w_group, gi) for gi in range(G)]:
        f.result()

    cfg = QC(granularity=SG.BLOCKWISE, format=Fmt.E4M3, block_size=128)
    ad = a.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    out = turbo.ops.grouped_gemm_fp8(ad, wd, gl, trans_b=True, config=cfg)
    out.backward(gout.cuda())
    torch.cuda.synchronize()
    o, da, dwg = f32(out), f32(ad.grad), f32(wd.grad)
    del ad, wd, out
    gc.collect()

    def per_group(gi):
        s0, s1, L = offs[gi], offs[gi + 1], int(lens[gi])
        if L == 0:
            assert not dwg[gi].any(), f"wgrad of empty expert {gi} must be zero"
            return
        dq_w = O.dequant_block2d(qw[gi], 0, sw[gi])
        dq_a = O.dequant_block1d(a_row[s0:s1], 0, a_srt[:, s0:s1].T, 1)
        dq_g = O.dequant_block1d(g_row[s0:s1], 0, g_srt[:, s0:s1].T, 1)
        _check(o[s0:s1], O.gemm_ref(dq_a, dq_w, False, True), f"cfg4 forward, expert {gi} ({L} rows)")
        _check(da[s0:s1], O.gemm_ref(dq_g, dq_w, False, False), f"cfg4 dgrad, expert {gi}")
        p0, p1 = int(vo[gi]), int(vo[gi + 1])
        dq_ac = O.dequant_block1d(a_col[p0:p1], 0, a_sc[p0 // 128:p1 // 128], 0)
        dq_gc = O.dequant_block1d(g_col[p0:p1], 0, g_sc[p0 // 128:p1 // 128], 0)
        _check(dwg[gi], O.gemm_ref(dq_gc, dq_ac, True, False), f"cfg4 wgrad, expert {gi}")

    # groups one after another: each product already uses every BLAS thread
    for gi in range(G):
        per_group(gi)


# ---------------------------------------------------------------------------
# config 5: MX-FP8 HYBRID (e4m3 forward, e5m2 gradient), Llama-3-70B shapes
# ---------------------------------------------------------------------------
def _lognormal(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    sign = torch.where(torch.rand(shape, generator=gen) < 0.5, -1.0, 1.0)
    return (sign * torch.exp(torch.randn(shape, generator=gen) * 1.5)).to(torch.bfloat16)


@pytest.mark.parametrize("MNK", [(8192, 28672, 8192), (8192, 8192, 28672)], ids=["up", "down"])
def test_cfg5_mx_hybrid_fwd_dgrad_wgrad(MNK):
    turbo, QC, Fmt, SD, SG, SR = _mods()
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_mxfp8_impl

    M, N, K = MNK
    print(f"cfg5 MX hybrid {M}x{N}x{K}", flush=True)
    a = _lognormal((M, K), 501 + K)
    w = _lognormal((N, K), 502 + K)
    g = _lognormal((M, N), 503 + K)
    # the autograd path's quantizers: activation 1 x 32 / 32 x 1, weight 32 x 32,
    # gradient e5m2 1 x 32 / 32 x 1; bytes and exponents against the oracle
    r1, r2 = SR(), SR(use_2d_block=True)
    ops = {}
    for name, x, fdt, rec in (("A", a, E4, r1), ("W", w, E4, r2), ("G", g, E5, r1)):
        qr, er, qc, ec = quantize_mxfp8_impl(x.cuda(), fdt, None, 32, with_trans=True, scaling_recipe=rec,
                                             scaling_recipe_for_trans=rec)
        qr, er, qc, ec = u8(qr), u8(er), u8(qc), u8(ec)
        fmt = 0 if fdt == E4 else 1
        oqr, oer = _o_mx(x, fmt, 1, rec.use_2d_block)
        assert_bytes_equal(qr, oqr, f"{name} row bytes")
        assert_bytes_equal(er, oer, f"{name} row exponents")
        del oqr, oer
        oqc, oec = _o_mx(x, fmt, 0, rec.use_2d_block)
        assert_bytes_equal(qc, oqc, f"{name} col bytes")
        assert_bytes_equal(ec, oec, f"{name} col exponents")
        del oqc, oec
        ops[name] = (qr, er, qc, ec, fmt)
    cfg = QC(granularity=SG.MX_BLOCKWISE, format=Fmt.HYBRID, block_size=32, scale_dtype=SD.E8M0)
    ad = a.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    out = turbo.ops.gemm_fp8(ad, wd, False, True, torch.bfloat16, cfg)
    out.backward(g.cuda())
    torch.cuda.synchronize()
    o, da, dw = f32(out), f32(ad.grad), f32(wd.grad)
    del ad, wd, out
    gc.collect()
    qa_r, ea_r, qa_c, ea_c, fa = ops["A"]
    qw_r, ew_r, qw_c, ew_c, fw = ops["W"]
    qg_r, eg_r, qg_c, eg_c, fg = ops["G"]
    # forward: A rows x W rows (K blocks of 32)
    _check(o, O.gemm_ref(_deq_mx_rows(qa_r, ea_r, fa, M, K), _deq_mx_rows(qw_r, ew_r, fw, N, K), False, True),
           "cfg5 forward vs fp64 oracle")
    # dgrad: G rows [M, N] x W colwise copy [K, N_pad] (blocks of 32 along N)
    _check(da, O.gemm_ref(_deq_mx_rows(qg_r, eg_r, fg, M, N), _deq_mx_rows(qw_c, ew_c, fw, K, N), False, True),
           "cfg5 dgrad vs fp64 oracle")
    # wgrad: G colwise copy [N, M_pad] x A colwise copy [K, M_pad] (blocks of 32 along M)
    _check(dw, O.gemm_ref(_deq_mx_rows(qg_c, eg_c, fg, N, M), _deq_mx_rows(qa_c, ea_c, fa, K, M), False, True),
           "cfg5 wgrad vs fp64 oracle")
