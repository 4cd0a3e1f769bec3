"""grouped_gemm_fp8 forward, dgrad and wgrad of the TENSORWISE, ROWWISE and
MX_BLOCKWISE layers against the fp64 oracle.

Each test restates the layer's whole chain on the CPU oracle, as the reference
runs it (ops/grouped_gemm_fp8.py:214-795): the forward quantizations, the
backward's re-quantization of the dequantized forward operands along the other
axis (rowwise), the byte transposes (tensorwise), the 32- / 128-padded grouped
layouts (MX), the grad quantizations (E5M2 under HYBRID), then the fp64
product of the dequantized operands per group.  The GPU's own quantized
tensors are checked bit for bit against the oracle's where the public ops
expose them, and every output, dA and dW group is held to SNR >= 40 dB and
max|err| / max|ref| <= 1e-2.  Empty groups must give empty forward rows and
a zero dW slice."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bitexact, f32, randn, u8

pytestmark = pytest.mark.gpu

SNR_MIN = 40.0
REL_MAX = 1e-2
LENS = [[300, 0, 513, 128, 59], [0, 0, 256], [64, 64, 64, 64], [1, 0, 700]]


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
    o = np.asarray(out, np.float64)
    snr = O.snr_db(ref, o)
    rel = O.max_rel_err(ref, o)
    assert snr >= SNR_MIN and rel <= REL_MAX, f"{what}: SNR {snr:.1f} dB, rel {rel:.2e}"


def _deq16(q, fmt, s, dtype=torch.bfloat16):
    """The product's dequantize: dtype(float(q) * scale_inv), one fp32 product."""
    v = torch.from_numpy(O.fp8_to_float(q, fmt))
    return (v * torch.from_numpy(np.asarray(s, np.float32))).to(dtype)


def _fmts(fmt):
    """(forward code, grad code) of a Format name."""
    return {"E4M3": (0, 0), "E5M2": (1, 1), "HYBRID": (0, 1)}[fmt]


def _inputs(lens, K, N, trans_b, seed):
    G, M = len(lens), sum(lens)
    a = randn((max(M, 1), K), seed=seed)[:M].contiguous()
    w = randn((G, N, K) if trans_b else (G, K, N), seed=seed + 1, scale=0.05)
    g = randn((max(M, 1), N), seed=seed + 2)[:M].contiguous()
    return a, w, g


def _run_layer(turbo, cfg, a, w, g, lens, trans_b):
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    ad = a.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    out = turbo.ops.grouped_gemm_fp8(ad, wd, gl, trans_b=trans_b, config=cfg)
    out.backward(g.cuda())
    torch.cuda.synchronize()
    return f32(out), f32(ad.grad), f32(wd.grad)


def _check_groups(lens, out, dA, dW, ref_out, ref_dA, ref_dW, what):
    off = 0
    for i, L in enumerate(lens):
        if L:
            _check(out[off:off + L], ref_out(i, off, L), f"{what} out group {i}")
            _check(dA[off:off + L], ref_dA(i, off, L), f"{what} dA group {i}")
            _check(dW[i], ref_dW(i, off, L), f"{what} dW group {i}")
        else:
            assert not dW[i].any(), f"{what}: expert {i} without tokens must get a zero dW"
        off += L


@pytest.mark.parametrize("lens", LENS)
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("fmt", ["E4M3", "HYBRID"])
def test_grouped_rowwise_layer_vs_oracle(lens, trans_b, fmt):
    """ROWWISE (ops/grouped_gemm_fp8.py:214-379): a rowwise along K, b along
    its K axis; the backward's copies re-quantize the bf16 dequantized
    forward tensors along the other axis (a over all packed rows, as the
    reference treats grouped ROWWISE tensors as plain ones); grad rowwise
    along N for dgrad and along M for wgrad."""
    turbo, Cfg, Format, _, SG, _ = _mods()
    from primus_turbo.pytorch.core.quantized_tensor import QuantizedTensor as QT

    G, K, N = len(lens), 512, 384
    fa, fg = _fmts(fmt)
    a, w, g = _inputs(lens, K, N, trans_b, seed=40)
    b_row_ax, b_col_ax = (2, 1) if trans_b else (1, 2)
    # --- oracle chain
    qa, sa = O.quant_rowwise(a, fa, 1)
    qb, sb = O.quant_rowwise(w, fa, b_row_ax)
    qa_t, sa_t = O.quant_rowwise(_deq16(qa, fa, sa), fa, 0)
    qb_t, sb_t = O.quant_rowwise(_deq16(qb, fa, sb), fa, b_col_ax)
    qg, sg = O.quant_rowwise(g, fg, 1)
    qg_t, sg_t = O.quant_rowwise(g, fg, 0)
    da, db = O.dequant_rowwise(qa, fa, sa), O.dequant_rowwise(qb, fa, sb)
    da_t, db_t = O.dequant_rowwise(qa_t, fa, sa_t), O.dequant_rowwise(qb_t, fa, sb_t)
    dg, dg_t = O.dequant_rowwise(qg, fg, sg), O.dequant_rowwise(qg_t, fg, sg_t)
    # --- the GPU's quantized copies of the same chain, bit for bit
    fdt = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    tqa = QT.quantize(a.cuda(), fdt[fa], SG.ROWWISE, axis=-1, group_lens=gl)
    tqb = QT.quantize(w.cuda(), fdt[fa], SG.ROWWISE, axis=b_row_ax - 3)
    tqa_t = QT.quantize(tqa.dequantize(), fdt[fa], SG.ROWWISE, axis=-2, group_lens=gl)
    tqb_t = QT.quantize(tqb.dequantize(), fdt[fa], SG.ROWWISE, axis=b_col_ax - 3)
    tqg_t = QT.quantize(g.cuda(), fdt[fg], SG.ROWWISE, axis=-2, group_lens=gl)
    for name, t, q, s in (("a", tqa, qa, sa), ("b", tqb, qb, sb), ("a_t", tqa_t, qa_t, sa_t),
                          ("b_t", tqb_t, qb_t, sb_t), ("g_t", tqg_t, qg_t, sg_t)):
        assert_bytes_equal(u8(t.qdata), q, f"{name} bytes")
        assert_f32_bitexact(f32(t.scale_inv).reshape(s.shape), s, f"{name} scales")
    # --- the layer
    cfg = Cfg(granularity=SG.ROWWISE, format=getattr(Format, fmt))
    out, dA, dW = _run_layer(turbo, cfg, a, w, g, lens, trans_b)
    _check_groups(
        lens, out, dA, dW,
        lambda i, o, L: O.gemm_ref(da[o:o + L], db[i], False, trans_b),
        lambda i, o, L: O.gemm_ref(dg[o:o + L], db_t[i], False, not trans_b),
        lambda i, o, L: O.gemm_ref(da_t[o:o + L], dg_t[o:o + L], True, False, trans_b),
        f"rowwise {fmt} trans_b={trans_b}",
    )


@pytest.mark.parametrize("lens", LENS)
@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("fmt", ["E4M3", "HYBRID"])
def test_grouped_tensorwise_layer_vs_oracle(lens, trans_b, fmt):
    """TENSORWISE (ops/grouped_gemm_fp8.py:382-567): one scale per tensor; the
    NT backward (trans_b) runs dgrad on the byte-transposed weight with the
    weight's scale; wgrad is variable-K over the packed rows."""
    turbo, Cfg, Format, _, SG, _ = _mods()
    G, K, N = len(lens), 512, 384
    fa, fg = _fmts(fmt)
    a, w, g = _inputs(lens, K, N, trans_b, seed=50)
    qa, sa = O.quant_tensorwise(a, fa)
    qb, sb = O.quant_tensorwise(w, fa)
    qg, sg = O.quant_tensorwise(g, fg)
    da, db, dg = O.dequant_tensorwise(qa, fa, sa), O.dequant_tensorwise(qb, fa, sb), O.dequant_tensorwise(qg, fg, sg)
    for name, x, fmt_, q, s in (("a", a, fa, qa, sa), ("b", w, fa, qb, sb), ("g", g, fg, qg, sg)):
        tq, ts = turbo.ops.quantize_fp8(x.cuda(), {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}[fmt_],
                                        SG.TENSORWISE)
        assert_bytes_equal(u8(tq), q, f"{name} bytes")
        assert_f32_bitexact(f32(ts).reshape(()), s, f"{name} scale")
    cfg = Cfg(granularity=SG.TENSORWISE, format=getattr(Format, fmt))
    out, dA, dW = _run_layer(turbo, cfg, a, w, g, lens, trans_b)
    _check_groups(
        lens, out, dA, dW,
        lambda i, o, L: O.gemm_ref(da[o:o + L], db[i], False, trans_b),
        lambda i, o, L: O.gemm_ref(dg[o:o + L], db[i], False, not trans_b),
        lambda i, o, L: O.gemm_ref(da[o:o + L], dg[o:o + L], True, False, trans_b),
        f"tensorwise {fmt} trans_b={trans_b}",
    )


@pytest.mark.parametrize("lens", LENS)
@pytest.mark.parametrize("fmt", ["E4M3", "HYBRID"])
def test_grouped_mx_layer_vs_oracle(lens, fmt):
    """MX_BLOCKWISE (ops/grouped_gemm_fp8.py:593-795), NT: activations and
    grads in the grouped layout (each group padded to 32 rows rowwise, to 128
    transposed colwise), the weight with 32 x 32 blocks and its transposed
    colwise copy; forward and dgrad read padded rows and write packed rows,
    wgrad sums over each group's 128-padded columns."""
    turbo, Cfg, Format, ScaleDtype, SG, SR = _mods()
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import grouped_quantize_mxfp8_impl

    G, K, N = len(lens), 512, 384
    fa, fg = _fmts(fmt)
    a, w, g = _inputs(lens, K, N, True, seed=60)
    ar, aer, aorw, ac, aec, aoc = O.quant_mx_grouped(a, fa, lens)
    gr, ger, gorw, gc, gec, goc = O.quant_mx_grouped(g, fg, lens)
    wr, wer = O.quant_mx(w, fa, 1, use_2d=True)  # [G, N, K]
    wc, wec = O.quant_mx(w, fa, 0, use_2d=True)  # [G, K, N_pad]
    # the GPU's grouped quantize of the grad (the dgrad / wgrad operand), bit for bit
    gl = torch.tensor(lens, dtype=torch.int64, device="cuda")
    t = grouped_quantize_mxfp8_impl(g.cuda(), {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}[fg], None, 32, gl,
                                    group_offs_from_lens(gl), True)
    R, C = int(gorw[-1]), int(goc[-1])
    assert_bytes_equal(u8(t[0])[:R], gr[:R], "grad rowwise bytes")
    assert_bytes_equal(u8(t[1])[:R], ger[:R], "grad rowwise exponents")
    assert_bytes_equal(u8(t[2])[:, :C], gc[:, :C], "grad colwise bytes")
    assert_bytes_equal(u8(t[3])[:, : C // 32], gec[:, : C // 32], "grad colwise exponents")
    da = O.dequant_mx(ar, fa, aer)
    dg = O.dequant_mx(gr, fg, ger)
    dwr = O.dequant_mx(wr.reshape(G * N, -1), fa, wer.reshape(G * N, -1)).reshape(G, N, -1)
    dwc = O.dequant_mx(wc.reshape(G * K, -1), fa, wec.reshape(G * K, -1)).reshape(G, K, -1)
    dac = O.dequant_mx(ac, fa, aec)
    dgc = O.dequant_mx(gc, fg, gec)
    cfg = Cfg(granularity=SG.MX_BLOCKWISE, format=getattr(Format, fmt), block_size=32, scale_dtype=ScaleDtype.E8M0)
    out, dA, dW = _run_layer(turbo, cfg, a, w, g, lens, True)
    starts = np.concatenate([[0], np.cumsum(lens)])

    def ref_out(i, o, L):
        r0 = aorw[i]
        return O.gemm_ref(da[r0:r0 + L, :K], dwr[i][:, :K], False, True)

    def ref_dA(i, o, L):
        r0 = gorw[i]
        return O.gemm_ref(dg[r0:r0 + L], dwc[i], False, True)[:, :K]

    def ref_dW(i, o, L):
        c0, c1 = aoc[i], aoc[i + 1]
        assert (goc[i], goc[i + 1]) == (c0, c1)
        return O.gemm_ref(dgc[:, c0:c1], dac[:, c0:c1], False, True)

    assert starts[-1] == sum(lens)
    _check_groups(lens, out, dA, dW, ref_out, ref_dA, ref_dW, f"mx {fmt}")
