"""Pins for the CPU oracle (oracle/fp8_oracle.c, oracle/oracle.py).

The reference holds no byte-level golden vectors for this path (its tests
check quantize->dequantize round trips and GEMM SNR only), so each oracle
function is pinned by checks chosen to fail on a plausible mistake:

* fp8 encode / decode: exhaustive agreement with torch's own casts (c10, an
  independent implementation) over every bf16 and fp16 bit pattern, plus a
  brute-force nearest-value-ties-to-even search over the 256-value grid.
* scale arithmetic: known answers that are exact in binary32 (amax == max
  gives scale 1, amax == 1 gives scale 448, all-zero blocks take the eps
  branch), the invariant that each block's max-magnitude element lands on
  +-max, and agreement with torch's IEEE fp32 division.
* block indexing: perturbing one block leaves every other block's bytes and
  scales unchanged; dual == (row, col) single-direction calls; a 128x128 tile
  equals a tensorwise quantization of that tile (eps aside); the grouped
  segment quantizer equals block1d on each zero-padded group.
* MX: the exponent rule against log2 closed forms and the in-range guarantee.
* GEMM reference: exact integer arithmetic on integer-valued operands.
* the reference's own tolerance: quantize->dequantize within rtol = atol = 0.1
  (tests/pytorch/test_utils.py:17-31 of the reference).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

FMTS = [(0, torch.float8_e4m3fn), (1, torch.float8_e5m2)]


def _bf16_all():
    return (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("fmt,tdt", FMTS)
def test_encode_matches_torch_on_all_bf16(fmt, tdt):
    f = _bf16_all()
    ours = np.array([O.fp8_encode_scalar(float(v), fmt) for v in f], dtype=np.uint8)
    th = torch.from_numpy(f.copy()).to(tdt).view(torch.uint8).numpy()
    fin = np.isfinite(f)
    assert np.array_equal(ours[fin], th[fin])


@pytest.mark.parametrize("fmt,tdt", FMTS)
def test_encode_matches_torch_on_all_fp16(fmt, tdt):
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ours = np.array([O.fp8_encode_scalar(float(v), fmt) for v in h], dtype=np.uint8)
    th = torch.from_numpy(h.copy()).to(tdt).view(torch.uint8).numpy()
    fin = np.isfinite(h)
    assert np.array_equal(ours[fin], th[fin])


@pytest.mark.parametrize("fmt,tdt", FMTS)
def test_encode_brute_force_nearest_even(fmt, tdt):
    """Round to nearest grid value, ties to the even mantissa, by exhaustive search."""
    dec = O.fp8_decode_table(fmt)
    grid = [(b, float(dec[b])) for b in range(256) if np.isfinite(dec[b]) and not (b == 0x80)]
    mx = O.FP8_MAX[fmt]
    rng = np.random.default_rng(0)
    # random values plus every exact midpoint between neighbours
    pos = sorted({v for _, v in grid if v >= 0})
    mids = [(pos[i] + pos[i + 1]) / 2 for i in range(len(pos) - 1)]
    vals = np.concatenate([rng.uniform(-mx, mx, 4000), np.array(mids), -np.array(mids)]).astype(np.float32)
    for v in vals:
        v = float(v)
        best = min(grid, key=lambda bv: (abs(bv[1] - v), bv[0] & 1))  # nearest, then even code
        got = O.fp8_encode_scalar(v, fmt)
        assert dec[got] == best[1], (v, got, best)


@pytest.mark.parametrize("fmt,tdt", FMTS)
def test_decode_matches_torch(fmt, tdt):
    dec = O.fp8_decode_table(fmt)
    th = torch.arange(256, dtype=torch.uint8).view(tdt).float().numpy()
    both_nan = np.isnan(dec) & np.isnan(th)
    assert np.array_equal(dec[~both_nan], th[~both_nan])


@pytest.mark.parametrize("fmt", [0, 1])
def test_tensorwise_known_answers(fmt):
    mx = O.FP8_MAX[fmt]
    x = np.array([mx, -0.5, 1.0, 3.0], np.float32)
    q, s = O.quant_tensorwise(x, fmt)
    assert float(s) == 1.0
    assert q.tolist() == [O.fp8_encode_scalar(float(v), fmt) for v in x]
    q, s = O.quant_tensorwise(np.array([1.0, -0.25], np.float32), fmt)
    assert float(s) == np.float32(1.0) / np.float32(mx)
    q, s = O.quant_tensorwise(np.zeros(7, np.float32), fmt)  # eps branch
    assert float(s) == np.float32(1.0) / (np.float32(mx) / np.float32(1e-12))
    assert not q.any()


@pytest.mark.parametrize("fmt", [0, 1])
def test_tensorwise_scale_is_ieee_and_amax_maps_to_max(fmt):
    x = torch.randn(4096, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    q, s = O.quant_tensorwise(x, fmt)
    xf = O.to_float32(x)
    amax = np.float32(np.max(np.abs(xf)))
    scale_t = torch.tensor(O.FP8_MAX[fmt], dtype=torch.float32) / torch.tensor(amax)
    assert np.float32(s) == (torch.tensor(1.0) / scale_t).item()
    i = int(np.argmax(np.abs(xf)))
    assert abs(O.fp8_to_float(q[i], fmt)) == O.FP8_MAX[fmt]


@pytest.mark.parametrize("fmt", [0, 1])
def test_rowwise_equals_tensorwise_per_slice(fmt):
    x = torch.randn(6, 50, 7, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    q, s = O.quant_rowwise(x, fmt, 1)
    assert s.shape == (6, 1, 7)
    for b in range(6):
        for n in range(7):
            qs, ss = O.quant_tensorwise(x[b, :, n].contiguous(), fmt)
            assert np.array_equal(q[b, :, n], qs)
            assert np.float32(s[b, 0, n]) == np.float32(ss)


def test_block1d_locality_and_eps():
    x = torch.randn(300, 260, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    x[:128, :128] = 0  # one all-zero block per direction
    x[128:256, 128:256] *= 1e-6  # tiny blocks: amax below eps
    for axis in (0, 1):
        q, s = O.quant_block1d(x, 0, axis)
        if axis == 1:
            assert s[0, 0] == np.float32(1.0) / (np.float32(448.0) / np.float32(1e-4))
        y = x.clone()
        y[5, 200] = 100.0  # perturb one element
        q2, s2 = O.quant_block1d(y, 0, axis)
        diff_q = np.argwhere(q != q2)
        diff_s = np.argwhere(s != s2)
        if axis == 1:  # only row 5, column block 1 may change
            assert all(r == 5 and 128 <= c < 256 for r, c in diff_q)
            assert all(r == 5 and c == 1 for r, c in diff_s)
        else:  # only column 200, row block 0
            assert all(c == 200 and r < 128 for r, c in diff_q)
            assert all(r == 0 and c == 200 for r, c in diff_s)


def test_block_max_element_maps_to_max():
    x = torch.randn(256, 384, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    xf = O.to_float32(x)
    q, s = O.quant_block1d(x, 0, 1)
    for r in range(0, 256, 17):
        for j in range(3):
            blk = xf[r, 128 * j:128 * (j + 1)]
            i = int(np.argmax(np.abs(blk)))
            assert abs(O.fp8_to_float(q[r, 128 * j + i], 0)) == 448.0


def test_dual_and_weight_consistency():
    x = torch.randn(300, 260, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    qr, sr, qc, sc = O.quant_block_dual(x, 1)
    assert np.array_equal(qr, O.quant_block1d(x, 1, 1)[0])
    assert np.array_equal(qc, O.quant_block1d(x, 1, 0)[0])
    qw, sw = O.quant_block_weight(x, 0)
    assert sw.shape == (3, 3)
    for i in range(3):
        for j in range(3):
            tile = x[128 * i:128 * (i + 1), 128 * j:128 * (j + 1)].contiguous()
            qt, st = O.quant_tensorwise(tile, 0)  # eps differs, amax here >> 1e-4
            assert np.array_equal(qw[128 * i:128 * i + tile.shape[0], 128 * j:128 * j + tile.shape[1]], qt)
            assert np.float32(sw[i, j]) == np.float32(st)


def test_segment_equals_block1d_on_padded_groups():
    lens = [100, 0, 300, 128, 5]
    M, N = sum(lens), 200
    x = torch.randn(M, N, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    q_row, q_col, s_row_t, s_col, vk_lens, vk_offs = O.quant_block_segment(x, 0, lens)
    assert vk_lens.tolist() == [128, 0, 384, 128, 128]
    assert vk_offs.tolist() == [0, 128, 128, 512, 640, 768]
    qr, sr = O.quant_block1d(x, 0, 1)
    assert np.array_equal(q_row, qr)
    assert np.array_equal(s_row_t, sr.T)
    off = 0
    for g, L in enumerate(lens):
        P = vk_lens[g]
        if L:
            seg = torch.zeros(P, N, dtype=torch.bfloat16)
            seg[:L] = x[off:off + L]
            qc, sc = O.quant_block1d(seg, 0, 0)
            p0 = vk_offs[g]
            assert np.array_equal(q_col[p0:p0 + P], qc)
            assert np.array_equal(s_col[p0 // 128:(p0 + P) // 128], sc)
        off += L


@pytest.mark.parametrize("fmt,emax", [(0, 8), (1, 15)])
def test_mx_exponent_rule(fmt, emax):
    """E = floor(log2 amax) - emax, plus 1 when the mantissa of amax exceeds
    1.75 (amax * 2^-E would exceed fp8_max = 1.75 * 2^emax), biased by 127 and
    clamped to [0, 254]; restated here with float64 log2."""
    fmax = O.FP8_MAX[fmt]
    for amax in [1.0, 1.5, 1.75, 1.7500001, 1.76, 1.99, 2.0, 3.5, 3.51, 447.0, 448.0, 449.0, 3e-5, 1e30,
                 2.0 ** -126, 1.9 * 2.0 ** -126, 2.0 ** -130, fmax, fmax * 1.0001, 3.4e38]:
        a32 = float(np.float32(amax))
        fl = int(np.floor(np.log2(a32)))
        bump = 1 if a32 / 2.0 ** fl > 1.75 else 0
        exp = fl - emax + bump + 127
        assert O.mx_e8m0(a32, fmt) == min(max(exp, 0), 254), amax
    assert O.mx_e8m0(0.0, fmt) == 0
    x = (torch.exp(torch.randn(64, 256, generator=torch.Generator().manual_seed(7)) * 3)).to(torch.bfloat16)
    q, e = O.quant_mx(x, fmt, 1)
    assert q.shape == (64, 256) and e.shape == (64, 8)
    y = O.dequant_mx(q, fmt, e)
    xf = O.to_float32(x).astype(np.float64)
    sc = O.e8m0_to_scale(e).astype(np.float64)
    s_full = np.repeat(sc, 32, axis=1)
    # nothing saturates, and the block max lands in the top binade below fp8_max
    assert np.all(np.abs(xf) / s_full <= fmax)
    blk = np.abs(xf).reshape(64, 8, 32).max(-1) / sc
    assert np.all((blk > fmax / 2) & (blk <= fmax))
    # every element is the RNE value of x / scale (half a quantum, or half the
    # smallest subnormal)
    mbits, bias = (3, 7) if fmt == 0 else (2, 15)
    v = np.abs(xf) / s_full
    half_q = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(v, 1e-300))) - mbits - 1), 2.0 ** (1 - bias - mbits - 1))
    err = np.abs(y - xf) / s_full
    assert np.all(err <= half_q * (1 + 1e-12))


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("use_2d", [False, True])
def test_mx_rule_meets_reference_roundtrip_and_floor_rule_does_not(fmt, use_2d):
    """The reference's MX round-trip criterion (test_quantization.py:304-460:
    |x - dq(q(x))| <= 0.1 + 0.1 |dq(q(x))| on 1024 x 1024 N(0,1) inputs) holds
    for the oracle's rule, while the plain OCP floor rule (no bump, so block
    maxima with mantissa above 1.75 clamp to +-fp8_max) breaks it on the same
    input.  The planted rule lives here, on the CPU, only as the counter-case."""
    x = torch.randn(1024, 1024, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    xf = O.to_float32(x).astype(np.float64)
    q, e = O.quant_mx(x, fmt, 1, use_2d)
    y = O.dequant_mx(q, fmt, e)
    assert np.all(np.abs(xf - y) <= 0.1 + 0.1 * np.abs(y))
    # counter-case: floor rule; saturated elements dequantize to +-fp8_max * 2^E
    fmax, emax = O.FP8_MAX[fmt], (8 if fmt == 0 else 15)
    blocks = np.abs(xf).reshape(32, 32, 32, 32).max(axis=(1, 3)) if use_2d else np.abs(xf).reshape(1024, 32, 32).max(-1)
    E = np.floor(np.log2(blocks)) - emax
    if use_2d:
        E = np.repeat(np.repeat(E, 32, 0), 32, 1)
    else:
        E = np.repeat(E, 32, 1)
    sat = np.abs(xf) * 2.0 ** -E > fmax
    y_sat = np.sign(xf) * fmax * 2.0 ** E
    bad = sat & (np.abs(xf - y_sat) > 0.1 + 0.1 * np.abs(y_sat))
    assert bad.sum() > 0


def test_mx_padding_and_transpose_layout():
    x = torch.randn(176, 160, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    qr, er = O.quant_mx(x, 0, 1)
    qc, ec = O.quant_mx(x, 0, 0)
    assert qr.shape == (176, 256) and er.shape == (176, 8)
    assert qc.shape == (160, 256) and ec.shape == (160, 8)
    assert not qr[:, 160:].any() and not qc[:, 176:].any()


def test_gemm_ref_exact_on_integers():
    rng = np.random.default_rng(9)
    a = rng.integers(-8, 9, (37, 256)).astype(np.float64)
    b = rng.integers(-8, 9, (19, 256)).astype(np.float64)
    ref = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float64)
    assert np.array_equal(O.gemm_ref(a, b, False, True), ref)
    assert np.array_equal(O.gemm_ref(a.T.copy(), b, True, True, True), ref.T)


def test_reference_roundtrip_tolerance():
    x = torch.randn(512, 1024, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    xf = O.to_float32(x)
    q, s = O.quant_tensorwise(x, 0)
    np.testing.assert_allclose(O.dequant_tensorwise(q, 0, s), xf, rtol=0.1, atol=0.1)
    q, s = O.quant_rowwise(x, 0, -1)
    np.testing.assert_allclose(O.dequant_rowwise(q, 0, s), xf, rtol=0.1, atol=0.1)
    for axis in (0, 1):
        q, s = O.quant_block1d(x, 0, axis)
        np.testing.assert_allclose(O.dequant_block1d(q, 0, s, axis), xf, rtol=0.1, atol=0.1)


def test_grouped_mx_layout_and_locality():
    """Grouped MXFP8 layout (reference quantization.cpp:969-1195): per-group
    rows padded to 32 (rowwise) / 128 (colwise) with exclusive-prefix offsets;
    rowwise bytes of a group equal the ungrouped rowwise quantization of its
    rows; padding is zero; a colwise block never sees another group's rows."""
    import torch

    g = torch.Generator().manual_seed(5)
    x = (torch.randn(330, 96, generator=g) * 4).bfloat16()
    lens = [100, 0, 37, 193]
    qr, er, orw, qc, ec, oc = O.quant_mx_grouped(x, 0, lens)
    assert list(orw) == [0, 128, 128, 192, 416]
    assert list(oc) == [0, 128, 128, 256, 512]
    assert qr.shape == ((330 + 4 * 32 + 31) // 32 * 32, 128) and qc.shape == (96, (330 + 4 * 128 + 127) // 128 * 128)
    s = 0
    for gi, L in enumerate(lens):
        if L:
            q0, e0 = O.quant_mx(x[s:s + L], 0, 1)
            assert np.array_equal(qr[orw[gi]:orw[gi] + L], q0) and np.array_equal(er[orw[gi]:orw[gi] + L], e0)
            assert not qr[orw[gi] + L:orw[gi + 1]].any() and not er[orw[gi] + L:orw[gi + 1]].any()
            assert not qc[:, oc[gi] + L:oc[gi + 1]].any()
        s += L
    # locality: scaling group 3 by 2^10 leaves every colwise byte / exponent of groups 0-2 unchanged
    y = x.clone()
    y[137:] = (y[137:].float() * 1024).bfloat16()
    _, _, _, qc2, ec2, _ = O.quant_mx_grouped(y, 0, lens)
    assert np.array_equal(qc2[:, :256], qc[:, :256]) and np.array_equal(ec2[:, :8], ec[:, :8])
    assert not np.array_equal(ec2[:, 8:16], ec[:, 8:16])


def test_shuffle_e8m0_layout():
    """The scale shuffle moves byte (16 h + r, 4 q + c) of each 32 x 8 tile to
    offset 64 c + 4 r + 2 q + h, tiles in row-major order, padding to
    [roundup(M, 256), roundup(N, 8)] with zeros (shuffle.cu:12-73)."""
    rng = np.random.default_rng(5)
    e = rng.integers(1, 255, size=(70, 13), dtype=np.uint8)
    y = O.shuffle_e8m0(e)
    assert y.shape == (256, 16)
    flat = y.reshape(-1)
    tiles_per_row = 16 // 8
    for row in range(256):
        for col in range(16):
            tile = (row // 32) * tiles_per_row + col // 8
            h, r = divmod(row % 32, 16)
            q, c = divmod(col % 8, 4)
            exp = e[row, col] if row < 70 and col < 13 else 0
            assert flat[tile * 256 + 64 * c + 4 * r + 2 * q + h] == exp
