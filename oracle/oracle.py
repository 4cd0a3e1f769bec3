"""CPU oracle for the FP8 linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``primus-turbo_amd/primus_turbo``) never imports it.

Two layers:

* ``liboracle.so`` (``oracle/fp8_oracle.c``): scalar C restatement of the
  reference's quantization arithmetic, bit for bit (see the header of that file
  for the reference lines each function follows).
* numpy helpers below: dequantization of every scale layout and an fp64 GEMM
  reference.  Blockwise / MX scales are constant inside a 128- or 32-wide
  K block, so ``sum_kb (sum_k a_q b_q) sa sb`` equals ``sum_k (a_q sa)(b_q sb)``
  exactly in real arithmetic; products of two fp8 values need at most 8
  significant bits and a 128-term fp8 dot product spans < 53 bits, so each
  per-block partial sum is exact in fp64 and the fp64 matmul of the dequantized
  operands carries the reference's partial-sum-then-scale structure
  (primus_turbo/triton/gemm/gemm_fp8_kernel.py:
  934-964); the only rounding left is fp64's own (~1e-16 relative), far below
  any tolerance used against it.

Pinning status of each function is documented in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

FMT_E4M3 = 0
FMT_E5M2 = 1
FP8_MAX = {FMT_E4M3: 448.0, FMT_E5M2: 57344.0}

IN_F32, IN_F16, IN_BF16 = 0, 1, 2

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.or_fp8_from_float.restype = ctypes.c_uint8
        L.or_fp8_from_float.argtypes = [ctypes.c_float, i32]
        L.or_fp8_to_float.restype = ctypes.c_float
        L.or_fp8_to_float.argtypes = [ctypes.c_uint8, i32]
        L.or_quant_tensorwise.argtypes = [vp, i32, i64, i32, vp, vp]
        L.or_quant_rowwise.argtypes = [vp, i32, i64, i64, i64, i32, vp, vp]
        L.or_quant_block1d.argtypes = [vp, i32, i64, i64, i64, i32, i32, vp, vp]
        L.or_quant_block_weight.argtypes = [vp, i32, i64, i64, i64, i64, i32, vp, vp]
        L.or_quant_block_segment.argtypes = [vp, i32, i64, i64, i64, vp, i64, i32, vp, vp, vp, vp, vp, vp]
        L.or_quant_mx.argtypes = [vp, i32, i64, i64, i64, i32, i32, i32, vp, vp]
        L.or_mx_e8m0.restype = i32
        L.or_mx_e8m0.argtypes = [ctypes.c_float, i32]
        L.or_e8m0_to_scale.restype = ctypes.c_float
        L.or_e8m0_to_scale.argtypes = [ctypes.c_uint8]
        _lib = L
    return _lib


# ---------------------------------------------------------------------------
# input normalisation: accept torch CPU tensors or numpy arrays
# ---------------------------------------------------------------------------
def _as_raw(x):
    """Return (contiguous numpy array holding the raw bits, in_dt code)."""
    try:
        import torch

        if isinstance(x, torch.Tensor):
            x = x.detach().cpu().contiguous()
            if x.dtype == torch.bfloat16:
                return x.view(torch.int16).numpy().view(np.uint16), IN_BF16
            if x.dtype == torch.float16:
                return x.view(torch.int16).numpy().view(np.uint16), IN_F16
            if x.dtype == torch.float32:
                return x.numpy(), IN_F32
            raise TypeError(f"unsupported dtype {x.dtype}")
    except ImportError:  # pragma: no cover
        pass
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return x, IN_F32
    if x.dtype == np.float16:
        return x.view(np.uint16), IN_F16
    raise TypeError(f"unsupported numpy dtype {x.dtype}")


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def to_float32(x):
    """Exact fp32 values of a bf16/fp16/fp32 input."""
    raw, dt = _as_raw(x)
    if dt == IN_F32:
        return raw.astype(np.float32)
    if dt == IN_F16:
        return raw.view(np.float16).astype(np.float32)
    return (raw.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# fp8 codec
# ---------------------------------------------------------------------------
def fp8_encode_scalar(v: float, fmt: int) -> int:
    return int(lib().or_fp8_from_float(ctypes.c_float(v), fmt))


def fp8_decode_table(fmt: int) -> np.ndarray:
    L = lib()
    return np.array([L.or_fp8_to_float(b, fmt) for b in range(256)], dtype=np.float32)


_DEC = {}


def fp8_to_float(q: np.ndarray, fmt: int) -> np.ndarray:
    if fmt not in _DEC:
        _DEC[fmt] = fp8_decode_table(fmt)
    return _DEC[fmt][np.asarray(q, dtype=np.uint8)]


# ---------------------------------------------------------------------------
# quantizers (bit-exact restatements, see fp8_oracle.c)
# ---------------------------------------------------------------------------
def quant_tensorwise(x, fmt):
    raw, dt = _as_raw(x)
    q = np.empty(raw.shape, np.uint8)
    s = np.zeros((), np.float32)
    lib().or_quant_tensorwise(_p(raw), dt, raw.size, fmt, _p(q), _p(s))
    return q, s


def quant_rowwise(x, fmt, axis):
    raw, dt = _as_raw(x)
    shape = raw.shape
    axis = axis % len(shape)
    B = int(np.prod(shape[:axis], dtype=np.int64))
    L = int(shape[axis])
    N = int(np.prod(shape[axis + 1 :], dtype=np.int64))
    q = np.empty(shape, np.uint8)
    sshape = list(shape)
    sshape[axis] = 1
    s = np.empty(sshape, np.float32)
    lib().or_quant_rowwise(_p(raw), dt, B, L, N, fmt, _p(q), _p(s))
    return q, s


def quant_block1d(x, fmt, axis, block=128):
    raw, dt = _as_raw(x)
    M, N = raw.shape
    axis = axis % 2
    q = np.empty((M, N), np.uint8)
    s = np.empty((M, -(-N // block)) if axis == 1 else (-(-M // block), N), np.float32)
    lib().or_quant_block1d(_p(raw), dt, M, N, block, axis, fmt, _p(q), _p(s))
    return q, s


def quant_block_dual(x, fmt, block=128):
    qr, sr = quant_block1d(x, fmt, 1, block)
    qc, sc = quant_block1d(x, fmt, 0, block)
    return qr, sr, qc, sc


def quant_block_weight(x, fmt, block=128):
    raw, dt = _as_raw(x)
    squeeze = raw.ndim == 2
    r3 = raw[None] if squeeze else raw
    B, M, N = r3.shape
    q = np.empty((B, M, N), np.uint8)
    s = np.empty((B, -(-M // block), -(-N // block)), np.float32)
    lib().or_quant_block_weight(_p(np.ascontiguousarray(r3)), dt, B, M, N, block, fmt, _p(q), _p(s))
    if squeeze:
        return q[0], s[0]
    return q, s


def quant_block_segment(x, fmt, group_lens, block=128):
    """Returns (q_row, q_col_pad, s_row_t, s_col_pad, vk_lens, vk_offs, valid_pad_rows).

    Rows of q_col_pad at or beyond ``vk_offs[-1]`` and scale rows beyond the
    padded tiles are left as 0 here; the reference leaves them unwritten.
    """
    raw, dt = _as_raw(x)
    M, N = raw.shape
    lens = np.ascontiguousarray(np.asarray(group_lens, dtype=np.int64))
    G = lens.size
    Mpad_max = M + G * block
    q_row = np.zeros((M, N), np.uint8)
    q_col = np.zeros((Mpad_max, N), np.uint8)
    s_row = np.zeros((-(-N // block), M), np.float32)
    s_col = np.zeros((-(-Mpad_max // block), N), np.float32)
    vk_lens = np.zeros(G, np.int64)
    vk_offs = np.zeros(G + 1, np.int64)
    lib().or_quant_block_segment(
        _p(raw), dt, M, N, G, _p(lens), block, fmt, _p(q_row), _p(q_col), _p(s_row), _p(s_col),
        _p(vk_lens), _p(vk_offs),
    )
    return q_row, q_col, s_row, s_col, vk_lens, vk_offs


def quant_mx(x, fmt, direction, use_2d=False):
    """direction 1 = rowwise, 0 = colwise (transposed output).  x is [M,N] or [G,M,N]."""
    raw, dt = _as_raw(x)
    return _quant_mx_raw(raw, dt, fmt, direction, use_2d)


def _quant_mx_raw(raw, dt, fmt, direction, use_2d=False):
    batched = raw.ndim == 3
    r3 = raw if batched else raw[None]
    G, M, N = r3.shape
    Mp, Np = -(-M // 128) * 128, -(-N // 128) * 128
    if direction == 1:
        q = np.empty((G * M, Np), np.uint8)
        e = np.empty((G * M, Np // 32), np.uint8)
    else:
        q = np.empty((G * N, Mp), np.uint8)
        e = np.empty((G * N, Mp // 32), np.uint8)
    lib().or_quant_mx(_p(np.ascontiguousarray(r3)), dt, G, M, N, direction, int(use_2d), fmt, _p(q), _p(e))
    if batched:
        q = q.reshape(G, -1, q.shape[-1])
        e = e.reshape(G, -1, e.shape[-1])
    return q, e


def quant_mx_grouped(x, fmt, group_lens):
    """Grouped MXFP8 of x[M, N] (rows split by group_lens): each group is
    zero-padded along M to 32 rows (rowwise output) and to 128 (colwise,
    transposed), the layout of grouped_quantize_mxfp8(_dual) in the reference
    (csrc/pytorch/quantization/quantization.cpp:969-1195).  Composed from
    quant_mx on each padded group, so each block sees exactly the rows of one
    group plus zeros.  Returns (q_row [Mr, Np], e_row, offs_row, q_col [N, Mc],
    e_col, offs_col) with rows / columns outside every group left at 0."""
    raw, dt = _as_raw(x)
    M, N = raw.shape
    lens = [int(v) for v in group_lens]
    G = len(lens)
    Mr = -(-(M + 32 * G) // 32) * 32
    Mc = -(-(M + 128 * G) // 128) * 128
    Np = -(-N // 128) * 128
    q_row = np.zeros((Mr, Np), np.uint8)
    e_row = np.zeros((Mr, Np // 32), np.uint8)
    q_col = np.zeros((N, Mc), np.uint8)
    e_col = np.zeros((N, Mc // 32), np.uint8)
    offs_row, offs_col = [0], [0]
    s = 0
    for L in lens:
        pr, pc = -(-L // 32) * 32, -(-L // 128) * 128
        if L:
            seg = raw[s:s + L]
            pad_c = np.zeros((pc, N), raw.dtype)
            pad_c[:L] = seg
            qr, er = _quant_mx_raw(np.ascontiguousarray(pad_c[:pr]), dt, fmt, 1)
            qc, ec = _quant_mx_raw(pad_c, dt, fmt, 0)
            q_row[offs_row[-1]:offs_row[-1] + pr] = qr[:, :Np]
            e_row[offs_row[-1]:offs_row[-1] + pr] = er
            q_col[:, offs_col[-1]:offs_col[-1] + pc] = qc[:, :pc]
            e_col[:, offs_col[-1] // 32:(offs_col[-1] + pc) // 32] = ec[:, :pc // 32]
        offs_row.append(offs_row[-1] + pr)
        offs_col.append(offs_col[-1] + pc)
        s += L
    return q_row, e_row, np.array(offs_row, np.int64), q_col, e_col, np.array(offs_col, np.int64)


def shuffle_e8m0(e) -> np.ndarray:
    """E8M0 16 x 16 MFMA scale shuffle (csrc/kernels/shuffle/shuffle.cu:12-73,
    padding csrc/pytorch/shuffle/shuffle_meta.cpp:13-29): pad e[M, N] with zeros
    to [roundup(M, 256), roundup(N, 8)], cut it into 32 x 8 tiles in row-major
    tile order, and inside a tile write row 16*i1 + i2, column 4*i4 + i5 at
    byte 64*i5 + 4*i2 + 2*i4 + i1 (the (i1, i2, i4, i5) -> (i5, i2, i4, i1)
    index permutation of the reference's comment)."""
    e = np.asarray(e, np.uint8)
    M, N = e.shape
    Mp, Np = -(-M // 256) * 256, -(-N // 8) * 8
    p = np.zeros((Mp, Np), np.uint8)
    p[:M, :N] = e
    # [tile_row, i1, i2, tile_col, i4, i5] -> [tile_row, tile_col, i5, i2, i4, i1]
    t = p.reshape(Mp // 32, 2, 16, Np // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1)
    return np.ascontiguousarray(t).reshape(Mp, Np)


def mx_e8m0(amax: float, fmt: int) -> int:
    return int(lib().or_mx_e8m0(ctypes.c_float(amax), fmt))


def e8m0_to_scale(e: np.ndarray) -> np.ndarray:
    """bits(e << 23) as fp32 (e == 0 -> 0.0, e == 255 -> inf)."""
    return (np.asarray(e, dtype=np.uint32) << 23).view(np.float32)


# ---------------------------------------------------------------------------
# dequantization to float64 (exact: fp8 * fp32 fits in fp64).  The reference
# multiplies in fp32 and then casts to the output type
# (csrc/kernels/quantization/quantization_tensorwise.cu:36-42), so a caller
# rounds these to float32 first and then to the output dtype.
# ---------------------------------------------------------------------------
def dequant_tensorwise(q, fmt, s):
    return fp8_to_float(q, fmt).astype(np.float64) * np.float64(np.asarray(s, np.float32))


def dequant_rowwise(q, fmt, s):
    return fp8_to_float(q, fmt).astype(np.float64) * np.asarray(s, np.float32).astype(np.float64)


def dequant_block1d(q, fmt, s, axis, block=128):
    v = fp8_to_float(q, fmt).astype(np.float64)
    M, N = v.shape
    s = np.asarray(s, np.float32).astype(np.float64)
    if axis % 2 == 1:
        full = np.repeat(s, block, axis=1)[:, :N]
    else:
        full = np.repeat(s, block, axis=0)[:M, :]
    return v * full


def dequant_block2d(q, fmt, s, block=128):
    v = fp8_to_float(q, fmt).astype(np.float64)
    s = np.asarray(s, np.float32).astype(np.float64)
    full = np.repeat(np.repeat(s, block, axis=-2), block, axis=-1)
    return v * full[..., : v.shape[-2], : v.shape[-1]]


def dequant_mx(q, fmt, e, block=32):
    """q[..., R, C] with e[..., R, C/32] along the last axis."""
    v = fp8_to_float(q, fmt).astype(np.float64)
    sc = e8m0_to_scale(e).astype(np.float64)
    return v * np.repeat(sc, block, axis=-1)[..., : v.shape[-1]]


# ---------------------------------------------------------------------------
# GEMM references (fp64)
# ---------------------------------------------------------------------------
def gemm_ref(a_deq: np.ndarray, b_deq: np.ndarray, trans_a: bool, trans_b: bool, trans_c: bool = False):
    """C = op(A) @ op(B) in float64 on dequantized operands."""
    A = a_deq.T if trans_a else a_deq
    B = b_deq.T if trans_b else b_deq
    C = A @ B
    return C.T if trans_c else C


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float64/float32 values to bf16 (RNE) and return them as float32."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(f)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def snr_db(ref: np.ndarray, out: np.ndarray) -> float:
    ref = np.asarray(ref, np.float64)
    out = np.asarray(out, np.float64)
    noise = np.sum((ref - out) ** 2)
    sig = np.sum(ref**2)
    if noise == 0:
        return float("inf")
    return float(10.0 * np.log10(sig / noise))


def max_rel_err(ref: np.ndarray, out: np.ndarray) -> float:
    ref = np.asarray(ref, np.float64)
    out = np.asarray(out, np.float64)
    den = np.max(np.abs(ref))
    if den == 0:
        return float(np.max(np.abs(out)))
    return float(np.max(np.abs(ref - out)) / den)
