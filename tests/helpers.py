"""Shared test helpers: seeded inputs, the reference-kernel driver, byte comparison."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_quant.so")

FMT = {torch.float8_e4m3fn: 0, torch.float8_e5m2: 1}


def randn(shape, dtype=torch.bfloat16, seed=0, scale=1.0, outliers=0.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32) * scale
    if outliers:
        n = x.numel()
        k = max(1, int(n * outliers))
        idx = torch.randperm(n, generator=g)[:k]
        x.view(-1)[idx] *= 50.0
    return x.to(dtype).to(device)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().contiguous().cpu().numpy()


def assert_bytes_equal(got: np.ndarray, exp: np.ndarray, what: str):
    got = np.asarray(got)
    exp = np.asarray(exp)
    assert got.shape == exp.shape, f"{what}: shape {got.shape} != {exp.shape}"
    bad = np.nonzero(got.reshape(-1) != exp.reshape(-1))[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at flat index {bad[:5]}: {got.reshape(-1)[bad[:5]]} vs {exp.reshape(-1)[bad[:5]]}"


def assert_f32_bitexact(got: np.ndarray, exp: np.ndarray, what: str):
    g = np.ascontiguousarray(got, dtype=np.float32).view(np.uint32)
    e = np.ascontiguousarray(exp, dtype=np.float32).view(np.uint32)
    assert_bytes_equal(g, e, what)


_ref = None


def ref_lib():
    """ctypes handle of the reference's own quantization kernels (oracle/_ref), or None."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        L = ctypes.CDLL(REF_LIB)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.ref_tensorwise_ws_bytes.restype = i64
        L.ref_tensorwise_ws_bytes.argtypes = [i64]
        L.ref_quant_tensorwise.argtypes = [vp, i64, i32, vp, vp, vp, vp]
        L.ref_quant_rowwise_last.argtypes = [vp, i64, i64, i32, vp, vp, vp, vp]
        L.ref_rowwise_col_ws_bytes.restype = i64
        L.ref_rowwise_col_ws_bytes.argtypes = [i64, i64, i64]
        L.ref_quant_rowwise_col.argtypes = [vp, i64, i64, i64, i32, vp, vp, vp, vp, vp]
        L.ref_quant_weight.argtypes = [vp, i64, i64, i64, i32, vp, vp, vp]
        L.ref_quant_segment.argtypes = [vp, i64, i64, i64, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp]
        if hasattr(L, "ref_shuffle_e8m0"):
            L.ref_shuffle_e8m0.argtypes = [vp, i64, i64, vp, vp]
        else:  # an older build of oracle/_ref without the shuffle kernel
            L.ref_shuffle_e8m0 = None
        if hasattr(L, "ref_moe_preprocess"):
            L.ref_moe_preprocess.argtypes = [vp, i32, i64, i32, i32, i32, i64, i32, vp, vp, vp, vp, vp]
            L.ref_moe_permute.argtypes = [vp, vp, i32, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]
            L.ref_moe_unpermute.argtypes = [vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, vp]
        else:  # an older build of oracle/_ref without the MoE permutation kernels
            L.ref_moe_preprocess = None
        if hasattr(L, "ref_dequant_mxfp8"):
            L.ref_dequant_mxfp8.argtypes = [vp, i32, i64, i64, vp, i64, i64, i32, vp, i32, vp]
            L.ref_transpose_2d.argtypes = [vp, vp, i64, i64, i64, i64, vp]
        else:  # an older build of oracle/_ref without the MX dequant / transpose kernels
            L.ref_dequant_mxfp8 = None
            L.ref_transpose_2d = None
        _ref = L
    return _ref


def stream():
    return torch.cuda.current_stream().cuda_stream
