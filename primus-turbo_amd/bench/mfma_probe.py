"""ctypes loader of libpta_mfma_probe.so, the register-only matrix-pipe kernel
bench.py times beside the scaled GEMM kernels (mfma_probe.hip).  Measurement
tooling: not part of the product library or its C ABI."""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpta_mfma_probe.so")
_lib = None

# variant -> (scale granularity whose main-loop work it carries, MFMAs' extra VALU)
VARIANTS = {
    0: "tensorwise / rowwise: MFMA only",
    1: "blockwise 1x128 x 128x128: MFMA into a fresh partial + 4 FMA",
    2: "blockwise 1x128 x 1x128: MFMA into a fresh partial + 4 multiply + 4 FMA",
    3: "MX: scaled MFMA (E8M0 exponents)",
}
THREADS = 512
OPERAND_BYTES = 4096 * 32


def flops(iters: int, workgroups: int) -> float:
    """Matrix work of one launch: 8 waves per workgroup, each 32 MFMAs of 16x16x128 per iteration."""
    return 2.0 * workgroups * 8 * iters * 64 * 128 * 128


def probe(variant: int, iters: int, workgroups: int, operands, out, stream: int) -> None:
    """One launch on `stream`; operands: OPERAND_BYTES of fp8 bytes, out:
    workgroups * THREADS floats (torch device tensors); raises on failure."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C primus-turbo_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        lib.pta_bench_mfma_probe.restype = ctypes.c_int
        lib.pta_bench_mfma_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_void_p]
        _lib = lib
    if operands.numel() * operands.element_size() < OPERAND_BYTES:
        raise ValueError("operands must hold OPERAND_BYTES bytes")
    if out.numel() < workgroups * THREADS or out.element_size() != 4:
        raise ValueError("out must hold workgroups * THREADS floats")
    rc = _lib.pta_bench_mfma_probe(variant, iters, workgroups, operands.data_ptr(), out.data_ptr(), stream)
    if rc != 0:
        raise RuntimeError(f"pta_bench_mfma_probe failed ({rc})")
