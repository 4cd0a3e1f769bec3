"""ctypes loader of libpta_stream_probe.so, the streaming kernel bench.py
times beside each quantize kernel (stream_probe.hip).  Measurement tooling:
not part of the product library or its C ABI."""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpta_stream_probe.so")
_lib = None


def probe(src, dst, write_bytes: int, read_ratio: int, nontemporal: int, stream: int) -> None:
    """Stream write_bytes into dst (torch uint8 device tensors) reading
    read_ratio * write_bytes from src, on `stream`; raises on failure."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C primus-turbo_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        lib.pta_bench_stream_probe.restype = ctypes.c_int
        lib.pta_bench_stream_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_void_p]
        _lib = lib
    rc = _lib.pta_bench_stream_probe(src.data_ptr(), dst.data_ptr(), write_bytes, read_ratio, nontemporal, stream)
    if rc != 0:
        raise RuntimeError(f"pta_bench_stream_probe failed ({rc})")
