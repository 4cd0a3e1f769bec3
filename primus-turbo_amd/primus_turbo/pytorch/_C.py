"""ctypes binding of ``libprimus_turbo_amd.so`` (C ABI: include/primus_turbo_amd.h).

The library is the only compute path: if it is missing, or no GPU is present,
every op raises.  There is no CPU or eager-PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libprimus_turbo_amd.so")

PTA_F32, PTA_F16, PTA_BF16 = 0, 1, 2
PTA_E4M3, PTA_E5M2 = 0, 1
PTA_TENSORWISE, PTA_ROWWISE, PTA_BLOCKWISE, PTA_MX_BLOCKWISE = 1, 2, 3, 4
# layout flags of pta_quantize_fp8_blockwise_dual
DUAL_COL_TRANSPOSED, DUAL_ROW_SCALE_KMAJOR = 1, 2
# exponent layout flag of pta_quantize_mxfp8
MX_EXP_KMAJOR = 1
# layout flag of pta_quantize_fp8_blockwise_segment_m_row_col
SEGMENT_COL_TRANSPOSED = 1
# expert_map kinds of pta_moe_permute_preprocess
MOE_MAP_BOOL, MOE_MAP_I32, MOE_MAP_I64 = 0, 1, 2

_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/primus_turbo_amd.h
SIGNATURES = {
    "pta_last_error": (ctypes.c_char_p, []),
    "pta_abi_version": (_i32, []),
    "pta_last_wait_status": (_i32, [ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int64)]),
    "pta_test_force_wait_giveup": (None, [_i32]),
    "pta_quantize_fp8_tensorwise_workspace_size": (_sz, [_i64]),
    "pta_quantize_fp8_tensorwise": (_i32, [_vp, _i32, _i64, _vp, _vp, _i32, _vp, _vp, _sz, _vp]),
    "pta_quantize_fp8_tensorwise_noalloc": (_i32, [_vp, _i32, _i64, _vp, _vp, _i32, _vp, _vp]),
    "pta_quantize_fp8_rowwise_workspace_size": (_sz, [_i64, _i64, _i64]),
    "pta_quantize_fp8_rowwise": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _sz, _vp]),
    "pta_quantize_fp8_blockwise": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _i32, _vp]),
    "pta_quantize_fp8_blockwise_dual": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "pta_quantize_fp8_blockwise_for_weight": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp]),
    "pta_quantize_fp8_blockwise_segment_m_row_col": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp],
    ),
    "pta_quantize_mxfp8": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp]),
    "pta_dequantize_fp8_tensorwise": (_i32, [_vp, _i32, _i64, _vp, _vp, _i32, _vp]),
    "pta_dequantize_fp8_rowwise": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp]),
    "pta_dequantize_fp8_blockwise": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _i32, _vp]),
    "pta_dequantize_mxfp8": (_i32, [_vp, _i32, _i64, _i64, _vp, _i32, _vp, _i32, _vp]),
    "pta_shuffle_e8m0_scale": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "pta_grouped_dequantize_mxfp8": (_i32, [_vp, _i32, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "pta_transpose_u8": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "pta_grouped_compute_offs": (_i32, [_vp, _vp, _i64, _vp]),
    "pta_grouped_compute_padded_offs": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "pta_gemm_fp8_workspace_size": (_sz, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "pta_gemm_fp8": (
        _i32,
        [_vp, _i32, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _i32, _i32, _i64, _i64, _i64, _i32, _vp, _sz, _vp],
    ),
    "pta_gemm_fp8_nt_strided": (
        _i32,
        [_vp, _i32, _i64, _vp, _i32, _i64, _vp, _i32, _i64, _i64, _i64, _i64, _i32,
         _vp, _i64, _i64, _i32, _i64, _vp, _i64, _i64, _i32, _i64, _vp],
    ),
    "pta_gemm_fp8_nt_strided_ws_size": (_sz, [_i64, _i64, _i64, _i32, _i64, _i64, _i64, _i64]),
    "pta_gemm_fp8_nt_strided_ws": (
        _i32,
        [_vp, _i32, _i64, _vp, _i32, _i64, _vp, _i32, _i64, _i64, _i64, _i64, _i32,
         _vp, _i64, _i64, _i32, _i64, _vp, _i64, _i64, _i32, _i64, _vp, _sz, _vp],
    ),
    "pta_grouped_gemm_fp8_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32, _i32]),
    "pta_grouped_gemm_fp8": (
        _i32,
        [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "pta_grouped_gemm_fp8_variable_k_nt": (
        _i32,
        [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _i32, _i32, _vp],
    ),
    "pta_grouped_quantize_mxfp8": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp],
    ),
    "pta_grouped_compute_padded_layout": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "pta_grouped_gemm_fp8_variable_k_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "pta_grouped_gemm_fp8_variable_k": (
        _i32,
        [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "pta_moe_permute_preprocess_workspace_size": (_sz, [_i64, _i32]),
    "pta_moe_permute_preprocess": (
        _i32,
        [_vp, _i32, _i64, _i32, _i32, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "pta_moe_permute": (
        _i32,
        [_vp, _i64, _i32, _i64, _vp, _i64, _vp, _i64, _vp, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _vp],
    ),
    "pta_moe_unpermute": (_i32, [_vp, _i64, _i32, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _vp]),
}

_lib = None
_lock = threading.Lock()


def lib_path() -> str:
    return _LIB_PATH


def load():
    """Load the native library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"primus_turbo native library not found at {_LIB_PATH}; build it with "
                    "`make -C primus-turbo_amd` (or __graft_entry__.build())"
                )
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_fns: dict = {}
_queries: dict = {}


def _fn(name: str):
    f = _fns.get(name)
    if f is None:
        f = _fns[name] = getattr(load(), name)
    return f


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise RuntimeError on failure."""
    rc = _fn(name)(*args)
    if rc != 0:
        msg = load().pta_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


# Debug mode (PRIMUS_TURBO_CHECK_WAITS=1): after each call that launched a
# bounded cross-workgroup wait, synchronize and raise if the wait gave up.
CHECK_WAITS = os.environ.get("PRIMUS_TURBO_CHECK_WAITS", "0") not in ("", "0")


def wait_gave_up(ws) -> bool:
    """Whether the last call on this thread launched a bounded wait that gave
    up (synchronizes the current stream).  ``ws`` is the uint8 workspace
    tensor that call was given."""
    tag, off = ctypes.c_uint64(0), ctypes.c_int64(-1)
    load().pta_last_wait_status(ctypes.byref(tag), ctypes.byref(off))
    if off.value < 0 or ws is None:
        return False
    torch.cuda.current_stream(ws.device).synchronize()
    word = ws[off.value:off.value + 8].cpu().view(torch.int64).item() & 0xFFFFFFFFFFFFFFFF
    return word == tag.value


def check_waits(name: str, ws) -> None:
    """In debug mode, raise RuntimeError if the last call's bounded wait gave up."""
    if CHECK_WAITS and wait_gave_up(ws):
        raise RuntimeError(f"{name}: a cross-workgroup wait gave up (outputs hold NaN); its workgroups "
                           "could not all run at once (concurrent work holding the CUs?)")


def query(name: str, *args) -> int:
    """A size query.  Answers are cached per (entry, arguments, current device):
    some sizes depend on the device as well (the GEMM workspaces hold the K
    split's partial tiles, whose use depends on the device's CU count)."""
    key = (name, args, _cur_device() if _gpu_checked else -1)
    v = _queries.get(key)
    if v is None:
        if len(_queries) >= 4096:  # shapes that vary per call (token counts) must not grow it forever
            _queries.clear()
        v = _queries[key] = int(_fn(name)(*args))
    return v


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


_gpu_checked = False
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_cur_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def stream(device=None) -> int:
    """Handle of torch's current stream on `device` (the stream every entry is launched on)."""
    global _gpu_checked
    if not _gpu_checked:
        if not torch.cuda.is_available():
            raise RuntimeError("primus_turbo FP8 ops need a ROCm GPU (torch.cuda.is_available() is False)")
        _gpu_checked = True
    if _raw_stream is not None:
        if device is not None and not isinstance(device, (torch.device, int)):
            device = torch.device(device)
        idx = device.index if isinstance(device, torch.device) else device
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def in_dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return PTA_BF16
    if dt == torch.float16:
        return PTA_F16
    if dt == torch.float32:
        return PTA_F32
    raise TypeError(f"unsupported high-precision dtype {dt}")


def fp8_code(dt: torch.dtype) -> int:
    if dt == torch.float8_e4m3fn:
        return PTA_E4M3
    if dt == torch.float8_e5m2:
        return PTA_E5M2
    raise TypeError(f"unsupported fp8 dtype {dt} (gfx950 uses OCP float8_e4m3fn / float8_e5m2)")


def out_dtype_code(dt: torch.dtype) -> int:
    return in_dtype_code(dt)


def workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)
