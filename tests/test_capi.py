"""C ABI checks that need no GPU: the library loads, exports every entry point
that include/primus_turbo_amd.h declares, the Python binding table matches the
header, and argument validation fails before any device work."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "primus_turbo_amd.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(pta_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = _declared()
    assert "pta_gemm_fp8" in names and "pta_quantize_fp8_blockwise_dual" in names
    assert len(names) >= 25


def test_library_exports_every_declared_symbol():
    from primus_turbo.pytorch import _C

    lib = ctypes.CDLL(_C.lib_path())
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    from primus_turbo.pytorch import _C

    assert sorted(_C.SIGNATURES) == _declared()


def test_argument_errors_raise_without_gpu():
    from primus_turbo.pytorch import _C

    lib = _C.load()
    assert lib.pta_abi_version() == 6
    # NULL input: rejected on the host before any HIP call
    rc = lib.pta_quantize_fp8_blockwise(None, 2, 128, 128, 128, 1, None, None, 0, None)
    assert rc == -1
    assert b"NULL" in lib.pta_last_error()
    # unsupported block size
    rc = lib.pta_quantize_fp8_blockwise(ctypes.c_void_p(16), 2, 128, 128, 64, 1, None, None, 0, None)
    assert rc == -1 and b"block size" in lib.pta_last_error()
    # bad granularity for the GEMM
    rc = lib.pta_gemm_fp8(None, 0, None, 0, None, 0, None, 1, None, 2, 0, 1, 1, 16, 9, None, 0, None)
    assert rc == -1 and b"granularity" in lib.pta_last_error()
    with pytest.raises(RuntimeError, match="granularity"):
        _C.call("pta_gemm_fp8", None, 0, None, 0, None, 0, None, 1, None, 2, 0, 1, 1, 16, 9, None, 0, None)


def test_workspace_queries():
    from primus_turbo.pytorch import _C

    assert _C.query("pta_gemm_fp8_workspace_size", 128, 256, 512, 0, 1, 3) == 0
    # few tiles: the small-tile kernel reads K-major operands in place
    assert _C.query("pta_gemm_fp8_workspace_size", 128, 256, 512, 1, 0, 0) == 0
    # unless a K-major row stride is not a multiple of 8 (then both are transposed)
    assert _C.query("pta_gemm_fp8_workspace_size", 132, 256, 512, 1, 0, 0) >= 132 * 512 + 256 * 512
    # many tiles: the large-tile kernel reads NT copies
    assert _C.query("pta_gemm_fp8_workspace_size", 4096, 4096, 512, 1, 0, 0) >= 2 * 4096 * 512
    assert _C.query("pta_gemm_fp8_workspace_size", 4096, 4096, 512, 0, 0, 0) >= 4096 * 512
    assert _C.query("pta_quantize_fp8_rowwise_workspace_size", 4, 100, 1) == 0
    assert _C.query("pta_quantize_fp8_rowwise_workspace_size", 1, 100, 64) > 0
    # the K split: at most half a round of 256 x 256 tiles with K >= 4096 (one
    # fp32 256 x 256 partial tile per split tile); shorter K runs whole
    split = 256 * 256 * 4
    assert _C.query("pta_gemm_fp8_workspace_size", 2304, 3072, 4096, 0, 1, 1) >= 108 * split
    assert _C.query("pta_gemm_fp8_workspace_size", 2304, 3072, 2048, 0, 1, 1) == 0
    assert _C.query("pta_gemm_fp8_workspace_size", 4096, 18432, 7168, 0, 1, 3) == 0


def test_strided_entry_workspace_queries():
    """pta_gemm_fp8_nt_strided_ws_size(M, N, K, granularity, lda, ldb, sa_bytes,
    sb_bytes): 0 where the small-tile kernel or the whole 256 x 256 kernel runs,
    the split partials where the K split does (host-side rules, no GPU)."""
    from primus_turbo.pytorch import _C

    q = lambda *a: _C.query("pta_gemm_fp8_nt_strided_ws_size", *a)  # noqa: E731
    assert q(512, 1024, 1024, 1, 1024, 1024, 4, 4) == 0        # 8 tiles: small-tile kernel
    assert q(2048, 2048, 2048, 3, 2048, 2048, 4 << 20, 4 << 20) == 0  # blockwise on 128x128 tiles: whole
    assert q(2048, 2048, 2048, 1, 2048, 2048, 4, 4) == 0       # tensorwise: small-tile kernel
    assert q(2304, 3072, 2048, 3, 2048, 2048, 1 << 20, 1 << 20) == 0  # 108 tiles, K < 4096: whole
    assert q(2304, 3072, 4096, 3, 4096, 4096, 1 << 20, 1 << 20) >= 108 * 256 * 256 * 4  # K split
    assert q(1024, 4096, 4096, 4, 4096, 4096, 1 << 20, 1 << 20) >= 64 * 256 * 256 * 4   # 64 tiles, K >= 4096
    assert q(1024, 4096, 3072, 3, 3072, 3072, 1 << 20, 1 << 20) >= 64 * 256 * 256 * 4   # a quarter round: K >= 3072
    assert q(2304, 3072, 3072, 3, 3072, 3072, 1 << 20, 1 << 20) == 0  # 108 tiles at K = 3072: whole
    assert q(4096, 18432, 7168, 3, 7168, 7168, 1 << 20, 1 << 20) == 0  # the headline: whole tiles
    assert q(0, 1024, 1024, 1, 1024, 1024, 4, 4) == 0


def test_argument_errors_of_the_grouped_and_moe_entries():
    """Host-side argument checks of the newer entry points fire before any HIP
    call, with a message naming the problem (so no GPU is needed)."""
    from primus_turbo.pytorch import _C

    p = ctypes.c_void_p(256)  # never dereferenced: the checks reject first
    with pytest.raises(RuntimeError, match="unknown layout 7"):
        _C.call("pta_quantize_fp8_blockwise_segment_m_row_col", p, _C.PTA_BF16, 128, 128, 1, p, p, 128, p, p, p, p,
                p, p, _C.PTA_E4M3, 7, None)
    with pytest.raises(RuntimeError, match="MX_BLOCKWISE and BLOCKWISE"):
        _C.call("pta_grouped_gemm_fp8_variable_k_nt", p, 0, p, p, 0, p, p, 1, 128, 128, 128, p, _C.PTA_BF16, 0,
                _C.PTA_TENSORWISE, None)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        _C.call("pta_grouped_gemm_fp8_variable_k_nt", p, 0, p, p, 0, p, p, 1, 192, 128, 128, p, _C.PTA_BF16, 0,
                _C.PTA_BLOCKWISE, None)
    with pytest.raises(RuntimeError, match="num_local_experts"):
        _C.call("pta_moe_permute_preprocess", p, _C.MOE_MAP_BOOL, 16, 600, 0, 0, 16, 0, p, p, p, p, p, 1 << 20,
                None)


def test_wait_status_without_a_bounded_wait():
    """pta_last_wait_status reports offset -1 after a call that launched no
    bounded wait (here: one rejected on the host)."""
    from primus_turbo.pytorch import _C

    lib = _C.load()
    lib.pta_quantize_fp8_blockwise(None, 2, 128, 128, 128, 1, None, None, 0, None)
    tag, off = ctypes.c_uint64(7), ctypes.c_int64(7)
    assert lib.pta_last_wait_status(ctypes.byref(tag), ctypes.byref(off)) == 0
    assert off.value == -1
    assert lib.pta_last_wait_status(None, None) == -1
