"""The bounded cross-workgroup waits report a give-up.

The single-launch tensorwise quantize and the K split of the dense GEMM hand
data between workgroups through the caller's workspace and wait for it with a
bounded poll.  The test hook pta_test_force_wait_giveup makes every wait poll
for a tag that is never published, with a short limit, so each wait gives up
and every kernel still exits normally.  A give-up must show as NaN outputs,
as the call's tag in the workspace's status word (pta_last_wait_status), and
as a RuntimeError in the Python layer's debug mode; with the hook off the
same calls succeed and the status word does not hold the tag."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_f32_bitexact, f32, randn, u8

pytestmark = pytest.mark.gpu


@pytest.fixture
def forced():
    from primus_turbo.pytorch import _C

    _C.load().pta_test_force_wait_giveup(1)
    try:
        yield _C
    finally:
        _C.load().pta_test_force_wait_giveup(0)


def _tensorwise_call(_C, x):
    n = x.numel()
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device="cuda")
    s = torch.empty((), dtype=torch.float32, device="cuda")
    ws = _C.workspace(_C.query("pta_quantize_fp8_tensorwise_workspace_size", n), x.device)
    _C.call("pta_quantize_fp8_tensorwise", _C.ptr(x), _C.PTA_BF16, n, None, _C.ptr(q), _C.PTA_E4M3, _C.ptr(s),
            _C.ptr(ws), ws.numel(), _C.stream(x.device))
    tag, off = ctypes.c_uint64(0), ctypes.c_int64(-1)
    _C.load().pta_last_wait_status(ctypes.byref(tag), ctypes.byref(off))
    return q, s, ws, off.value


def test_tensorwise_single_launch_giveup(forced):
    _C = forced
    x = randn((1024, 1024), seed=1).cuda()  # 2^20 elements: the single-launch form
    q, s, ws, off = _tensorwise_call(_C, x)
    assert off >= 0 and off % 8 == 0, "the single-launch form has a bounded wait"
    assert _C.wait_gave_up(ws), "the status word must hold the call's tag"
    assert torch.isnan(s).item(), "a give-up makes the scale NaN"
    # the debug mode of the Python layer raises
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_fp8_tensorwise_impl

    old = _C.CHECK_WAITS
    _C.CHECK_WAITS = True
    try:
        with pytest.raises(RuntimeError, match="wait gave up"):
            quantize_fp8_tensorwise_impl(x, torch.float8_e4m3fn)
    finally:
        _C.CHECK_WAITS = old
    # hook off: the same call succeeds, bit-exact against the oracle
    _C.load().pta_test_force_wait_giveup(0)
    q, s, ws, off = _tensorwise_call(_C, x)
    assert off >= 0 and not _C.wait_gave_up(ws)
    oq, os_ = O.quant_tensorwise(x.cpu(), 0)
    assert np.array_equal(u8(q), oq)
    assert_f32_bitexact(f32(s).reshape(()), os_, "scale")


def test_gemm_k_split_giveup(forced):
    _C = forced
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_impl
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import quantize_fp8_tensorwise_impl

    M, N, K = 1024, 4096, 4096  # 64 tiles of 256 x 256 with K >= 3072: every tile is split
    _C.load().pta_test_force_wait_giveup(0)
    qa, sa = quantize_fp8_tensorwise_impl(randn((M, K), seed=2).cuda(), torch.float8_e4m3fn)
    qb, sb = quantize_fp8_tensorwise_impl(randn((N, K), seed=3).cuda(), torch.float8_e4m3fn)
    ref = gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, 1)
    assert torch.isfinite(ref).all()
    _C.load().pta_test_force_wait_giveup(1)
    old = _C.CHECK_WAITS
    _C.CHECK_WAITS = True
    try:
        with pytest.raises(RuntimeError, match="wait gave up"):
            gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, 1)
    finally:
        _C.CHECK_WAITS = old
    # the raw entry: every split tile's waiting half gives up -> NaN output, tag in the status word
    ws = _C.workspace(_C.query("pta_gemm_fp8_workspace_size", M, N, K, 0, 1, 1), qa.device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _C.call("pta_gemm_fp8", _C.ptr(qa), 0, _C.ptr(sa), 0, _C.ptr(qb), 0, _C.ptr(sb), 1, _C.ptr(out), _C.PTA_BF16, 0,
            M, N, K, 1, _C.ptr(ws), ws.numel(), _C.stream(qa.device))
    assert _C.wait_gave_up(ws)
    assert torch.isnan(out.float()).all()
    # hook off: the same call matches the earlier result bit for bit
    _C.load().pta_test_force_wait_giveup(0)
    out2 = gemm_fp8_impl(qa, sa, False, qb, sb, True, torch.bfloat16, False, 1)
    assert torch.equal(out2, ref)
