"""The allocation-free tensorwise quantize entry point
(pta_quantize_fp8_tensorwise_noalloc) against the workspace entry point
(pta_quantize_fp8_tensorwise), through the C ABI: FP8 bytes and scale_inv
bits must be identical.  Two calls in a row, the second on a smaller input
with a much smaller amax, so a call that read partial maxima left in the
static scratch by the previous one would produce a different scale."""

import pytest
import torch

pytestmark = pytest.mark.gpu

FMTS = [(torch.float8_e4m3fn, 0), (torch.float8_e5m2, 1)]


def _quant(_C, x, fmt_dtype, fmt, noalloc, scale=None):
    n = x.numel()
    q = torch.empty(x.shape, dtype=fmt_dtype, device=x.device)
    s_inv = torch.empty((), dtype=torch.float32, device=x.device)
    sp = None if scale is None else scale.data_ptr()
    dt = _C.in_dtype_code(x.dtype)
    st = _C.stream(x.device)
    if noalloc:
        _C.call("pta_quantize_fp8_tensorwise_noalloc", x.data_ptr(), dt, n, sp, q.data_ptr(), fmt, s_inv.data_ptr(),
                st)
    else:
        ws = torch.empty(_C.query("pta_quantize_fp8_tensorwise_workspace_size", n), dtype=torch.uint8,
                         device=x.device)
        _C.call("pta_quantize_fp8_tensorwise", x.data_ptr(), dt, n, sp, q.data_ptr(), fmt, s_inv.data_ptr(),
                ws.data_ptr(), ws.numel(), st)
    return q, s_inv


@pytest.mark.parametrize("fmt_dtype,fmt", FMTS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_noalloc_tensorwise_matches_workspace_entry(fmt_dtype, fmt, dtype):
    from primus_turbo.pytorch import _C

    g = torch.Generator().manual_seed(11)
    # first call: 40M elements (the amax pass uses all 2048 partials); second:
    # 4099 elements with values 100x smaller (2 partials), odd length and offset
    big = (torch.randn(40_000_003, generator=g) * 3.0).to(dtype).cuda()
    small = (torch.randn(4100, generator=g) * 0.03).to(dtype).cuda()[1:]
    for x in (big, small):
        q0, s0 = _quant(_C, x, fmt_dtype, fmt, noalloc=False)
        q1, s1 = _quant(_C, x, fmt_dtype, fmt, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(s0.view(torch.int32), s1.view(torch.int32)), f"scale_inv differs at n={x.numel()}"
        assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8)), f"fp8 bytes differ at n={x.numel()}"
    # with a caller-given scale (no amax pass, no scratch use)
    sc = torch.tensor(7.5, dtype=torch.float32, device="cuda")
    for x in (small, big[:1000]):
        q0, s0 = _quant(_C, x, fmt_dtype, fmt, noalloc=False, scale=sc)
        q1, s1 = _quant(_C, x, fmt_dtype, fmt, noalloc=True, scale=sc)
        torch.cuda.synchronize()
        assert torch.equal(s0.view(torch.int32), s1.view(torch.int32))
        assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8))


def test_noalloc_tensorwise_empty_and_bad_arguments():
    from primus_turbo.pytorch import _C

    x = torch.empty(0, dtype=torch.bfloat16, device="cuda")
    q0, s0 = _quant(_C, torch.ones(16, dtype=torch.bfloat16, device="cuda"), torch.float8_e4m3fn, 0, noalloc=True)
    torch.cuda.synchronize()
    assert float(s0) == (torch.tensor(1.0) / torch.tensor(448.0)).item() and torch.all(q0.float() == 448.0)
    with pytest.raises(RuntimeError, match="bad arguments"):
        _C.call("pta_quantize_fp8_tensorwise_noalloc", x.data_ptr() or 16, _C.PTA_BF16, -1, None, 16, 0, 16,
                _C.stream(x.device))
