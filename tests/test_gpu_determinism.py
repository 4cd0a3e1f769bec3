"""Run-to-run determinism of gemm_fp8 forward + backward for every scaling
granularity, on the reference's determinism grids
(tests/pytorch/ops/test_gemm_fp8.py:120-214 and :574-661): ten runs of
forward and backward on the same inputs give bit-identical C, dA and dB, and
the first run meets the reference's end-to-end criterion (SNR against an
unquantized matmul > 25 dB for e4m3, > 20 dB for e5m2 / HYBRID).

The reference has no MX determinism grid; the MX case here uses the MX GEMM's
own constraints (NT only) on a grid of the same sizes.  The unquantized
reference runs in fp32 on contiguous operands."""

import pytest
import torch

pytestmark = pytest.mark.gpu

REPEATS = 10


def _snr_db(ref, out):
    ref, out = ref.double(), out.double()
    noise = (ref - out).pow(2).sum()
    return float(10.0 * torch.log10(ref.pow(2).sum() / noise.clamp_min(1e-300)))


def _run(m, n, k, layout, fmt_name, dtype, gran_name, block_size):
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScaleDtype, ScalingGranularity

    gran = getattr(ScalingGranularity, gran_name)
    fmt = getattr(Format, fmt_name)
    torch.manual_seed(42)
    torch.cuda.manual_seed(42)
    ta, tb = layout[0] == "T", layout[1] == "T"
    a0 = torch.randn((k, m) if ta else (m, k), dtype=dtype, device="cuda")
    b0 = torch.randn((n, k) if tb else (k, n), dtype=dtype, device="cuda")
    # unquantized fp32 reference, contiguous operands
    a_ref = a0.float().requires_grad_()
    b_ref = b0.float().requires_grad_()
    am = (a_ref.t() if ta else a_ref).contiguous()
    bm = (b_ref.t() if tb else b_ref).contiguous()
    c_ref = am @ bm
    grad_c = torch.randn(c_ref.shape, dtype=dtype, device="cuda")
    c_ref.backward(grad_c.float())
    if block_size is not None:
        sd = ScaleDtype.E8M0 if gran == ScalingGranularity.MX_BLOCKWISE else ScaleDtype.FP32
        cfg = Float8QuantConfig(granularity=gran, format=fmt, block_size=block_size, scale_dtype=sd)
    else:
        cfg = Float8QuantConfig(granularity=gran, format=fmt)

    outs = []
    for _ in range(REPEATS):
        a = a0.detach().clone().requires_grad_()
        b = b0.detach().clone().requires_grad_()
        c = turbo.ops.gemm_fp8(a, b, ta, tb, dtype, cfg)
        c.backward(grad_c)
        outs.append((c.detach(), a.grad.detach(), b.grad.detach()))
        torch.cuda.synchronize()
    c0, da0, db0 = outs[0]
    for ci, dai, dbi in outs[1:]:
        assert torch.equal(c0, ci), "C differs between runs"
        assert torch.equal(da0, dai), "dA differs between runs"
        assert torch.equal(db0, dbi), "dB differs between runs"
    thr = 25.0 if fmt == Format.E4M3 else 20.0
    for what, r, o in (("C", c_ref, c0), ("dA", a_ref.grad, da0), ("dB", b_ref.grad, db0)):
        s = _snr_db(r.detach(), o.float())
        assert s > thr, f"{what} SNR {s:.1f} dB <= {thr}"


@pytest.mark.parametrize("m", [255, 507, 1032, 2056])
@pytest.mark.parametrize("n", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("k", [256, 512, 576, 1024, 2048])
@pytest.mark.parametrize("layout", ["NN", "NT"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fp8_tensorwise_deterministic(m, n, k, layout, fmt, dtype):
    _run(m, n, k, layout, fmt, dtype, "TENSORWISE", None)


@pytest.mark.parametrize("m", [255, 507, 1032, 2056])
@pytest.mark.parametrize("n", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("k", [256, 512, 576, 1024, 2048])
@pytest.mark.parametrize("layout", ["NN", "NT"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fp8_rowwise_deterministic(m, n, k, layout, fmt, dtype):
    _run(m, n, k, layout, fmt, dtype, "ROWWISE", None)


@pytest.mark.parametrize("m", [255, 257, 512, 1024])
@pytest.mark.parametrize("n", [256, 512, 1024, 4096])
@pytest.mark.parametrize("k", [256, 1024, 4096])
@pytest.mark.parametrize("layout", ["NT", "NN"])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fp8_blockwise_deterministic(m, n, k, layout, fmt, dtype):
    _run(m, n, k, layout, fmt, dtype, "BLOCKWISE", 128)


@pytest.mark.parametrize("m", [256, 512, 1024])
@pytest.mark.parametrize("n", [256, 1024, 4096])
@pytest.mark.parametrize("k", [256, 1024, 4096])
@pytest.mark.parametrize("fmt", ["E4M3", "E5M2", "HYBRID"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fp8_mx_deterministic(m, n, k, fmt, dtype):
    _run(m, n, k, "NT", fmt, dtype, "MX_BLOCKWISE", 32)
