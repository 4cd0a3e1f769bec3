"""The matrix-pipe kernel bench.py measures the scaled GEMMs against
(primus-turbo_amd/bench/mfma_probe.hip, a library of its own): every variant
runs, folds finite accumulators, and every workgroup computes the same values
(its operands depend on the thread only); bad arguments are rejected."""

import os
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "primus-turbo_amd",
                                "bench"))


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_mfma_probe_runs(variant):
    import mfma_probe

    g = torch.Generator().manual_seed(variant)
    ops = torch.randn(mfma_probe.OPERAND_BYTES, generator=g).to(torch.float8_e4m3fn).view(torch.uint8).cuda()
    wgs = 3
    out = torch.full((wgs * mfma_probe.THREADS + 64,), float("nan"), dtype=torch.float32, device="cuda")
    mfma_probe.probe(variant, 4, wgs, ops, out, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    res = out[: wgs * mfma_probe.THREADS].view(wgs, mfma_probe.THREADS)
    assert bool(torch.isfinite(res).all())
    assert bool((res != 0).any())
    assert torch.equal(res[0], res[1]) and torch.equal(res[0], res[2])
    assert bool(torch.isnan(out[wgs * mfma_probe.THREADS:]).all()), "floats past the output were written"


def test_mfma_probe_rejects_bad_arguments():
    import mfma_probe

    ops = torch.zeros(mfma_probe.OPERAND_BYTES, dtype=torch.uint8, device="cuda")
    out = torch.empty(mfma_probe.THREADS, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(RuntimeError):
        mfma_probe.probe(4, 1, 1, ops, out, s)
    with pytest.raises(RuntimeError):
        mfma_probe.probe(0, 0, 1, ops, out, s)
    with pytest.raises(ValueError):
        mfma_probe.probe(0, 1, 2, ops, out, s)
    with pytest.raises(ValueError):
        mfma_probe.probe(0, 1, 1, ops[:100], out, s)
