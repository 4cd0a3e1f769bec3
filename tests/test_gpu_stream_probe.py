"""The streaming kernel bench.py measures the quantize kernels against
(primus-turbo_amd/bench/stream_probe.hip, a library of its own): a copy writes the source bytes; read 2 write 1 writes the
XOR of each pair of 16-byte source chunks; every byte of the destination is
written and nothing past it."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ratio", [1, 2])
@pytest.mark.parametrize("nontemporal", [0, 1])
@pytest.mark.parametrize("nbytes", [16, 4096 + 48, (1 << 20) + 16 * 37])
def test_stream_probe_bytes(ratio, nontemporal, nbytes):
    import os
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "primus-turbo_amd",
                                    "bench"))
    import stream_probe

    g = torch.Generator().manual_seed(nbytes + ratio)
    src = torch.randint(0, 256, (ratio * nbytes,), generator=g, dtype=torch.uint8).cuda()
    dst = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    stream_probe.probe(src, dst, nbytes, ratio, nontemporal, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    if ratio == 1:
        want = src
    else:
        chunks = src.view(-1, 2, 16)
        want = (chunks[:, 0] ^ chunks[:, 1]).reshape(-1)
    assert torch.equal(dst[:nbytes], want)
    assert bool((dst[nbytes:] == 0xA5).all()), "bytes past the destination were written"
