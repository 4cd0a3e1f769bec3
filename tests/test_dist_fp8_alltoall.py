"""FP8AllToAll (primus_turbo/pytorch/dist/fp8_alltoall.py:25-194).

* Host behaviour (no GPU): the reference's asserts and format rule, and the
  one-rank bypass in both directions.
* The exchange logic over two real ranks (gloo, CPU, spawned processes): equal
  and unequal splits, a rank that receives nothing, fwd_quant off, the
  reverse exchange in backward with HYBRID's E5M2.  The tensorwise quantize /
  dequantize of the payload are swapped for the CPU oracle there (the
  product's kernels need a GPU), so these cases check the module's own steps:
  split bookkeeping, the MIN reduction of scale_inv, the byte payload.
* On the GPU, the product's quantize -> uint8 payload -> dequantize with this
  build's kernels, with the collectives replaced by a loopback (one GPU has
  no peer): bit-exact against the oracle, forward and backward.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from oracle import oracle as O

FMT = {torch.float8_e4m3fn: 0, torch.float8_e5m2: 1}


def _mods():
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScalingGranularity
    from primus_turbo.pytorch.dist import fp8_alltoall as mod

    return turbo, Float8QuantConfig, Format, ScalingGranularity, mod


def _oracle_quant(x, dtype, granularity):
    """Tensorwise quantize on the CPU oracle, in quantize_fp8's return form."""
    q, s = O.quant_tensorwise(x, FMT[dtype])
    return torch.from_numpy(q).view(dtype), torch.tensor(float(s), dtype=torch.float32)


def _oracle_dequant(x, out_dtype, granularity, *, scale_inv, **_):
    """out_dtype(float(q) * scale_inv), the fp32 product rounded once."""
    v = torch.from_numpy(O.fp8_to_float(x.view(torch.uint8).numpy(), FMT[x.dtype]))
    return (v * scale_inv.to(torch.float32)).to(out_dtype)


def _expected(xs, dtype, orig_dtype, in_splits_all, rank):
    """Rows rank `rank` receives: from each sender s, its chunk for `rank`,
    dequantized with the group's minimum scale_inv (the reference's order)."""
    qs = [_oracle_quant(x, dtype, None) for x in xs]
    smin = min(float(s) for _, s in qs)
    parts = []
    for s, (q, _) in enumerate(qs):
        splits = in_splits_all[s]
        start = sum(splits[:rank])
        chunk = q[start:start + splits[rank]]
        parts.append(_oracle_dequant(chunk, orig_dtype, None, scale_inv=torch.tensor(smin)))
    return torch.cat(parts)


def test_asserts_and_formats():
    _, Cfg, Format, SG, mod = _mods()
    x = torch.zeros(8, 4, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        mod.FP8AllToAll.apply(None, x, None, None, True, True, Cfg())
    with pytest.raises(AssertionError):
        mod.FP8AllToAll.apply(object(), x, None, None, True, True, Cfg(granularity=SG.ROWWISE))
    with pytest.raises(ValueError, match="E4M3 and HYBRID"):
        mod.FP8AllToAll.apply(object(), x, None, None, True, True, Cfg(format=Format.E5M2))
    assert mod._fp8_dtype(Format.E4M3, False) == torch.float8_e4m3fn
    assert mod._fp8_dtype(Format.HYBRID, True) == torch.float8_e4m3fn
    assert mod._fp8_dtype(Format.HYBRID, False) == torch.float8_e5m2


def _run(rank, world, path, case):
    os.environ.setdefault("GLOO_SOCKET_IFNAME", "lo")
    store = dist.FileStore(path, world)
    dist.init_process_group("gloo", store=store, rank=rank, world_size=world)
    try:
        case(rank, world)
    finally:
        dist.destroy_process_group()


def _spawn(world, case, tmp_path):
    mp.spawn(_run, args=(world, str(tmp_path / "store"), case), nprocs=world, join=True)


def _inputs(world, rows_per_rank, h, dtype):
    # every rank can rebuild every rank's input; rank r's amax grows with r
    xs = []
    for r in range(world):
        g = torch.Generator().manual_seed(100 + r)
        xs.append((torch.randn(rows_per_rank[r], h, generator=g) * (1.0 + 3 * r)).to(dtype))
    return xs


def _case_bypass(rank, world):
    _, Cfg, _, _, mod = _mods()
    x = torch.randn(6, 5, dtype=torch.bfloat16, requires_grad=True)
    y = mod.FP8AllToAll.apply(dist.group.WORLD, x, None, None, True, True, Cfg())
    assert torch.equal(y, x)
    g = torch.randn(6, 5, dtype=torch.bfloat16)
    y.backward(g)
    assert torch.equal(x.grad, g)


def test_one_rank_bypass(tmp_path):
    _spawn(1, _case_bypass, tmp_path)


def _case_equal(rank, world):
    _, Cfg, Format, _, mod = _mods()
    mod.quantize_fp8, mod.dequantize_fp8 = _oracle_quant, _oracle_dequant
    for orig in (torch.bfloat16, torch.float16, torch.float32):
        xs = _inputs(world, [4 * world] * world, 24, orig)
        x = xs[rank].clone().requires_grad_()
        y = mod.FP8AllToAll.apply(dist.group.WORLD, x, None, None, True, True, Cfg(format=Format.HYBRID))
        splits = [[4] * world] * world
        exp = _expected(xs, torch.float8_e4m3fn, orig, splits, rank)
        assert y.dtype == orig and torch.equal(y, exp), f"forward {orig}"
        # backward: the reverse exchange, E5M2 under HYBRID
        gs = [(torch.randn(4 * world, 24, generator=torch.Generator().manual_seed(7 + r))).to(orig)
              for r in range(world)]
        y.backward(gs[rank])
        assert torch.equal(x.grad, _expected(gs, torch.float8_e5m2, orig, splits, rank)), f"backward {orig}"


def _case_unequal(rank, world):
    _, Cfg, _, _, mod = _mods()
    mod.quantize_fp8, mod.dequantize_fp8 = _oracle_quant, _oracle_dequant
    # in_splits[s][r]: rows sender s sends to r; rank 1 receives nothing
    in_splits = [[3, 0], [5, 0]]
    out_splits = [[in_splits[s][r] for s in range(world)] for r in range(world)]
    xs = _inputs(world, [sum(s) for s in in_splits], 16, torch.bfloat16)
    x = xs[rank].clone().requires_grad_()
    y = mod.FP8AllToAll.apply(dist.group.WORLD, x, out_splits[rank], in_splits[rank], True, True, Cfg())
    exp = _expected(xs, torch.float8_e4m3fn, torch.bfloat16, in_splits, rank)
    assert y.shape == exp.shape and torch.equal(y, exp)
    # backward sends each received row back to its sender
    gs = [torch.randn(sum(out_splits[r]), 16, generator=torch.Generator().manual_seed(30 + r)).bfloat16()
          for r in range(world)]
    y.backward(gs[rank])
    exp_g = _expected(gs, torch.float8_e4m3fn, torch.bfloat16, out_splits, rank)
    assert x.grad.shape == x.shape and torch.equal(x.grad, exp_g)


def _case_no_quant(rank, world):
    _, Cfg, _, _, mod = _mods()
    xs = _inputs(world, [2 * world] * world, 8, torch.bfloat16)
    y = mod.FP8AllToAll.apply(dist.group.WORLD, xs[rank], None, None, False, False, Cfg())
    exp = torch.cat([xs[s][2 * rank:2 * rank + 2] for s in range(world)])
    assert torch.equal(y, exp)


@pytest.mark.parametrize("case", [_case_equal, _case_unequal, _case_no_quant])
def test_two_ranks(tmp_path, case):
    _spawn(2, case, tmp_path)


@pytest.mark.gpu
@pytest.mark.parametrize("orig", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("fmt", ["E4M3", "HYBRID"])
def test_payload_kernels_loopback(monkeypatch, orig, fmt):
    """The product's payload path on the GPU: tensorwise quantize, uint8
    bytes, dequantize with the reduced scale_inv (the only rank's own), the
    exchange replaced by a copy.  Forward and backward bit-exact against the
    oracle."""
    _, Cfg, Format, _, mod = _mods()
    monkeypatch.setattr(dist, "get_world_size", lambda group=None: 2)
    monkeypatch.setattr(dist, "all_reduce", lambda t, op=None, group=None: None)

    def loopback(output, input, output_split_sizes=None, input_split_sizes=None, group=None):
        assert output.dtype == torch.uint8 and input.dtype == torch.uint8, "payload travels as bytes"
        output.copy_(input)

    monkeypatch.setattr(dist, "all_to_all_single", loopback)
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(1, 1024, 7168 // 8, generator=g) * 3).to(orig)
    xd = x.cuda().requires_grad_()
    y = mod.FP8AllToAll.apply(object(), xd, None, None, True, True, Cfg(format=getattr(Format, fmt)))
    torch.cuda.synchronize()
    exp = _expected([x], torch.float8_e4m3fn, orig, [[x.shape[0]]], 0)
    assert y.dtype == orig and torch.equal(y.cpu(), exp)
    dy = (torch.randn(x.shape, generator=g) * 1e-3).to(orig)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    bwd = torch.float8_e5m2 if fmt == "HYBRID" else torch.float8_e4m3fn
    assert torch.equal(xd.grad.cpu(), _expected([dy], bwd, orig, [[x.shape[0]]], 0))
