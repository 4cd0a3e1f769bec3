"""Benchmark of the FP8 linear path on one MI355X (BASELINE.json metric:
"FP8 GEMM TFLOP/s (% of FP8 MFMA peak); quantize GB/s (% HBM), 1 GPU").

Workload (the north-star configuration, BASELINE.json configs[2] shape S1):
DeepSeek-V3-style blockwise FP8 -- activations 1x128 scales, weights 128x128
scales, e4m3, M=4096, K=7168, N=18432, bf16 inputs N(0,1) with 0.1% outliers x50.

A step is one forward blockwise GEMM (gemm_fp8 NT kernel) on operands already
quantized and resident in HBM; `value` is 2*M*N*K / (time per step).  The
same run also times the quantize kernels of that workload (activation dual
quantization, 128x128 weight quantization) and the full forward + backward
of gemm_fp8 (quantize + NT fwd + dgrad + wgrad), reported as extra fields.

Roofline: the dominant kernel is the GEMM (MFMA-bound); peak = 5.0 PFLOP/s
dense FP8 (MI355X).  The quantize kernels are HBM-bound, peak 8 TB/s.

cpu_baseline: the reference's torch CPU path for the same GEMM restated with
torch CPU ops (blockwise quantize, dequantize, fp32 matmul, bf16 out), repeated
for about 15 s of CPU work, median reported in TFLOP/s with torch's thread
count (os.cpu_count() reported beside it).  The timed GPU output is checked
separately against the CPU oracle's fp64 product (the `accuracy` field).

Profiling: --only gemm times the headline GEMM alone and --copy-calibration
appends three 256 MiB device copies, whose FETCH_SIZE / WRITE_SIZE readings
calibrate the HBM-traffic counters of the GEMM (rocprofv3 --pmc runs).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "primus-turbo_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP8_TFLOPS = 5000.0  # dense FP8 MFMA, MI355X
PEAK_HBM_GBS = 8000.0     # HBM3E, MI355X


def _time_cuda(fn, steps: int, warmup: int):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per call (events on the launch stream)


def _per_call_ms(fn, n: int):
    """Median and p10 / p90 of n calls, each bracketed by its own HIP events
    on the launch stream (a distribution next to the bracketed average)."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for s, e in evs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    t = sorted(s.elapsed_time(e) for s, e in evs)
    q = lambda f: t[min(n - 1, int(f * (n - 1) + 0.5))]  # noqa: E731
    return {"n": n, "p10": round(q(0.1), 4), "median": round(q(0.5), 4), "p90": round(q(0.9), 4)}


def _time_settled(fn, steps: int, settle_ms: float = 40.0):
    """_time_cuda after _settle: each extra measurement first runs its call
    until settle_ms of GPU time has passed."""
    _settle(fn, settle_ms)
    return _time_cuda(fn, steps, 0)


# the sources of the headline kernel: a traffic figure measured on other
# sources is stale and is not reported
_GEMM_SOURCES = ("primus-turbo_amd/csrc/gemm_kernel.h", "primus-turbo_amd/csrc/gemm.hip",
                 "primus-turbo_amd/csrc/gemm_inst_block.hip", "primus-turbo_amd/csrc/common.h")


def gemm_sources_sha256() -> str:
    """sha256 over the headline kernel's source files (in _GEMM_SOURCES order)."""
    import hashlib

    h = hashlib.sha256()
    for p in _GEMM_SOURCES:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def _traffic_from_profiles(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/<name>.txt)
    and where it came from.  The profile records the sha256 of the kernel
    sources it was measured on; a figure whose sources differ from the current
    ones is stale and comes back as None."""
    path = os.path.join(ROOT, "profiles", f"{name}.txt")
    src = {"profile": f"profiles/{name}.txt", "kernel_sources_sha256": None, "current": False}
    if not os.path.exists(path):
        return None, src
    value = None
    for line in open(path):
        key, _, rest = line.partition(":")
        if key == "hbm_bytes_per_launch":
            try:
                value = float(rest)
            except ValueError:
                value = None
        elif key == "kernel_sources_sha256":
            src["kernel_sources_sha256"] = rest.strip()
    src["current"] = src["kernel_sources_sha256"] == gemm_sources_sha256()
    return (value if src["current"] else None), src


def _settle(fn, settle_ms: float = 40.0) -> float:
    """Run fn until settle_ms of GPU time has passed (untimed): the clock ramps
    down while the host prepares inputs and takes tens of milliseconds of
    load to come back.  Returns the GPU milliseconds spent."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    n, spent = 0, 0.0
    while spent < settle_ms and n < 10000:
        start.record()
        for _ in range(4):
            fn()
        end.record()
        torch.cuda.synchronize()
        spent += start.elapsed_time(end)
        n += 4
    return spent


def _cpu_baseline(a_cpu, w_cpu, budget_s=15.0, max_reps=9):
    """The reference's torch CPU path for this GEMM, restated with torch CPU
    ops: blockwise quantization as the reference's torch quantize ref does it
    in fp32 (tests/pytorch/ref/quantization_ref.py; 1x128 activation and
    128x128 weight blocks, eps 1e-4, scale = fp8_max / amax, clamp, e4m3
    cast), dequantization, an fp32 matmul (tests/pytorch/ref/gemm_ref.py:13-24
    accumulates in fp32) and the bf16 output.  One warm-up, then repetitions
    until about `budget_s` seconds; the median is reported.  Threads: torch's
    intra-op pool as the box sets it (its CPU share), reported beside
    os.cpu_count()."""
    import torch

    M, K = a_cpu.shape
    N = w_cpu.shape[0]
    fmax = 448.0

    def q_act(x):
        xf = x.float().view(M, K // 128, 128)
        s = fmax / torch.clamp(xf.abs().amax(-1, keepdim=True), min=1e-4)
        return torch.clamp(xf * s, -fmax, fmax).to(torch.float8_e4m3fn), 1.0 / s

    def q_w(x):
        xf = x.float().view(N // 128, 128, K // 128, 128)
        s = fmax / torch.clamp(xf.abs().amax(dim=(1, 3), keepdim=True), min=1e-4)
        return torch.clamp(xf * s, -fmax, fmax).to(torch.float8_e4m3fn), 1.0 / s

    def step():
        qa, sa = q_act(a_cpu)
        qw, sw = q_w(w_cpu)
        da = (qa.float() * sa).view(M, K)
        dw = (qw.float() * sw).view(N, K)
        return (da @ dw.t()).to(torch.bfloat16)

    step()
    times = []
    while len(times) < max_reps and (sum(times) < budget_s or len(times) < 3):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    threads = torch.get_num_threads()
    print(f"cpu_baseline: os.cpu_count()={os.cpu_count()} torch.get_num_threads()={threads}", file=sys.stderr)
    return {
        "value": 2.0 * M * N * K / med / 1e12,
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "os_cpu_count": os.cpu_count(),
        "torch_threads": int(threads),
        "sample": f"whole {M}x{N}x{K} blockwise step on the CPU (torch fp32: quantize A 1x128 and W 128x128, "
                  f"dequantize, matmul, bf16), median of {len(times)} after 1 warm-up",
    }


def _accuracy(seed_inputs, gpu_out):
    """Checker of the timed output: the CPU oracle's fp64 product of the same
    dequantized FP8 operands over the whole output (the stated tolerance:
    SNR >= 40 dB, max rel <= 1e-2)."""
    from oracle import oracle as O

    a_q, a_s, w_q, w_s = seed_inputs
    ref = O.gemm_ref(O.dequant_block1d(a_q, 0, a_s, 1), O.dequant_block2d(w_q, 0, w_s), False, True)
    return {"snr_db": round(O.snr_db(ref, gpu_out), 2), "max_rel_err": float(f"{O.max_rel_err(ref, gpu_out):.3e}"),
            "tolerance": "SNR >= 40 dB and max rel <= 1e-2",
            "reference": "fp64 product of the dequantized FP8 operands (CPU oracle), whole output"}


def _stream_ceiling(args):
    """Each BASELINE quantize kernel next to the streaming probe
    (primus-turbo_amd/bench/stream_probe.hip, a library of its own) at the same
    bytes: "copy" when the kernel writes about what it reads, "read 2 write 1"
    for a cast; the faster of plain and non-temporal accesses.  Two timings of
    each, in one process, settled clock:
    - warm: the same buffers every call (inputs under the 256 MB memory-side
      cache can be served from it);
    - cold: calls rotate over enough copies of the inputs and outputs that
      at least 768 MB lie between two uses of one copy, three times the
      memory-side cache, so every call reads and writes HBM.
    The probe's rate is the ceiling the kernel is compared with."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "primus-turbo_amd", "bench"))
    import stream_probe

    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
        quant_fp8_blockwise_segment_m_row_col_impl,
        quantize_fp8_rowwise_impl,
        quantize_mxfp8_impl,
    )

    e4 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(4)
    dev = "cuda"
    it = max(12, args.steps // 2)
    cold_bytes = 768 << 20

    def rnd(shape):
        return torch.randn(shape, generator=g).bfloat16().to(dev)

    lens = _zipf_counts(65536, 32, 28, 0).to(dev)
    offs = group_offs_from_lens(lens)
    cases = [
        ("act dual 1x128 + transposed column copy (config 3 / headline)", (4096, 7168),
         lambda x: quant_fp8_blockwise_dual_impl(x, e4, 128, col_transposed=True, row_scale_kmajor=True)),
        ("weight 128x128 (headline)", (18432, 7168), lambda x: quant_fp8_blockwise_for_weight_impl(x, e4, 128)),
        ("rowwise (config 2)", (8192, 4096), lambda x: quantize_fp8_rowwise_impl(x, e4, -1)),
        ("weight 128x128, 32 experts (config 4)", (32, 2048, 7168),
         lambda x: quant_fp8_blockwise_for_weight_impl(x, e4, 128)),
        ("grouped segment row + col (config 4)", (65536, 7168),
         lambda x: quant_fp8_blockwise_segment_m_row_col_impl(x, e4, 128, lens, offs)),
        ("MX dual, k-major exponents (config 5)", (8192, 8192),
         lambda x: quantize_mxfp8_impl(x, e4, None, 32, with_trans=True, exp_kmajor=True)),
    ]
    stream = torch.cuda.current_stream().cuda_stream

    def rotating(calls):
        """Calls in turn; each result stays alive until its slot comes round
        again, so the outputs rotate over distinct buffers as well."""
        state = {"i": 0, "keep": [None] * len(calls)}

        def call():
            k = state["i"] % len(calls)
            state["keep"][k] = None
            state["keep"][k] = calls[k]()
            state["i"] += 1

        return call

    out = []
    for name, shape, fn in cases:
        x = rnd(shape)
        res = fn(x)
        res = res if isinstance(res, (tuple, list)) else (res,)
        rd = x.numel() * x.element_size()
        wr = sum(t.numel() * t.element_size() for t in res if isinstance(t, torch.Tensor) and t.device.type == "cuda")
        del res
        ncopy = max(2, -(-cold_bytes // (rd + wr)))
        # warm: one input; cold: ncopy inputs (and their outputs) in turn
        xs = [x] + [x.clone() for _ in range(ncopy - 1)]
        q_warm = _time_settled(lambda: fn(x), it)
        q_cold = _time_settled(rotating([lambda xi=xi: fn(xi) for xi in xs]), max(it, 2 * ncopy))
        del xs
        ratio = 2 if wr < 0.6 * rd else 1
        wb = (wr if ratio == 2 else (rd + wr) // 2) // 16 * 16
        srcs = [torch.empty(ratio * wb, dtype=torch.uint8, device=dev).random_(0, 255) for _ in range(ncopy)]
        dsts = [torch.empty(wb, dtype=torch.uint8, device=dev) for _ in range(ncopy)]
        best = {}
        for nt_try in (0, 1):  # the faster of plain and non-temporal accesses is the ceiling
            warm = _time_settled(lambda: stream_probe.probe(srcs[0], dsts[0], wb, ratio, nt_try, stream), it)
            cold = _time_settled(rotating([lambda s_=s_, d_=d_: stream_probe.probe(s_, d_, wb, ratio, nt_try, stream)
                                           for s_, d_ in zip(srcs, dsts)]), max(it, 2 * ncopy))
            for k, t in (("warm", warm), ("cold", cold)):
                if k not in best or t < best[k][0]:
                    best[k] = (t, nt_try)
        tb = lambda ms, nb: nb / (ms * 1e-3) / 1e12  # noqa: E731
        pb = (ratio + 1) * wb
        rec = {"kernel": name, "shape": list(shape), "read_MB": round(rd / 1e6, 1), "write_MB": round(wr / 1e6, 1),
               "probe": "read 2 write 1" if ratio == 2 else "copy", "cold_copies": ncopy}
        for k, q_ms in (("warm", q_warm), ("cold", q_cold)):
            p_ms, nt = best[k]
            q_tbs, p_tbs = tb(q_ms, rd + wr), tb(p_ms, pb)
            rec[k] = {"kernel_us": round(q_ms * 1e3, 1), "kernel_TBps": round(q_tbs, 2),
                      "probe_us": round(p_ms * 1e3, 1), "probe_TBps": round(p_tbs, 2),
                      "probe_nontemporal": bool(nt), "kernel_frac_of_probe": round(q_tbs / p_tbs, 3),
                      "kernel_frac_of_hbm": round(q_tbs / 8.0, 3)}
        out.append(rec)
        print(json.dumps({"case_done": name}), file=sys.stderr, flush=True)
        del x, srcs, dsts
        torch.cuda.empty_cache()
    print(json.dumps({"stream_ceiling": out, "hbm_peak_TBps": 8.0}))


def _best_ms(fn, n):
    """Fastest of n calls, each bracketed by its own HIP events on the launch
    stream, after a 40 ms settle."""
    import torch

    _settle(fn, 40.0)
    times = []
    for _ in range(n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return min(times)


def _mfma_probe_rates(variants, n):
    """TFLOP/s of the matrix-pipe probe (primus-turbo_amd/bench/mfma_probe.hip)
    variants: quantized N(0,1) operand bytes (finite e4m3), four workgroups
    per CU, ~4 ms per launch, fastest of n launches."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "primus-turbo_amd", "bench"))
    import mfma_probe

    g = torch.Generator().manual_seed(7)
    ops = torch.randn(mfma_probe.OPERAND_BYTES, generator=g).to(torch.float8_e4m3fn).view(torch.uint8).cuda()
    wgs, iters = 4 * torch.cuda.get_device_properties(0).multi_processor_count, 500
    pout = torch.empty(wgs * mfma_probe.THREADS, dtype=torch.float32, device=ops.device)
    stream = torch.cuda.current_stream().cuda_stream
    rates = {}
    for v in variants:
        ms = _best_ms(lambda v=v: mfma_probe.probe(v, iters, wgs, ops, pout, stream), n)
        rates[v] = mfma_probe.flops(iters, wgs) / (ms * 1e-3) / 1e12
    torch.cuda.synchronize()
    if not bool(torch.isfinite(pout).all()):
        raise RuntimeError("matrix-pipe probe produced non-finite output")
    return rates, mfma_probe.VARIANTS


def _gemm_ceiling(args):
    """Each scaled GEMM granularity at the headline shape (4096 x 18432 x
    7168, NT; the 1x128 x 1x128 case at the config-3 wgrad shape 18432 x 7168
    x 4096) next to the matrix-pipe probe (primus-turbo_amd/bench/mfma_probe.hip,
    a library of its own) variant that carries the same per-MFMA work with its
    operands in registers: no global or LDS traffic.  The probe's rate is the
    compute ceiling of that granularity's main loop; kernel / probe is what
    operand delivery, step synchronisation and the epilogue cost on top.
    Clock settled, one process, best of the timed calls."""
    import torch

    from primus_turbo.pytorch.core.low_precision import ScalingGranularity
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_impl, gemm_fp8_nt
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
        quantize_fp8_tensorwise_impl,
        quantize_mxfp8_impl,
    )
    from primus_turbo.pytorch.ops.gemm_fp8 import _mx_strides

    SG = ScalingGranularity
    dev = "cuda:0"
    fdt = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(0)
    it = max(10, args.steps // 4)

    probe, names = _mfma_probe_rates([0, 1, 2, 3], it)

    def outl(shape):
        x = torch.randn(shape, generator=g)
        idx = torch.randperm(x.numel(), generator=g)[: x.numel() // 1000]
        x.view(-1)[idx] *= 50.0
        return x.to(torch.bfloat16).to(dev)

    M, K, N = 4096, 7168, 18432
    a, w = outl((M, K)), outl((N, K))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    nbk = K // 128
    kernels = {}
    qa, sa = quantize_fp8_tensorwise_impl(a, fdt)
    qw, sw = quantize_fp8_tensorwise_impl(w, fdt)
    kernels[0] = (f"tensorwise NT {M}x{N}x{K}", 2.0 * M * N * K,
                  lambda: gemm_fp8_impl(qa, sa, False, qw, sw, True, torch.bfloat16, False, SG.TENSORWISE.value))
    a_row, a_s, _, _ = quant_fp8_blockwise_dual_impl(a, fdt, 128, col_transposed=True, row_scale_kmajor=True)
    w_q, w_s = quant_fp8_blockwise_for_weight_impl(w, fdt, 128)
    kernels[1] = (f"blockwise 1x128 x 128x128 NT {M}x{N}x{K} (headline)", 2.0 * M * N * K,
                  lambda: gemm_fp8_nt(a_row, w_q, torch.bfloat16, SG.BLOCKWISE, a_s, a_s.stride(), False, w_s,
                                      (nbk, 1), True, out=out))
    # wgrad of config 3: dW[N, K] = grad^T a over the M = 4096 tokens, both
    # operands the quantizer's transposed 1x128 column copies
    grad = outl((M, N))
    _, _, g_colT, g_cs = quant_fp8_blockwise_dual_impl(grad, fdt, 128, col_transposed=True)
    _, _, a_colT, a_cs = quant_fp8_blockwise_dual_impl(a, fdt, 128, col_transposed=True)
    dw = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    kernels[2] = (f"blockwise 1x128 x 1x128 NT {N}x{K}x{M} (config-3 wgrad)", 2.0 * M * N * K,
                  lambda: gemm_fp8_nt(g_colT, a_colT, torch.bfloat16, SG.BLOCKWISE, g_cs, (1, N), False, a_cs,
                                      (1, K), False, out=dw))
    qa5, ea5 = quantize_mxfp8_impl(a, fdt, 1, 32, exp_kmajor=True)
    qw5, ew5 = quantize_mxfp8_impl(w, fdt, 1, 32, exp_kmajor=True)
    kernels[3] = (f"MX NT {M}x{N}x{K}", 2.0 * M * N * K,
                  lambda: gemm_fp8_nt(qa5, qw5, torch.bfloat16, SG.MX_BLOCKWISE, ea5, _mx_strides(ea5), False, ew5,
                                      _mx_strides(ew5), False, out=out))
    res = []
    for v in sorted(kernels):
        name, fl, fn = kernels[v]
        k_tf = fl / (_best_ms(fn, it) * 1e-3) / 1e12
        res.append({"granularity": names[v], "probe_TFLOPs": round(probe[v], 1),
                    "probe_frac_of_peak": round(probe[v] / PEAK_FP8_TFLOPS, 3), "kernel": name,
                    "kernel_TFLOPs": round(k_tf, 1), "kernel_frac_of_peak": round(k_tf / PEAK_FP8_TFLOPS, 3),
                    "kernel_frac_of_probe": round(k_tf / probe[v], 3)})
        print(json.dumps({"case_done": name}), file=sys.stderr, flush=True)
    print(json.dumps({"gemm_ceiling": res, "peak_TFLOPs": PEAK_FP8_TFLOPS}))


def _grouped_steps(args):
    """Three config-4 grouped layer steps through turbo.ops.grouped_gemm_fp8
    (segment / weight quantize, persistent forward, dgrad, variable-K wgrad),
    for counter passes; with --copy-calibration, three 256 MiB copies after."""
    import torch

    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScalingGranularity

    g = torch.Generator().manual_seed(1)
    dev = "cuda:0"
    lens = _zipf_counts(65536, 32, 28, 0).to(dev)
    a = torch.randn((65536, 7168), generator=g).bfloat16().to(dev).requires_grad_(True)
    w = (torch.randn((32, 2048, 7168), generator=g) * 0.02).bfloat16().to(dev).requires_grad_(True)
    gout = torch.randn((65536, 2048), generator=g).bfloat16().to(dev)
    cfg = Float8QuantConfig(granularity=ScalingGranularity.BLOCKWISE, format=Format.E4M3, block_size=128)
    for _ in range(3):
        a.grad = w.grad = None
        turbo.ops.grouped_gemm_fp8(a, w, lens, trans_b=True, config=cfg).backward(gout)
    torch.cuda.synchronize()
    if args.copy_calibration:
        x = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
    print(json.dumps({"grouped_steps": 3, "group_lens": [int(v) for v in lens.cpu()]}))


def _quant_calls(a, w):
    """Three calls of each BASELINE quantize kernel on its config's shape, each
    followed by three calls of the streaming probe moving the same bytes (the
    pattern --stream-ceiling compares it with), for counter passes (no timing)."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "primus-turbo_amd", "bench"))
    import stream_probe

    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
        quant_fp8_blockwise_segment_m_row_col_impl,
        quantize_fp8_rowwise_impl,
        quantize_mxfp8_impl,
    )

    e4 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(2)
    dev = a.device
    x2 = torch.randn((8192, 4096), generator=g).bfloat16().to(dev)
    lens = _zipf_counts(65536, 32, 28, 0).to(dev)
    offs = group_offs_from_lens(lens)
    x4 = torch.randn((65536, 7168), generator=g).bfloat16().to(dev)
    x5 = torch.randn((8192, 8192), generator=g).bfloat16().to(dev)
    calls = [
        lambda: quant_fp8_blockwise_dual_impl(a, e4, 128, col_transposed=True, row_scale_kmajor=True),
        lambda: quant_fp8_blockwise_for_weight_impl(w, e4, 128),
        lambda: quantize_fp8_rowwise_impl(x2, e4, -1),
        lambda: quant_fp8_blockwise_segment_m_row_col_impl(x4, e4, 128, lens, offs),
        lambda: quantize_mxfp8_impl(x5, e4, None, 32, with_trans=True, exp_kmajor=True),
    ]
    stream = torch.cuda.current_stream().cuda_stream
    for f in calls:
        res = None
        for _ in range(3):
            res = f()
        torch.cuda.synchronize()
        outs = [t for t in (res if isinstance(res, (tuple, list)) else (res,)) if isinstance(t, torch.Tensor)]
        wr = sum(t.numel() * t.element_size() for t in outs)
        del res, outs
        rd = {0: a, 1: w, 2: x2, 3: x4, 4: x5}[calls.index(f)]
        rd = rd.numel() * rd.element_size()
        ratio = 2 if wr < 0.6 * rd else 1
        wb = (wr if ratio == 2 else (rd + wr) // 2) // 16 * 16
        src = torch.empty(ratio * wb, dtype=torch.uint8, device=dev)
        dst = torch.empty(wb, dtype=torch.uint8, device=dev)
        for _ in range(3):
            stream_probe.probe(src, dst, wb, ratio, 1, stream)  # non-temporal: the faster form at these sizes
        torch.cuda.synchronize()
        del src, dst


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20, help="untimed calls after the settle, before the timed ones")
    ap.add_argument("--settle-ms", type=float, default=60.0,
                    help="GPU milliseconds of untimed calls before the warm-up (the clock settles after input setup)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["all", "gemm", "quant", "grouped"], default="all",
                    help="gemm: time only the headline GEMM; quant: the headline GEMM, then three calls of each "
                         "BASELINE quantize kernel; grouped: three config-4 grouped layer steps (forward, dgrad, "
                         "variable-K wgrad) and nothing else (all for counter passes)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="end with three 256 MiB device copies (reference for the FETCH/WRITE counters)")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="only: each BASELINE quantize kernel next to a plain streaming kernel of the same bytes")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="only: each scaled GEMM granularity next to a register-only matrix-pipe kernel carrying "
                         "the same per-MFMA work")
    ap.add_argument("--sources-sha256", action="store_true",
                    help="only: print the sha256 of the headline kernel's sources (recorded in the traffic profile)")
    args = ap.parse_args()
    if args.sources_sha256:
        print(gemm_sources_sha256())
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the FP8 linear path is benchmarked on a "
                                   "single MI355X (multi-GPU sharding is a design note, not a run)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.stream_ceiling:
        _stream_ceiling(args)
        return
    if args.gemm_ceiling:
        _gemm_ceiling(args)
        return
    if args.only == "grouped":
        _grouped_steps(args)
        return

    import torch

    from primus_turbo.pytorch.core.low_precision import ScalingGranularity
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
    )

    M, K, N = 4096, 7168, 18432
    dev = "cuda:0"
    g = torch.Generator().manual_seed(0)

    def outl(shape, scale=1.0):
        x = torch.randn(shape, generator=g) * scale
        n = x.numel()
        idx = torch.randperm(n, generator=g)[: n // 1000]
        x.view(-1)[idx] *= 50.0
        return x.to(torch.bfloat16)

    a = outl((M, K)).to(dev)
    w = outl((N, K)).to(dev)
    grad = outl((M, N)).to(dev)
    fdt = torch.float8_e4m3fn
    SG = ScalingGranularity

    # ---- quantized operands (resident in HBM) ------------------------------
    # the activation layout gemm_fp8's forward produces (row scales K-block major)
    a_row, a_s, _, _ = quant_fp8_blockwise_dual_impl(a, fdt, 128, col_transposed=True, row_scale_kmajor=True)
    w_q, w_s = quant_fp8_blockwise_for_weight_impl(w, fdt, 128)
    nbk = K // 128
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def gemm():
        gemm_fp8_nt(a_row, w_q, torch.bfloat16, SG.BLOCKWISE, a_s, a_s.stride(), False, w_s, (nbk, 1), True, out=out)

    # settle the clock by time first (the count-based warm-up alone is too
    # short for a 0.5 ms kernel), then the W warm-up calls, then K timed ones
    settle_ms = _settle(gemm, args.settle_ms)
    ms = _time_cuda(gemm, args.steps, args.warmup)
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    per_call = _per_call_ms(gemm, 100)  # distribution, after (outside) the timed region
    ceiling = None
    if args.only == "all":
        # the compute ceiling of this granularity's main loop: the matrix-pipe
        # probe with the same MFMAs and scale FMAs, operands in registers
        # (a bench-only library: without it the line still prints, saying why)
        try:
            rates, names = _mfma_probe_rates([1], 10)
            ceiling = {"probe": names[1] + ", operands in registers (primus-turbo_amd/bench/mfma_probe.hip)",
                       "probe_TFLOPs": round(rates[1], 1),
                       "probe_frac_of_peak": round(rates[1] / PEAK_FP8_TFLOPS, 4),
                       "kernel_frac_of_probe": round(tflops / rates[1], 4)}
        except (OSError, RuntimeError) as e:
            ceiling = {"error": str(e)}

    extras = {}
    if args.only == "quant":
        _quant_calls(a, w)
    if args.only == "all":
        extras = _extras(args, a, w, grad, M, N, K, flops)
        del grad
        extras["other_configs"] = _other_configs(args)
        extras["vendor_reference"] = _vendor_reference(args, M, N, K)

    cpu, accuracy = None, None
    if not args.no_cpu_baseline:
        import numpy as np

        host = (a_row.cpu().view(torch.uint8).numpy(), a_s.cpu().numpy(),
                w_q.cpu().view(torch.uint8).numpy(), w_s.cpu().numpy())
        accuracy = _accuracy(host, out.float().cpu().numpy())
        accuracy["quantize_bitexact"] = _quant_parity(a.cpu(), w.cpu(), host[0], np.ascontiguousarray(host[1]),
                                                      host[2], host[3])
        cpu = _cpu_baseline(a.cpu(), w.cpu())

    if args.copy_calibration:
        x = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()

    traffic, traffic_src = _traffic_from_profiles("gemm_blockwise_nt_4096x18432x7168_traffic")
    line = {
        "metric": "FP8 GEMM TFLOP/s (% of FP8 MFMA peak); quantize GB/s (% HBM), 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "settle_ms": round(settle_ms, 1),
        "per_call_ms": per_call,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded N(0,1) bf16 with 0.1% outliers x50)",
        "config": {
            "workload": "blockwise FP8 gemm_fp8 forward NT (1x128 act / 128x128 weight scales, e4m3)",
            "M": M, "N": N, "K": K, "baseline_config_index": 2,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_FP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_FP8_TFLOPS, 4),
            "traffic": traffic,
        },
        "traffic_source": traffic_src,
        "compute_ceiling": ceiling,
        "cpu_baseline": cpu,
        "accuracy": accuracy,
    }
    line.update(extras)
    print(json.dumps(line))


def _quant_parity(a_cpu, w_cpu, a_q, a_s, w_q, w_s):
    """Checker run with the CPU baseline: the timed quantizers' FP8 bytes and
    scales against the CPU oracle's, element for element (the bar is bit-exact)."""
    import numpy as np

    from oracle import oracle as O

    qr, sr, _, _ = O.quant_block_dual(a_cpu, 0)
    qw, sw = O.quant_block_weight(w_cpu, 0)
    return {
        "activation_1x128": bool(np.array_equal(qr, a_q) and np.array_equal(sr.view(np.uint32), a_s.view(np.uint32))),
        "weight_128x128": bool(np.array_equal(qw, w_q) and np.array_equal(sw.view(np.uint32), w_s.view(np.uint32))),
        "reference": "CPU oracle (oracle/fp8_oracle.c), bytes and fp32 scale bits",
    }


def _vendor_reference(args, M, N, K):
    """The vendor library on the headline shape, for context (not `value`):
    torch._scaled_mm (hipBLASLt) with e4m3 operands and tensorwise scales,
    bf16 out. hipBLASLt has no 1x128 / 128x128 blockwise mode, so this is the
    closest library kernel to the measured blockwise one; it skips the
    per-K-block scale work the blockwise kernel does."""
    import torch

    e4 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(3)
    try:
        a = torch.randn((M, K), generator=g).to("cuda").to(e4)
        b = torch.randn((N, K), generator=g).to("cuda").to(e4).t()  # K x N, column-major
        one = torch.tensor(1.0, device="cuda")
        fn = lambda: torch._scaled_mm(a, b, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)  # noqa: E731
        ms = _time_settled(fn, max(20, args.steps // 2))
    except Exception as exc:  # a torch build without the fp8 hipBLASLt path
        return {"hipblaslt_tensorwise": None, "error": f"{type(exc).__name__}: {exc}"[:200]}
    rec = _gemm_rec(ms, 2.0 * M * N * K)
    rec["what"] = "torch._scaled_mm e4m3 tensorwise (hipBLASLt), same shape, bf16 out"
    return {"hipblaslt_tensorwise": rec}


def _gemm_rec(ms, flops):
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / PEAK_FP8_TFLOPS, 4)}


def _quant_rec(ms, nbytes):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "algorithmic_bytes": int(nbytes)}


def _zipf_counts(total, experts, nonempty, seed):
    """BASELINE config 4 split: rank weights r^-1.1 over `nonempty` experts, the
    rest empty, experts permuted with a seeded generator."""
    import torch

    g = torch.Generator().manual_seed(seed)
    w = torch.tensor([r ** -1.1 for r in range(1, nonempty + 1)], dtype=torch.float64)
    cnt = torch.floor(total * w / w.sum()).to(torch.int64)
    cnt[0] += total - int(cnt.sum())
    full = torch.zeros(experts, dtype=torch.int64)
    full[:nonempty] = cnt
    return full[torch.randperm(experts, generator=g)]


def _other_configs(args):
    """The remaining BASELINE.json configurations, each timed on the GPU
    (GEMM TFLOP/s against the dense FP8 peak, quantize GB/s against HBM)."""
    import torch

    from primus_turbo.pytorch.core.low_precision import ScalingGranularity
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_impl, gemm_fp8_nt
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_fp8_impl import grouped_gemm_fp8_impl
    from primus_turbo.pytorch.kernels.grouped_gemm.grouped_gemm_utils import group_offs_from_lens
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
        quant_fp8_blockwise_segment_m_row_col_impl,
        quantize_fp8_rowwise_impl,
        quantize_fp8_tensorwise_impl,
        quantize_mxfp8_impl,
    )
    from primus_turbo.pytorch.ops.gemm_fp8 import _mx_strides

    SG = ScalingGranularity
    dev = "cuda:0"
    e4 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(1)
    it = max(20, args.steps // 2)
    res = {}

    # config 1: tensorwise 512x1024 @ 1024x1024 (NN), launch-bound
    a1 = torch.randn((512, 1024), generator=g).bfloat16().to(dev)
    b1 = torch.randn((1024, 1024), generator=g).bfloat16().to(dev)
    qa1, sa1 = quantize_fp8_tensorwise_impl(a1, e4)
    qb1, sb1 = quantize_fp8_tensorwise_impl(b1, e4)
    res["cfg1_tensorwise_512x1024x1024_NN"] = {
        "quant_A": _quant_rec(_time_settled(lambda: quantize_fp8_tensorwise_impl(a1, e4), it), 3 * a1.numel() + 4),
        "gemm": _gemm_rec(_time_settled(lambda: gemm_fp8_impl(qa1, sa1, False, qb1, sb1, False, torch.bfloat16, False,
                                                           SG.TENSORWISE.value), it), 2.0 * 512 * 1024 * 1024),
    }
    del a1, b1, qa1, qb1

    # config 2: rowwise, Llama-3-8B up-proj 8192 x 4096 @ [14336 x 4096]^T
    a2 = torch.randn((8192, 4096), generator=g).bfloat16().to(dev)
    w2 = (torch.randn((14336, 4096), generator=g) * 0.02).bfloat16().to(dev)
    qa2, sa2 = quantize_fp8_rowwise_impl(a2, e4, -1)
    qw2, sw2 = quantize_fp8_rowwise_impl(w2, e4, -1)
    res["cfg2_rowwise_8192x14336x4096_NT"] = {
        "quant_A": _quant_rec(_time_settled(lambda: quantize_fp8_rowwise_impl(a2, e4, -1), it),
                              3 * a2.numel() + 4 * 8192),
        "gemm": _gemm_rec(_time_settled(lambda: gemm_fp8_impl(qa2, sa2, False, qw2, sw2, True, torch.bfloat16, False,
                                                           SG.ROWWISE.value), it), 2.0 * 8192 * 14336 * 4096),
    }
    del a2, w2, qa2, qw2

    # config 3, shape 2: blockwise 4096 x 2048 @ [7168 x 2048]^T
    a3 = torch.randn((4096, 2048), generator=g).bfloat16().to(dev)
    w3 = torch.randn((7168, 2048), generator=g).bfloat16().to(dev)
    ar3, as3, _, _ = quant_fp8_blockwise_dual_impl(a3, e4, 128, col_transposed=True, row_scale_kmajor=True)
    wq3, ws3 = quant_fp8_blockwise_for_weight_impl(w3, e4, 128)
    o3 = torch.empty((4096, 7168), dtype=torch.bfloat16, device=dev)
    res["cfg3_blockwise_4096x7168x2048_NT"] = {
        "gemm": _gemm_rec(_time_settled(lambda: gemm_fp8_nt(ar3, wq3, torch.bfloat16, SG.BLOCKWISE, as3, as3.stride(), False,
                                                         ws3, (16, 1), True, out=o3), it), 2.0 * 4096 * 7168 * 2048),
    }
    del a3, w3, ar3, wq3, o3

    # config 4: grouped MoE, 32 experts, 65536 routed rows, hidden 7168, FFN 2048
    lens = _zipf_counts(65536, 32, 28, 0).to(dev)
    offs = group_offs_from_lens(lens)
    a4 = torch.randn((65536, 7168), generator=g).bfloat16().to(dev)
    w4 = (torch.randn((32, 2048, 7168), generator=g) * 0.02).bfloat16().to(dev)
    seg = lambda: quant_fp8_blockwise_segment_m_row_col_impl(a4, e4, 128, lens, offs)  # noqa: E731
    ar4, _, asr4, _, _, _ = seg()
    wq4, ws4 = quant_fp8_blockwise_for_weight_impl(w4, e4, 128)
    seg_ms = _time_settled(seg, it)
    n4 = a4.numel()
    res["cfg4_grouped_blockwise_moe_32x2048x7168"] = {
        "group_lens": [int(v) for v in lens.cpu()],
        "segment_quant_A": _quant_rec(seg_ms, n4 * (2 + 1 + 1) + 4 * (n4 // 128) * 2),
        "weight_quant": _quant_rec(_time_settled(lambda: quant_fp8_blockwise_for_weight_impl(w4, e4, 128), it),
                                   3 * w4.numel() + 4 * w4.numel() // 16384),
        "grouped_gemm_fwd": _gemm_rec(_time_settled(lambda: grouped_gemm_fp8_impl(ar4, wq4, asr4, ws4, lens, offs, False,
                                                                              True, torch.bfloat16,
                                                                              SG.BLOCKWISE.value), it),
                                      2.0 * 65536 * 2048 * 7168),
    }
    del ar4, wq4
    # the whole grouped layer step through the public op: quantize + fwd + dgrad + variable-K wgrad
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format

    cfg4 = Float8QuantConfig(granularity=SG.BLOCKWISE, format=Format.E4M3, block_size=128)
    a4g = a4.detach().requires_grad_(True)
    w4g = w4.detach().requires_grad_(True)
    gout4 = torch.randn((65536, 2048), generator=g).bfloat16().to(dev)

    def step4():
        a4g.grad = w4g.grad = None  # fresh gradients: no accumulation adds in the step
        o = turbo.ops.grouped_gemm_fp8(a4g, w4g, lens, trans_b=True, config=cfg4)
        o.backward(gout4)

    res["cfg4_grouped_blockwise_moe_32x2048x7168"]["fwd_bwd_step"] = dict(
        _gemm_rec(_time_settled(step4, max(5, it // 4)), 3 * 2.0 * 65536 * 2048 * 7168),
        includes="quantize activation / weight / grad + grouped fwd + dgrad + variable-K wgrad")
    del a4, w4, a4g, w4g, gout4

    # config 5: MX-FP8 (block 32, e8m0), Llama-3-70B up-proj 8192 x 8192 @ [28672 x 8192]^T
    sign = lambda t: torch.where(torch.rand(t, generator=g) < 0.5, -1.0, 1.0)  # noqa: E731
    a5 = (sign((8192, 8192)) * torch.exp(torch.randn((8192, 8192), generator=g) * 1.5)).bfloat16().to(dev)
    w5 = (sign((28672, 8192)) * torch.exp(torch.randn((28672, 8192), generator=g) * 1.5)).bfloat16().to(dev)
    # the layout gemm_fp8's MX forward uses: exponents K-block major
    qa5, ea5 = quantize_mxfp8_impl(a5, e4, 1, 32, exp_kmajor=True)
    qw5, ew5 = quantize_mxfp8_impl(w5, e4, 1, 32, exp_kmajor=True)
    o5 = torch.empty((8192, 28672), dtype=torch.bfloat16, device=dev)
    res["cfg5_mxfp8_8192x28672x8192_NT"] = {
        "quant_dual_A": _quant_rec(_time_settled(lambda: quantize_mxfp8_impl(a5, e4, None, 32, with_trans=True,
                                                                          exp_kmajor=True), it),
                                   a5.numel() * (2 + 1 + 1) + 2 * a5.numel() // 32),
        "gemm": _gemm_rec(_time_settled(lambda: gemm_fp8_nt(qa5, qw5, torch.bfloat16, SG.MX_BLOCKWISE, ea5,
                                                         _mx_strides(ea5), False, ew5, _mx_strides(ew5), False,
                                                         out=o5), it), 2.0 * 8192 * 28672 * 8192),
    }
    del qa5, qw5, o5
    # second shape: down-proj x[8192, 28672] @ W[8192, 28672]^T (K = 28672)
    x5 = (sign((8192, 28672)) * torch.exp(torch.randn((8192, 28672), generator=g) * 1.5)).bfloat16().to(dev)
    wd5 = (sign((8192, 28672)) * torch.exp(torch.randn((8192, 28672), generator=g) * 1.5)).bfloat16().to(dev)
    qx5, ex5 = quantize_mxfp8_impl(x5, e4, 1, 32, exp_kmajor=True)
    qd5, ed5 = quantize_mxfp8_impl(wd5, e4, 1, 32, exp_kmajor=True)
    od5 = torch.empty((8192, 8192), dtype=torch.bfloat16, device=dev)
    res["cfg5_mxfp8_8192x28672x8192_NT"]["gemm_down_8192x8192x28672"] = _gemm_rec(
        _time_settled(lambda: gemm_fp8_nt(qx5, qd5, torch.bfloat16, SG.MX_BLOCKWISE, ex5, _mx_strides(ex5), False,
                                          ed5, _mx_strides(ed5), False, out=od5), it), 2.0 * 8192 * 8192 * 28672)
    del x5, wd5, qx5, qd5, od5
    # the up-proj layer step through the public op, HYBRID format (e4m3 forward, e5m2 gradient)
    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScaleDtype

    cfg5 = Float8QuantConfig(granularity=SG.MX_BLOCKWISE, format=Format.HYBRID, block_size=32,
                             scale_dtype=ScaleDtype.E8M0)
    a5g = a5.detach().requires_grad_(True)
    w5g = w5.detach().requires_grad_(True)
    gout5 = torch.randn((8192, 28672), generator=g).bfloat16().to(dev)

    def step5():
        a5g.grad = w5g.grad = None
        o = turbo.ops.gemm_fp8(a5g, w5g, False, True, torch.bfloat16, cfg5)
        o.backward(gout5)

    res["cfg5_mxfp8_8192x28672x8192_NT"]["fwd_bwd_step_hybrid"] = dict(
        _gemm_rec(_time_settled(step5, max(5, it // 4)), 3 * 2.0 * 8192 * 28672 * 8192),
        includes="MX dual quantize of activation / weight / grad + fwd + dgrad + wgrad")
    del a5, w5, a5g, w5g, gout5

    # MoE token permutation producing config 4's operand shape: 8192 dispatched
    # tokens, each routed to 8 of the 32 local experts, hidden 7168 -> 65536
    # expert-major rows (and the inverse reduction)
    from primus_turbo.pytorch.kernels.moe.moe_permute_impl import (
        permute_impl,
        permute_preprocessing_impl,
        unpermute_impl,
    )

    T6, E6, k6, H6 = 8192, 32, 8, 7168
    idx6 = torch.sort(torch.argsort(torch.rand((T6, E6), generator=g), dim=1)[:, :k6], dim=1).values.to(dev)
    pre = lambda: permute_preprocessing_impl(idx6, E6, k6, 0, -1, 0)  # noqa: E731
    rim6, tpe6, _, nd6 = pre()
    P6 = int(tpe6.sum().item())
    tok6 = torch.randn((T6, H6), generator=g).bfloat16().to(dev)
    out6 = torch.empty((P6, H6), dtype=torch.bfloat16, device=dev)
    back6 = torch.empty((T6, H6), dtype=torch.bfloat16, device=dev)
    nb6 = (T6 + P6) * H6 * 2
    res["moe_permute_8192x7168_top8_of_32"] = {
        "preprocess": {"ms": round(_time_settled(pre, it), 4)},
        "permute": _quant_rec(_time_settled(lambda: permute_impl(tok6, out6, None, None, None, None, rim6, nd6, 0, E6, H6,
                                                              0, False, False, P6, 0), it), nb6),
        "unpermute": _quant_rec(_time_settled(lambda: unpermute_impl(out6, back6, None, None, rim6, nd6, E6, H6, False,
                                                                     0), it), nb6),
    }
    return res


def _extras(args, a, w, grad, M, N, K, flops):
    """Quantize kernels, backward GEMM layouts and the full fwd+bwd step."""
    import torch

    import primus_turbo.pytorch as turbo
    from primus_turbo.pytorch.core.low_precision import Float8QuantConfig, Format, ScalingGranularity
    from primus_turbo.pytorch.kernels.gemm.gemm_fp8_impl import gemm_fp8_nt
    from primus_turbo.pytorch.kernels.quantization.quantization_impl import (
        quant_fp8_blockwise_dual_impl,
        quant_fp8_blockwise_for_weight_impl,
    )

    dev = a.device
    fdt = torch.float8_e4m3fn
    SG = ScalingGranularity
    nbk = K // 128

    # ---- quantize kernels ----------------------------------------------------
    def q_act():  # the layout of gemm_fp8's forward
        quant_fp8_blockwise_dual_impl(a, fdt, 128, col_transposed=True, row_scale_kmajor=True)

    def q_w():
        quant_fp8_blockwise_for_weight_impl(w, fdt, 128)

    qa_ms = _time_settled(q_act, max(args.steps, 20))
    qw_ms = _time_settled(q_w, max(args.steps, 20))
    qa_bytes = M * K * (2 + 1 + 1) + 4 * (M * (K // 128) + (M // 128) * K)
    qw_bytes = N * K * (2 + 1) + 4 * (N // 128) * (K // 128)
    qa_gbs = qa_bytes / (qa_ms * 1e-3) / 1e9
    qw_gbs = qw_bytes / (qw_ms * 1e-3) / 1e9

    # ---- full forward + backward of gemm_fp8 -------------------------------
    cfg = Float8QuantConfig(granularity=SG.BLOCKWISE, format=Format.E4M3, block_size=128)
    a_p = a.detach().requires_grad_()
    w_p = w.detach().requires_grad_()

    def train_step():
        a_p.grad = None
        w_p.grad = None
        o = turbo.ops.gemm_fp8(a_p, w_p, trans_b=True, config=cfg)
        o.backward(grad)

    step_ms = _time_settled(train_step, max(5, args.steps // 5))

    # ---- layouts of the backward GEMMs, timed alone -------------------------
    g_row, g_s, g_colT, g_cs = quant_fp8_blockwise_dual_impl(grad, fdt, 128, col_transposed=True,
                                                              row_scale_kmajor=True)
    _, _, a_colT, a_cs = quant_fp8_blockwise_dual_impl(a, fdt, 128, col_transposed=True)
    _, w_s, w_t = quant_fp8_blockwise_for_weight_impl(w, fdt, 128, with_transpose=True)
    da = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    dw = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    nbn = N // 128

    def dgrad():
        gemm_fp8_nt(g_row, w_t, torch.bfloat16, SG.BLOCKWISE, g_s, g_s.stride(), False, w_s, (1, nbk), True, out=da)

    def wgrad():
        gemm_fp8_nt(g_colT, a_colT, torch.bfloat16, SG.BLOCKWISE, g_cs, (1, N), False, a_cs, (1, K), False, out=dw)

    dg_ms = _time_settled(dgrad, max(10, args.steps // 2))
    wg_ms = _time_settled(wgrad, max(10, args.steps // 2))

    return {
        "quantize": {
            "act_dual_1x128": {"ms": round(qa_ms, 4), "GB/s": round(qa_gbs, 1), "frac_hbm": round(qa_gbs / PEAK_HBM_GBS, 4),
                               "algorithmic_bytes": qa_bytes},
            "weight_128x128": {"ms": round(qw_ms, 4), "GB/s": round(qw_gbs, 1), "frac_hbm": round(qw_gbs / PEAK_HBM_GBS, 4),
                               "algorithmic_bytes": qw_bytes},
        },
        "backward_gemms": {
            "dgrad_NT_on_transposed_weight": {"ms": round(dg_ms, 4), "TFLOP/s": round(flops / dg_ms / 1e9, 1)},
            "wgrad_NT_on_transposed_columns": {"ms": round(wg_ms, 4), "TFLOP/s": round(flops / wg_ms / 1e9, 1)},
        },
        "fwd_bwd_step": {"ms": round(step_ms, 4), "TFLOP/s": round(3 * flops / step_ms / 1e9, 1),
                         "includes": "quantize a/w/grad + fwd + dgrad + wgrad"},
    }


if __name__ == "__main__":
    main()
