#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-contraction hot path (one JSON line).

Headline: W4A16 decode GEMV, M=1, K=N=4096, asymmetric
uint4 g=128 -> ``value`` in GB/s of algorithmic HBM bytes per second.
The ``extra`` object carries the other configurations (decode M=16, prefill
M=2048 TFLOP/s, W8A8, quantized MoE, W8A16), each measured the same way.

A step is one pass of the hot path over one batch already resident in HBM.
Steps are captured into a HIP graph and replayed; HIP events on the launch
stream time it (graph_time explains how the graph-start latency is taken
out), so the per-step time is the average kernel duration plus the gaps
between back-to-back kernels. Inputs rotate over enough copies to exceed
the 256 MB Infinity Cache, so decode weights stream from HBM, not MALL.
``cpu_baseline`` times the C oracle (a port of the reference's CPU numerics)
on this host's cores over a bounded sample of the headline workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W4A16 GEMM TFLOP/s & HBM GB/s (% of MI355X peak), decode M=1 + prefill M=2048"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2516.6  # dense MFMA, no sparsity
I8_PEAK_TOPS = 5033.2
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", choices=["decode", "all"], default="all",
                    help="'decode' times only the headline workload")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--probe", choices=["traffic", "read", "mfma", "kn", "ablation", "decode"], default=None,
                    help="'traffic': only run 40 decode launches over distinct weight copies, then four 64 MiB "
                         "device copies (run under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE; the copies calibrate "
                         "the counters). 'read': time the plain HBM read of the decode's byte count (the floor "
                         "of any kernel streaming those bytes) beside the decode GEMV itself. 'mfma': three "
                         "launches each of the compute-bound lines (prefill, W8A8, MoE), for rocprofv3 --pmc "
                         "MFMA-busy counters. 'kn': the scaled FP8 GEMM (N=14336, K=4096) with its [K, N] "
                         "operand read in place against the transposed copy plus the row-form kernel, over M. "
                         "'ablation': the W8A8 line (config 3) with the product library and with each "
                         "measurement-only library of `python -m intent_amd.build --ablations`. 'decode': 40 "
                         "launches each of the decode GEMV at M=1 and M=16 over distinct weight copies (run "
                         "under rocprofv3 --pmc for per-dispatch L1 / address-unit counters)")
    return ap.parse_args()


WARM_SECONDS = 0.2
PAIRS = 9


def graph_time(launches, steps: int, warmup: int) -> float:
    """Average ms per step of `steps` launches replayed from a HIP graph.

    Launch i uses input set i % len(launches). Two graphs are captured: the
    rotation R (every input set once, in cyclic order) and R followed by the
    `steps` timed launches. The timed launches start at set 0, whose last use
    lies a full rotation (more than the 256 MB Infinity Cache, see copies_for)
    behind them, so every one reads its operands from HBM whatever `steps` is.
    Each graph replay carries a fixed start latency (about 10 us on this
    stack, far above a decode kernel); timing both graphs with HIP events on
    their stream and subtracting cancels it, leaving exactly the `steps`
    launches and the gaps between them. The median of PAIRS back-to-back
    pairs is returned, after at least WARM_SECONDS of rotation replays.
    """
    import torch

    n = len(launches)
    for i in range(warmup):
        launches[i % n]()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    rotation = torch.cuda.CUDAGraph()
    timed = torch.cuda.CUDAGraph()
    with torch.cuda.graph(rotation, stream=stream):
        for i in range(n):
            launches[i]()
    with torch.cuda.graph(timed, stream=stream):
        for i in range(n):
            launches[i]()
        for i in range(steps):
            launches[i % n]()
    timed.replay()  # first replay of a fresh graph carries one-time set-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while True:
        rotation.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= WARM_SECONDS:
            break
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(4 * PAIRS)]
    with torch.cuda.stream(stream):
        for p in range(PAIRS):
            a, b, c, d = marks[4 * p: 4 * p + 4]
            a.record(stream)
            rotation.replay()
            b.record(stream)
            c.record(stream)
            timed.replay()
            d.record(stream)
    torch.cuda.synchronize()
    diffs = sorted(marks[4 * p + 2].elapsed_time(marks[4 * p + 3]) - marks[4 * p].elapsed_time(marks[4 * p + 1])
                   for p in range(PAIRS))
    return diffs[PAIRS // 2] / steps


def copies_for(bytes_per_set: int, minimum: int = 1) -> int:
    return max(minimum, int(np.ceil(1.25 * MALL_BYTES / max(bytes_per_set, 1))) + 1)


def bench_w4a16(M: int, K: int, N: int, steps: int, warmup: int, kernel: str = "auto", copies: int | None = None) -> dict:
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    d = inputs.to_device(inputs.config1_w4a16_decode(0, M=M, K=K, N=N))
    work = inputs.w4a16_work(M, K, N)
    art = intent.compile(intent.weight_only_int4_asym_matmul, target=intent.MI355XTarget(0),
                         constexprs={"KERNEL": kernel})
    n = copies if copies is not None else copies_for(work.bytes)
    sets = [(d["x"].clone(), d["packed"].clone(), d["scales"].clone(), d["zeros"].clone()) for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    entry, kernel = art.observation.entry, art.observation.kernel
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "entry": entry, "kernel": kernel, "copies": n,
            "rotation_bytes": n * work.bytes}


def bench_w8a16(steps: int, warmup: int) -> dict:
    import intent_amd as intent
    from intent_amd import inputs

    d = inputs.to_device(inputs.config0_w8a16(0))
    work = inputs.w8a16_work(16, 1024, 1024)
    art = intent.compile(intent.weight_only_int8_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes)
    calls = [art.prepare(d["x"].clone(), d["w"].clone(), d["scales"].clone()) for _ in range(n)]
    return {"ms": graph_time([c.launch for c in calls], steps, warmup), "work": work, "copies": n}


def bench_w8a8(steps: int, warmup: int) -> dict:
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    d = inputs.to_device(inputs.config3_w8a8(0))
    work = inputs.w8a8_work(4096, 8192, 8192)
    art = intent.compile(intent.w8a8_scaled_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [tuple(d[k].clone() for k in ("a", "a_scales", "w", "w_scales")) for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_moe(steps: int, warmup: int) -> dict:
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    h = inputs.config4_moe(0)
    d = inputs.to_device(h)
    T, H = h["x"].shape
    E, F2, _ = h["wgu"].shape
    work = inputs.moe_work(T, H, E, 2, F2 // 2)
    art = intent.compile(intent.moe_expert_ffn_w4, target=intent.MI355XTarget(0), constexprs={"TOP_K": 2})
    y = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    call = art.prepare(d["logits"], d["x"], d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], y)
    ms = graph_time([call.launch], steps, warmup)
    return {"ms": ms, "work": work, "copies": 1}


def bench_q4k(steps: int, warmup: int) -> dict:
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    d = inputs.kquant_projection(0, N=4096, K=4096)
    work = inputs.kquant_work(4096, 4096)
    art = intent.compile(intent.quantized_projection, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes)
    w = torch.from_numpy(d["w"]).cuda()
    x = torch.from_numpy(d["x"]).cuda()
    calls = [art.prepare(w.clone(), x.clone()) for _ in range(n)]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_w4a8(steps: int, warmup: int) -> dict:
    """The reference's W4A8 case (experiments/cpu/providers/mojo/contraction.py:201-206)."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    rng = np.random.default_rng(0)
    M, K, N = 4096, 4096, 14336
    a = torch.from_numpy(rng.integers(-128, 128, (M, K), dtype=np.int8)).cuda()
    p = torch.from_numpy(rng.integers(0, 256, (N, K // 2), dtype=np.uint8)).cuda()
    work = inputs.Workload(f"w4a8 M{M} K{K} N{N}", 2 * M * N * K, M * K + N * K // 2 + M * N * 4)
    art = intent.compile(intent.w4a8_packed_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    calls = [art.prepare(a.clone(), p.clone()) for _ in range(n)]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_sfp8_splitk(steps: int, warmup: int) -> dict:
    """The reference's split-K FP8 case (experiments/gpu/providers/triton/contraction.py:174-186):
    M=4096, N=14336, K=4096 as [IT=4, SP=4, 256], E4M3FN, scales 1, f16 InOut output. The
    [K, N] right operand is read in place."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M, N, IT, SP = 4096, 14336, 4, 4
    K = IT * SP * 256
    g = torch.Generator(device="cuda").manual_seed(0)
    lhs = torch.randn((M, K), device="cuda", generator=g).to(torch.float8_e4m3fn)
    rhs = torch.randn((K, N), device="cuda", generator=g).to(torch.float8_e4m3fn)
    work = inputs.Workload(f"scaled fp8 split-K M{M} K{K} N{N} SP{SP}", 2 * M * N * K,
                           M * K + K * N + 2 * M * N * 2)
    art = intent.compile(intent.scaled_fp8_splitk_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [(lhs.clone().view(M, IT, SP, 256), rhs.clone().view(IT, SP, 256, N),
             torch.zeros((M, N), device="cuda", dtype=torch.float16)) for _ in range(n)]
    calls = [art.prepare(l4, r4, o, 1.0, 1.0) for l4, r4, o in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_deepgemm(steps: int, warmup: int) -> dict:
    """The reference's deepgemm_fp8_2xacc case (experiments/cpu/providers/mojo/contraction.py:227-236):
    M = N = K = 4096, E4M3FN with f32 scales per (row, 128-k) and per 128 x 128 rhs block, bf16 out."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M = N = K = 4096
    KB = K // 128
    g = torch.Generator(device="cuda").manual_seed(0)
    lhs = torch.randn((M, K), device="cuda", generator=g).to(torch.float8_e4m3fn).view(M, KB, 128)
    rhs = torch.randn((N, K), device="cuda", generator=g).to(torch.float8_e4m3fn).view(N, KB, 128)
    ls = torch.rand((M, KB), device="cuda", generator=g) + 0.5
    rs = torch.rand((N // 128, KB), device="cuda", generator=g) + 0.5
    work = inputs.Workload(f"deepgemm fp8 M{M} K{K} N{N}", 2 * M * N * K,
                           M * K + N * K + (M + N // 128) * KB * 4 + M * N * 2)
    art = intent.compile(intent.deepgemm_fp8_2xacc, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [(lhs.clone(), rhs.clone(), ls.clone(), rs.clone()) for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_fp4(steps: int, warmup: int) -> dict:
    """The reference's dequant_bf16_fp4 case (experiments/cpu/providers/mojo/contraction.py:220-224):
    bf16 activations [4096, 4096] * 0.125, packed E2M1 weights [4096, 2048], bf16 out."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M = N = K = 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    x = (torch.randn((M, K), device="cuda", generator=g) * 0.125).bfloat16()
    w = torch.randint(0, 256, (N, K // 2), device="cuda", generator=g, dtype=torch.uint8)
    work = inputs.Workload(f"fp4 x bf16 M{M} K{K} N{N}", 2 * M * N * K, M * K * 2 + N * K // 2 + M * N * 2)
    art = intent.compile(intent.dequant_bf16_fp4_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [(x.clone(), w.clone()) for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_moe_f16(steps: int, warmup: int) -> dict:
    """The reference's f16 moe_expert_ffn at its own size (moe.py:6-10: T = D = 4096, F = 14336,
    E = 8, top-2, routes by support.py:113-130): two grouped [K, N] projections + combine."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    T, D, F, E, K = 4096, 4096, 14336, 8, 2
    d = {k: torch.from_numpy(v).cuda() for k, v in inputs.moe_routes(T, K, E, "reference").items()}
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(T, D, device="cuda", generator=g).half()
    w1 = (torch.randn(E, D, F, device="cuda", generator=g) / 64).half()
    w2 = (torch.randn(E, F, D, device="cuda", generator=g) / 128).half()
    y = torch.zeros(T, D, device="cuda")
    R = T * K
    work = inputs.Workload(f"moe_expert_ffn f16 T{T} D{D} F{F} E{E} top{K}", 2 * 2 * R * D * F,
                           2 * E * D * F * 2 + T * D * 2 + T * D * 8)
    art = intent.compile(intent.moe_expert_ffn, target=intent.MI355XTarget(0))
    call = art.prepare(x, d["route_offsets"], d["member_routes"], d["route_token"], d["route_weights"], w1, w2, y)
    ms = graph_time([call.launch], steps, warmup)
    return {"ms": ms, "work": work}


def bench_quantized_gemm(steps: int, warmup: int) -> dict:
    """The reference's quantized_gemm case (experiments/cpu/providers/mojo/contraction.py:177-186):
    f16 [4096, 4096] x [4096, 14336] with bias, ReLU, residual, per-column scale, int8 out;
    b reaches the kernel as [K, N] (no transposed copy)."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M, K, N = 4096, 4096, 14336
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn((M, K), device="cuda", generator=g).half() / 64.0
    b = torch.randn((K, N), device="cuda", generator=g).half()
    bias = torch.randn((N,), device="cuda", generator=g) * 0.25
    residual = (torch.randn((M, N), device="cuda", generator=g) * 0.25).half()
    scale = torch.linspace(1.0 / 48.0, 1.0 / 24.0, N, device="cuda")
    work = inputs.Workload(f"quantized_gemm M{M} K{K} N{N}", 2 * M * N * K,
                           M * K * 2 + K * N * 2 + N * 8 + M * N * 2 + M * N)
    art = intent.compile(intent.quantized_gemm, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [(a.clone(), b.clone(), bias, residual.clone(), scale) for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_mxfp8(steps: int, warmup: int) -> dict:
    """The reference's mxfp8_gemm case (experiments/cpu/providers/mojo/contraction.py:285-305):
    M=4096, K=4096, N=14336, E4M3FN with E8M0 scales per 32, rhs given as the [KB, 32, N]
    view of [N, K] rows."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M, K, N = 4096, 4096, 14336
    rng = np.random.default_rng(0)

    def operand(rows):
        v = rng.integers(0, 256, (rows, K), dtype=np.uint8)
        v[(v & 0x7F) == 0x7F] = 0x38
        return torch.from_numpy(v).cuda().view(torch.float8_e4m3fn)

    a, b = operand(M), operand(N)
    sa = torch.from_numpy(rng.integers(120, 134, (M, K // 32), dtype=np.uint8)).cuda()
    sb = torch.from_numpy(rng.integers(120, 134, (N, K // 32), dtype=np.uint8)).cuda()
    work = inputs.Workload(f"mxfp8 M{M} K{K} N{N}", 2 * M * N * K, M * K + N * K + (M + N) * K // 32 + M * N * 4)
    art = intent.compile(intent.block_scaled_matmul, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    sets = [(a.clone().view(M, K // 32, 32), sa.clone(), b.clone().T.view(K // 32, 32, N), sb.clone().T)
            for _ in range(n)]
    calls = [art.prepare(*s) for s in sets]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls, sets
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def bench_i8_quant(steps: int, warmup: int) -> dict:
    """Per-token int8 quantizer feeding config 3: f16 [4096, 8192] -> int8 + f32 scales."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    M, K = 4096, 8192
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn((M, K), device="cuda", generator=g).half()
    work = inputs.Workload(f"per-token int8 quantize M{M} K{K} f16", 0, M * K * 2 + M * K + M * 4)
    art = intent.compile(intent.per_token_int8_quantize, target=intent.MI355XTarget(0))
    n = copies_for(work.bytes, minimum=2)
    calls = [art.prepare(x.clone()) for _ in range(n)]
    ms = graph_time([c.launch for c in calls], steps, warmup)
    del calls
    torch.cuda.empty_cache()
    return {"ms": ms, "work": work, "copies": n}


def measured_traffic(kernel: str) -> int | None:
    """HBM bytes per decode launch from the committed FETCH_SIZE/WRITE_SIZE profile, if that
    profile covers `kernel` (the variant this run dispatched to); otherwise None."""
    path = ROOT / "profiles" / "w4a16_gemv_decode_m1_traffic.md"
    if not path.exists():
        return None
    text = path.read_text().splitlines()
    covered = next((ln.split(":", 1)[1].strip() for ln in text if ln.startswith("kernel:")), None)
    if covered is None or covered.replace(" ", "") != kernel.replace(" ", ""):
        return None
    for line in text:
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def traffic_probe() -> None:
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    d = inputs.to_device(inputs.config1_w4a16_decode(0, M=1))
    art = intent.compile(intent.weight_only_int4_asym_matmul, target=intent.MI355XTarget(0))
    sets = [(d["x"].clone(), d["packed"].clone(), d["scales"].clone(), d["zeros"].clone()) for _ in range(40)]
    for call in [art.prepare(*s) for s in sets]:
        call.launch()
    torch.cuda.synchronize()
    n = 64 << 20
    for _ in range(4):
        a = torch.empty(n, dtype=torch.uint8, device="cuda")
        b = torch.empty(n, dtype=torch.uint8, device="cuda")
        b.copy_(a)
    torch.cuda.synchronize()


def decode_probe() -> None:
    """40 plain launches each of config 1's decode at M = 1 and M = 16, every launch on its own
    copy of the weights (so each reads them from HBM), for per-dispatch PMC counters."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    art = intent.compile(intent.weight_only_int4_asym_matmul, target=intent.MI355XTarget(0))
    for M in (1, 16):
        d = inputs.to_device(inputs.config1_w4a16_decode(0, M=M))
        sets = [(d["x"].clone(), d["packed"].clone(), d["scales"].clone(), d["zeros"].clone()) for _ in range(40)]
        for call in [art.prepare(*s) for s in sets]:
            call.launch()
        torch.cuda.synchronize()
        log(f"[probe] decode M={M}: {art.observation.kernel}")
        del sets, d


def read_probe(steps: int) -> None:
    """Plain HBM read of the decode's bytes, without and with one small store per wave (a
    GEMV writes its outputs, and a kernel's end waits for its stores), with plain and with
    non-temporal loads, against the decode GEMV, all rotated over the same copy count."""
    import ctypes

    import torch

    from intent_amd import _native, inputs

    work = inputs.w4a16_work(1, 4096, 4096)
    nbytes = (work.bytes + 15) // 16 * 16
    n = copies_for(nbytes)
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(n)]
    words = 8 * ((nbytes + 4095) // 4096)
    sink = torch.zeros(words, dtype=torch.int32, device="cuda")
    lib = _native.library()
    results = {}
    for store in (0, 1, 2, 3):  # bit 0: one store per wave; bit 1: non-temporal loads
        for unroll in (1, 2, 4, 8, 16):
            def make(buf, u=unroll, st_=store):
                def go():
                    stream = torch.cuda.current_stream().cuda_stream
                    st = lib.intent_hbm_read_probe(ctypes.c_void_p(buf.data_ptr()), nbytes, u, st_,
                                                   ctypes.c_void_p(sink.data_ptr()), words, ctypes.c_void_p(stream))
                    if st != 0:
                        raise RuntimeError(_native.last_error())
                return go
            ms = graph_time([make(b) for b in bufs], steps, 10)
            name = f"hbm_read_probe_kernel<{unroll}, {store}>"
            results[name] = ms
            log(f"[probe] read unroll={unroll} store={store}: {ms * 1e3:.3f} us, "
                f"{nbytes / (ms * 1e-3) / 1e9:.1f} GB/s")
    del bufs
    torch.cuda.empty_cache()
    dec = bench_w4a16(1, 4096, 4096, steps, 10)
    results[dec["kernel"]] = dec["ms"]
    log(f"[probe] decode {dec['kernel']}: {dec['ms'] * 1e3:.3f} us")
    print(json.dumps({"probe": "read", "bytes": nbytes, "copies": n, "steps": steps,
                      "us": {k: round(v * 1e3, 4) for k, v in results.items()},
                      "GB/s": {k: round(nbytes / (v * 1e-3) / 1e9, 1) for k, v in results.items()}}), flush=True)


def mfma_ceiling() -> dict:
    """Sustained register-only MFMA rate (f16 and i8) over the whole chip, timed with HIP events."""
    import ctypes

    import torch

    from intent_amd import _native

    lib = _native.library()
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    out = {}
    wgs, iters = 2048, 256  # 8 waves per SIMD; about 0.15 ms per launch, so ramp-up and drain stay small
    for kind, label, per in ((0, "f16", 32768), (1, "i8", 65536)):
        def go():
            st = lib.intent_mfma_peak_probe(kind, iters, wgs, ctypes.c_void_p(sink.data_ptr()),
                                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if st != 0:
                raise RuntimeError(_native.last_error())
        go()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            go()
        b.record()
        b.synchronize()
        ms = a.elapsed_time(b) / 5
        flops = wgs * 4 * iters * 4 * per
        out[label] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
        log(f"[probe] mfma ceiling {label}: {out[label]}")
    return out


def mfma_probe() -> None:
    """The MFMA ceiling probe, then three plain launches of each compute-bound line, for
    per-dispatch rocprofv3 counters."""
    import torch

    import intent_amd as intent
    from intent_amd import inputs

    print(json.dumps({"probe": "mfma_ceiling", **mfma_ceiling()}), flush=True)
    target = intent.MI355XTarget(0)
    d = inputs.to_device(inputs.config1_w4a16_decode(0, M=2048, K=4096, N=11008))
    art = intent.compile(intent.weight_only_int4_asym_matmul, target=target)
    call = art.prepare(d["x"], d["packed"], d["scales"], d["zeros"])
    for _ in range(3):
        call.launch()
    torch.cuda.synchronize()
    log(f"[probe] prefill: {art.observation.kernel}")
    del call, d
    d = inputs.to_device(inputs.config3_w8a8(0))
    art = intent.compile(intent.w8a8_scaled_matmul, target=target)
    call = art.prepare(d["a"], d["a_scales"], d["w"], d["w_scales"])
    for _ in range(3):
        call.launch()
    torch.cuda.synchronize()
    log(f"[probe] w8a8: {art.observation.kernel}")
    del call, d
    h = inputs.config4_moe(0)
    d = inputs.to_device(h)
    T, H = h["x"].shape
    art = intent.compile(intent.moe_expert_ffn_w4, target=target, constexprs={"TOP_K": 2})
    y = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    call = art.prepare(d["logits"], d["x"], d["wgu"], d["sgu"], d["zgu"], d["wd"], d["sd"], d["zd"], y)
    for _ in range(3):
        call.launch()
    torch.cuda.synchronize()
    log("[probe] moe done")


def kn_probe() -> None:
    """Scaled FP8 GEMM, N=14336, K=4096, plain and split-K (SP 4): the [K, N] operand
    read in place (intent_scaled_fp8_gemm_kn) against intent_fp8_transpose followed by
    the row-form kernel, one JSON line per M (graph-timed, operands resident)."""
    import torch

    from intent_amd import _native

    N, K = 14336, 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    b = torch.randn((K, N), device="cuda", generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
    bt = torch.empty((N, K), dtype=torch.uint8, device="cuda")

    def stream():
        return torch.cuda.current_stream().cuda_stream

    for M in (256, 512, 1024, 2048, 4096):
        a = torch.randn((M, K), device="cuda", generator=g).to(torch.float8_e4m3fn).view(torch.uint8)
        o = torch.zeros((M, N), device="cuda", dtype=torch.float16)
        for sp in (1, 4):
            def in_place(a=a, o=o, sp=sp, M=M):
                _native.call("intent_scaled_fp8_gemm_kn", a.data_ptr(), M, K, K, b.data_ptr(), N, N, 1.0, 1.0, sp,
                             int(sp > 1), o.data_ptr(), N, stream())

            def transpose():
                _native.call("intent_fp8_transpose", b.data_ptr(), K, N, N, bt.data_ptr(), K, stream())

            def copy_rows(a=a, o=o, sp=sp, M=M):
                transpose()
                _native.call("intent_scaled_fp8_gemm", a.data_ptr(), M, K, K, bt.data_ptr(), N, K, 1.0, 1.0, sp,
                             int(sp > 1), o.data_ptr(), N, stream())

            row = {"probe": "fp8_kn", "M": M, "N": N, "K": K, "splits": sp,
                   "in_place_us": round(graph_time([in_place], 30, 3) * 1e3, 1),
                   "copy_plus_rows_us": round(graph_time([copy_rows], 30, 3) * 1e3, 1)}
            if M == 256 and sp == 1:
                row["copy_alone_us"] = round(graph_time([transpose], 30, 3) * 1e3, 1)
            print(json.dumps(row), flush=True)


def ablation_probe(steps: int, warmup: int) -> None:
    """Config 3 (W8A8, M=4096, N=K=8192) through `intent_w8a8_gemm` and the FP4 x bf16 case
    (M=N=K=4096) through `intent_fp4_bf16_matmul`, each in the product library and in every
    ablation library (intent_amd.build.ABLATIONS) that has been built: one JSON line per
    (library, entry), HIP-graph timed over rotations of input copies as in the bench."""
    import ctypes

    import torch

    from intent_amd import _native, build as B
    from intent_amd import inputs

    h = inputs.config3_w8a8(0)
    M, K = h["a"].shape
    N = h["w"].shape[0]
    n = copies_for(M * K + N * K + 2 * M * N, minimum=2)
    w8_sets = []
    for _ in range(n):
        d = inputs.to_device(h)
        d["out"] = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        w8_sets.append(d)
    F = 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    x = (torch.randn((F, F), device="cuda", generator=g) * 0.125).bfloat16()
    wq = torch.randint(0, 256, (F, F // 2), device="cuda", generator=g, dtype=torch.uint8)
    fp4_sets = [(x.clone(), wq.clone(), torch.empty((F, F), dtype=torch.bfloat16, device="cuda"))
                for _ in range(copies_for(F * F * 2 + F * F // 2 + F * F * 2, minimum=2))]

    def w8a8_calls(fn):
        def make(d):
            return lambda: fn(d["a"].data_ptr(), M, K, K, d["a_scales"].data_ptr(), d["w"].data_ptr(), N, K,
                              d["w_scales"].data_ptr(), d["out"].data_ptr(), N,
                              torch.cuda.current_stream().cuda_stream)
        return [make(d) for d in w8_sets], 2 * M * N * K

    def fp4_calls(fn):
        def make(xs, ws, ys):
            return lambda: fn(xs.data_ptr(), F, F, F, ws.data_ptr(), F, F // 2, ys.data_ptr(), F,
                              torch.cuda.current_stream().cuda_stream)
        return [make(*s) for s in fp4_sets], 2 * F * F * F

    libs = [("product", B.LIBRARY)] + [(name, B.ablation_library(name)) for name in B.ABLATIONS]
    for name, path in libs:
        if not path.exists():
            print(json.dumps({"probe": "ablation", "variant": name, "missing": str(path)}), flush=True)
            continue
        lib = ctypes.CDLL(str(path))
        for entry, calls_for in (("intent_w8a8_gemm", w8a8_calls), ("intent_fp4_bf16_matmul", fp4_calls)):
            fn = getattr(lib, entry)
            fn.argtypes, fn.restype = _native.SIGNATURES[entry][0], ctypes.c_int

            def checked(f, entry=entry):
                def go():
                    rc = f()
                    if rc != 0:
                        raise RuntimeError(f"{name}: {entry} returned {rc}")
                return go

            calls, work = calls_for(fn)
            ms = graph_time([checked(c) for c in calls], steps, warmup)
            print(json.dumps({"probe": "ablation", "variant": name, "library": path.name, "entry": entry,
                              "us": round(ms * 1e3, 1), "TOP/s": round(work / ms / 1e9, 1)}), flush=True)


def _numa_physical_cores(limit: int = 16) -> list[int]:
    """Up to `limit` physical cores (one hardware thread each) of one NUMA node, within this
    process's affinity: the node holding the most allowed cores."""
    allowed = sorted(os.sched_getaffinity(0))

    def cpulist(text: str) -> list[int]:
        out = []
        for part in text.strip().split(","):
            if part:
                lo, _, hi = part.partition("-")
                out.extend(range(int(lo), int(hi or lo) + 1))
        return out

    nodes = []
    for node in sorted(Path("/sys/devices/system/node").glob("node[0-9]*")):
        try:
            cpus = set(cpulist((node / "cpulist").read_text()))
        except OSError:
            continue
        nodes.append([c for c in allowed if c in cpus])
    pool = max(nodes, key=len) if nodes and max(len(n) for n in nodes) else allowed
    chosen, seen = [], set()
    for c in pool:
        try:
            sib = (Path(f"/sys/devices/system/cpu/cpu{c}/topology/thread_siblings_list").read_text().strip())
        except OSError:
            sib = str(c)
        if sib in seen:
            continue
        seen.add(sib)
        chosen.append(c)
        if len(chosen) == limit:
            break
    return chosen or allowed[:limit]


def _median_of_7(run, budget_s: float) -> tuple[float, int]:
    """The reference's CPU timing (experiments/_common/measurement.py:418-438): warm up, then
    the median over 7 batches of the mean wall time per call; batches here are sized to
    fill budget_s in total. Returns (seconds per call, calls timed)."""
    t0 = time.perf_counter()
    run()
    first = time.perf_counter() - t0
    reps = max(1, int(budget_s / 7 / max(first, 1e-6)))
    means = []
    for _ in range(7):
        t0 = time.perf_counter()
        for _ in range(reps):
            run()
        means.append((time.perf_counter() - t0) / reps)
    means.sort()
    return means[3], 7 * reps


def cpu_baseline(budget_s: float) -> dict:
    """The headline workload on this host's CPU, timed the reference's way (median of 7 batches),
    pinned to physical cores of one NUMA node: the C oracle (plain-C port of the reference
    CPU numerics, OpenMP over output rows) as `value`, and a PyTorch-eager restatement
    (dequantise, f32 matmul, f16 cast) beside it."""
    import torch

    import oracle
    from intent_amd import inputs

    cores = _numa_physical_cores(16)
    saved = os.sched_getaffinity(0)
    saved_threads = torch.get_num_threads()
    d = inputs.config1_w4a16_decode(0, M=1)
    work = inputs.w4a16_work(1, 4096, 4096)
    try:
        os.sched_setaffinity(0, cores)
        n = len(cores)
        per, calls = _median_of_7(lambda: oracle.w4a16(d["x"], d["packed"], d["scales"], d["zeros"], n),
                                  budget_s * 0.7)
        torch.set_num_threads(n)
        x = torch.from_numpy(d["x"])
        q = torch.from_numpy(d["packed"])
        sc = torch.from_numpy(d["scales"])
        z = torch.from_numpy(d["zeros"])
        gsz = 4096 // sc.shape[1]

        def eager():
            nib = torch.stack((q & 15, q >> 4), dim=-1).reshape(q.shape[0], -1).float()
            w = (nib - z.float().repeat_interleave(gsz, dim=1)) * sc.float().repeat_interleave(gsz, dim=1)
            return (x.float() @ w.T).half()

        eper, ecalls = _median_of_7(eager, budget_s * 0.3)
    finally:
        os.sched_setaffinity(0, saved)
        torch.set_num_threads(saved_threads)
    return {"value": round(work.bytes / per / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"{calls} W4A16 M=1 K=N=4096 g128 GEMVs, median of 7 batches (oracle/oracle.c, OpenMP), "
                      f"pinned to {n} physical cores of one NUMA node",
            "ms_per_step": round(per * 1e3, 3),
            "torch_eager": {"value": round(work.bytes / eper / 1e9, 3), "unit": "GB/s", "threads": n,
                            "ms_per_step": round(eper * 1e3, 3), "calls": ecalls}}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is not launched in this build)"}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        return 1
    from intent_amd import _native

    if args.probe == "traffic":
        traffic_probe()
        return 0
    if args.probe == "read":
        read_probe(args.steps)
        return 0
    if args.probe == "mfma":
        mfma_probe()
        return 0
    if args.probe == "kn":
        kn_probe()
        return 0
    if args.probe == "decode":
        decode_probe()
        return 0
    if args.probe == "ablation":
        ablation_probe(args.steps, args.warmup)
        return 0
    arch = _native.device_arch(0)
    log(f"[bench] device 0: {arch}; decode M=1 steps={args.steps} warmup={args.warmup}")
    dec = bench_w4a16(1, 4096, 4096, args.steps, args.warmup)
    ms = dec["ms"]
    gbs = dec["work"].bytes / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded numpy draws of BASELINE configs (weights copied to exceed MALL)",
        "config": {"workload": "w4a16 decode GEMV M=1 K=4096 N=4096 g128 asymmetric uint4 (BASELINE configs[1])",
                   "entry": dec["entry"], "weight_copies": dec["copies"],
                   "rotation_bytes": dec["rotation_bytes"], "arch": arch},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dec["kernel"]),
                     "bytes_per_launch": dec["work"].bytes, "kernel": dec["kernel"]},
    }
    extra = {}
    if args.only == "all":
        steps = max(10, min(args.steps, 50))
        warm = max(2, min(args.warmup, 5))  # plus WARM_SECONDS of rotation replays inside graph_time
        log("[bench] decode M=16")
        r = bench_w4a16(16, 4096, 4096, args.steps, args.warmup)
        extra["w4a16_decode_m16"] = dict(_hbm_entry(r), kernel=r["kernel"], rotation_bytes=r["rotation_bytes"])
        log("[bench] prefill M=2048 N=11008")
        r = bench_w4a16(2048, 4096, 11008, steps, warm)
        extra["w4a16_prefill_m2048"] = _flop_entry(r, F16_PEAK_TFLOPS, "TFLOP/s")
        log("[bench] per-token int8 quantize M=4096 K=8192")
        r = bench_i8_quant(args.steps, args.warmup)
        extra["i8_per_token_quantize_m4096_k8192"] = _hbm_entry(r)
        log("[bench] w8a8 M=4096 K=N=8192")
        r = bench_w8a8(steps, warm)
        extra["w8a8_m4096"] = _flop_entry(r, I8_PEAK_TOPS, "TOP/s")
        log("[bench] moe T=512 E8 top2")
        r = bench_moe(max(5, steps // 5), warm)
        e = _flop_entry(r, F16_PEAK_TFLOPS, "TFLOP/s")
        e["GB/s"] = round(r["work"].bytes / (r["ms"] * 1e-3) / 1e9, 2)
        e["hbm_frac"] = round(e["GB/s"] / HBM_PEAK_GBS, 4)
        extra["moe_w4_t512"] = e
        log("[bench] w8a16 M=16")
        r = bench_w8a16(args.steps, args.warmup)
        extra["w8a16_m16"] = _hbm_entry(r)
        log("[bench] w4a8 M=4096 K=4096 N=14336")
        r = bench_w4a8(steps, warm)
        extra["w4a8_m4096_n14336"] = _flop_entry(r, I8_PEAK_TOPS, "TOP/s")
        log("[bench] mxfp8 M=4096 K=4096 N=14336")
        r = bench_mxfp8(steps, warm)
        extra["mxfp8_m4096_n14336"] = _flop_entry(r, 5033.2, "TFLOP/s")
        log("[bench] scaled fp8 split-K M=4096 K=4096 N=14336")
        r = bench_sfp8_splitk(steps, warm)
        extra["scaled_fp8_splitk_m4096_n14336"] = _flop_entry(r, 5033.2, "TFLOP/s")
        log("[bench] deepgemm fp8 M=N=K=4096")
        r = bench_deepgemm(steps, warm)
        extra["deepgemm_fp8_4096"] = _flop_entry(r, 5033.2, "TFLOP/s")
        log("[bench] fp4 x bf16 M=N=K=4096")
        r = bench_fp4(steps, warm)
        extra["fp4_bf16_4096"] = _flop_entry(r, F16_PEAK_TFLOPS, "TFLOP/s")
        log("[bench] quantized_gemm M=4096 K=4096 N=14336")
        r = bench_quantized_gemm(steps, warm)
        extra["quantized_gemm_m4096_n14336"] = _flop_entry(r, F16_PEAK_TFLOPS, "TFLOP/s")
        log("[bench] f16 moe_expert_ffn T=D=4096 F=14336")
        r = bench_moe_f16(max(2, steps // 10), 1)
        extra["moe_expert_ffn_f16_t4096"] = _flop_entry(r, F16_PEAK_TFLOPS, "TFLOP/s")
        log("[bench] q4_k projection N=K=4096")
        r = bench_q4k(args.steps, args.warmup)
        extra["q4k_projection_n4096"] = _hbm_entry(r)
    line["extra"] = extra
    if not args.no_cpu:
        log(f"[bench] cpu baseline ({args.cpu_seconds:.0f} s budget)")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


def _hbm_entry(r: dict) -> dict:
    gbs = r["work"].bytes / (r["ms"] * 1e-3) / 1e9
    return {"workload": r["work"].name, "ms": round(r["ms"], 6), "GB/s": round(gbs, 2),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "TFLOP/s": round(r["work"].flops / (r["ms"] * 1e-3) / 1e12, 3)}


def _flop_entry(r: dict, peak: float, unit: str) -> dict:
    tf = r["work"].flops / (r["ms"] * 1e-3) / 1e12
    return {"workload": r["work"].name, "ms": round(r["ms"], 6), unit: round(tf, 2), "peak": peak,
            "frac": round(tf / peak, 4), "GB/s": round(r["work"].bytes / (r["ms"] * 1e-3) / 1e9, 2)}


if __name__ == "__main__":
    sys.exit(main())
