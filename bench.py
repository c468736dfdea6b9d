#!/usr/bin/env python3
"""Benchmark of the ConvRot INT8 linear path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle S] [--no-cpu]

A *step* is one ``xpu_kernels.int8.linear`` at config 3 of BASELINE.json
(x bf16 [4096,1280] with 1% outlier channels x30, W prepared from bf16
[10240,1280], bias bf16 [10240]): rotate+quantize of x, then the int8 MFMA
GEMM with the dequant+bias epilogue fused into its store.  Inputs are resident
in HBM before the timed region and *cold*: each call takes its own set of
(x, w8, w_scale, bias), and the sets together exceed 640 MB, so no call finds
its operands in the 256 MB Infinity Cache or the L2s (the buffer-warmth trap
the reference's docs/performance.md:104-114 warns about).  The same call on
one set of buffers is reported beside it as the warm figure.  Weights are
prepared once, untimed.  An untimed run-in of S seconds (default 0.25, so the
GPU clock reaches its sustained level), W warm-up steps, then exactly K steps
between two ``torch.cuda.synchronize()`` calls, timed with HIP events on the
stream the kernels run on (torch's current stream).

``value`` is end-to-end TOP/s at config 3 (2*M*N*K = 107.37 GOP per step).
The other configurations are measured after it and reported under ``extra``,
the HBM-bound ones cold and warm.  ``roofline`` is the GEMM kernel's own
average duration (cold operands) against the dense INT8 MFMA peak;
``cpu_baseline`` times the reference's oracle (reference/convrot_linear.py,
restated in torch with the real rotation: oracle/torch_chain.py) on this
host's cores.  One JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "oko-xpu-kernels_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_INT8_TOPS = 5000.0          # MI355X dense int8 MFMA, TOP/s
PEAK_HBM_GBPS = 8000.0           # MI355X HBM3E, GB/s
CALIB_BYTES = 256 << 20          # size of the --calibrate-copy kernel's input and output
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_i8_dequant_c3_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the config-3 GEMM, as measured by the two
    rocprofv3 counter passes summarised in TRAFFIC_FILE (the line
    ``traffic_bytes_per_launch: N``); None when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def activation(torch, m, k, seed=0, n_out=None, mult=30.0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * scale
    n_out = max(1, round(0.01 * k)) if n_out is None else n_out
    if n_out:
        x[:, torch.randperm(k, generator=g)[:n_out]] *= mult
    return x.to(torch.bfloat16)


def weight(torch, n, k, seed=1, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=g) * std).to(torch.bfloat16)


SETTLE_S = 0.25                  # untimed run-in per measurement, seconds (see settle())


def settle(torch, fn, seconds):
    """Run ``fn`` untimed for about ``seconds``.  The MI355X's shader clock
    ramps up over the first tens of milliseconds of sustained load (measured
    with s_memtime against s_memrealtime inside the GEMM: ~1.6 GHz after an
    idle period, ~2.0 GHz after 30 ms of back-to-back launches on full-range
    int8 data), so without a run-in a short timed region measures the ramp,
    not the steady state a serving loop runs at."""
    if seconds <= 0:
        return
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


def timed(torch, fn, steps, warmup, settle_s=0.0):
    """Average ms per call of ``fn(i)`` over calls i = 0 .. steps-1 (HIP events
    on the current stream, after a ``settle_s`` run-in and ``warmup`` untimed
    calls).  ``fn`` takes the call index so that a cold measurement can walk
    through several buffer sets."""
    settle(torch, lambda: fn(0), settle_s)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def timed_graph(torch, fn, calls, reps=4, settle_s=0.0):
    """Average ms per launch of ``fn(i, stream)`` for i = 0 .. calls-1,
    captured once into a HIP graph on a side stream and replayed ``reps``
    times (after a ``settle_s`` run-in of replays).  Launches in a graph leave
    the host's per-call cost (ctypes, argument checks, the launch itself,
    ~4 us from a Python loop) out of the figure, so a kernel shorter than
    that is timed by the GPU, back to back with its neighbours, each launch
    still on its own buffer set."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            fn(i, s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(calls):
            fn(i, s.cuda_stream)
    settle(torch, g.replay, settle_s)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) / (reps * calls)


COLD_BYTES = 640 << 20           # buffer sets per cold measurement: > 2.5x the 256 MB MALL


def n_sets(bytes_per_set, cap=48):
    """How many distinct buffer sets a cold measurement rotates through, so
    that the bytes touched between two uses of one set exceed the MI355X's
    256 MB Infinity Cache (and the 4 MB L2s): each call then reads its inputs
    from HBM, as the reference's own measurement notes require (fresh
    buffers, docs/performance.md:104-114)."""
    return max(2, min(cap, -(-COLD_BYTES // int(bytes_per_set))))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds):
    """The reference's own oracle, reference/convrot_linear.py:5-23, as a
    torch-CPU chain with the real rotation in place of its identity
    (oracle/torch_chain.py), on this host's cores: the full config 1 and a
    row sample of config 3, median of >= 5 runs each."""
    import statistics
    import torch
    from oracle import torch_chain as TC
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", affinity) or affinity)
    threads = max(1, min(affinity, share))
    torch.set_num_threads(threads)
    h = TC.hadamard_matrix()

    def case(m, k, n, seed):
        x = activation(torch, m, k, seed=seed, n_out=8 if m == 1024 and n == 1280 else None,
                       mult=20.0 if m == 1024 and n == 1280 else 30.0)
        g = torch.Generator().manual_seed(seed + 1)
        w8 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        ws = torch.rand(n, generator=g) * 1e-3 + 1e-4
        bias = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
        return x, w8, ws, bias

    def median_ms(args, budget):
        TC.convrot_int8_linear(*args, h=h)                   # warm-up
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            TC.convrot_int8_linear(*args, h=h)
            times.append(time.perf_counter() - t0)
        return statistics.median(times) * 1e3, len(times)

    c1 = case(1024, 1280, 1280, 0)
    ms1, n1 = median_ms(c1, seconds * 0.25)
    m3 = 1024
    c3 = case(m3, 1280, 10240, 3)
    ms3, n3 = median_ms(c3, seconds * 0.75)
    ops3 = 2.0 * m3 * 10240 * 1280
    return {
        "value": round(ops3 / (ms3 * 1e-3) / 1e12, 5),
        "unit": "TOP/s",
        "cores": threads,
        "kind": "port",
        "cpu": cpu_model(),
        "affinity_cpus": affinity,
        "config1_ms": round(ms1, 3),
        "config1_GOP/s": round(2.0 * 1024 * 1280 * 1280 / (ms1 * 1e-3) / 1e9, 2),
        "sample": f"reference/convrot_linear.py restated in torch on the CPU (fp32 256x256 "
                  f"Hadamard matmul, fp32 scale, IEEE division, torch._int_mm, dequant, bf16 "
                  f"bias) at {threads} threads: config 3 on {m3} of its 4096 rows "
                  f"(K=1280, N=10240), median of {n3} runs ({ms3:.1f} ms each); config 1 "
                  f"(1024x1280x1280) in full, median of {n1} runs",
    }


def measure_side_rows(torch, int8, lib, L, st, dev, K, W, SET, extra, hbm_line, dev_gen,
                      dev_act, dev_weight, x, w8, ws, bias):
    """The entry points beside the config-3 step, each at the shape its caller
    uses: the int32 GEMM of ``linear_acc``, ``linear``'s fused residual, the
    standalone epilogues, the activation quantizers, ``dequant_weight``, the
    reference's SDXL shape table (``linear`` against torch's bf16 linear) and
    an ``int8_linear`` training step (forward + backward) at config 5.  The
    HBM-bound ones are timed cold (rotating buffer sets) and warm; the GEMMs
    of config 3 warm, on its operands; the SDXL shapes cold."""
    M, Kd, N = 4096, 1280, 10240
    ops3 = 2.0 * M * N * Kd
    xq, xs = int8.quantize(x)

    def C(fn, *a):
        if fn(st, *a) != 0:
            L._err(lib, fn.__name__)

    # linear_acc's GEMM (int32 out, 4 bytes per element stored) and
    # linear(residual=, residual_scale=) with the addcmul in the store
    acc = torch.empty((M, N), device=dev, dtype=torch.int32)
    out = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    res = (torch.randn(M, N, device=dev, generator=dev_gen(900)) * 0.1).to(torch.bfloat16)
    rsc = (torch.rand(N, device=dev, generator=dev_gen(901)) + 0.5).to(torch.bfloat16)
    ms_i32 = timed(torch, lambda i: C(lib.xpuint8_int8_gemm_stream, L._ptr(xq), L._ptr(w8),
                                      L._ptr(acc), M, N, Kd), K, W, SET)
    ms_res = timed(torch, lambda i: C(lib.xpuint8_linear_gemm_residual_stream, L._ptr(xq),
                                      L._ptr(xs), L._ptr(w8), L._ptr(ws), L._ptr(bias), 1,
                                      L._ptr(res), L._ptr(rsc), L._ptr(out), M, N, Kd),
                   K, W, SET)
    ms_acc_api = timed(torch, lambda i: int8.linear_acc(x, w8, ws), K, W, SET)
    # the API calls: one library call each (quantize into the GEMM's block
    # layout, then the GEMM reading the weight's packed copy)
    bias16 = bias.to(torch.bfloat16)
    ms_res_api = timed(torch, lambda i: int8.linear(x, w8, ws, bias16, residual=res,
                                                    residual_scale=rsc), K, W, SET)
    extra["config3_linear_acc"] = {
        "gemm_int32_ms_warm": round(ms_i32, 5),
        "gemm_int32_TOP/s_warm": round(ops3 / (ms_i32 * 1e-3) / 1e12, 1),
        "api_ms_warm": round(ms_acc_api, 5),
        "api_TOP/s_warm": round(ops3 / (ms_acc_api * 1e-3) / 1e12, 1)}
    extra["config3_linear_residual"] = {
        "gemm_residual_ms_warm": round(ms_res, 5),
        "TOP/s_warm": round(ops3 / (ms_res * 1e-3) / 1e12, 1),
        "api_ms_warm": round(ms_res_api, 5),
        "api_TOP/s_warm": round(ops3 / (ms_res_api * 1e-3) / 1e12, 1)}
    log(f"[bench] linear_acc int32 GEMM {ms_i32:.4f} ms (API {ms_acc_api:.4f}); "
        f"GEMM + residual {ms_res:.4f} ms (API {ms_res_api:.4f})")
    del out, res

    # the standalone epilogues on an int32 accumulator: dequant of [M, N], and
    # dequant_slice of the q columns [M, 3072] of a [M, 9216] qkv accumulator
    xs32 = torch.rand(M, device=dev, generator=dev_gen(902)) * 0.01
    ws32 = torch.rand(N, device=dev, generator=dev_gen(903)) * 0.01
    b32 = torch.randn(N, device=dev, generator=dev_gen(904)) * 0.01
    bytes_dq = 6 * M * N + 4 * M + 8 * N
    ndq = n_sets(bytes_dq)
    dq = [(acc if i == 0 else torch.randint(-2 ** 20, 2 ** 20, (M, N), device=dev,
                                            generator=dev_gen(910 + i), dtype=torch.int32),
           torch.empty((M, N), device=dev, dtype=torch.bfloat16)) for i in range(ndq)]

    def deq(i):
        a, o = dq[i % ndq]
        C(lib.xpuint8_dequant_epilogue_stream, L._ptr(a), L._ptr(o), L._ptr(xs32), L._ptr(ws32),
                                            L._ptr(b32), M, N)
    extra["config3_dequant"] = hbm_line(bytes_dq, timed(torch, deq, K, W, SET),
                                        timed(torch, lambda i: deq(0), K, W, SET), sets=ndq)
    del dq, acc

    # the GEMM the reference itself calls (torch._int_mm, ops.py:634; hipBLASLt
    # here) against this library's int32 GEMM, cold, on the same int8 operands:
    # with the standalone dequant and quantize above, the reference's unfused
    # step on this GPU
    nim = n_sets(M * Kd + Kd * N + 4 * M * N)
    im = [(torch.randint(-127, 128, (M, Kd), device=dev, generator=dev_gen(990 + i),
                         dtype=torch.int8),
           torch.randint(-127, 128, (Kd, N), device=dev, generator=dev_gen(1090 + i),
                         dtype=torch.int8)) for i in range(nim)]
    imw = [b.t().contiguous() for _, b in im]
    imo = [torch.empty((M, N), device=dev, dtype=torch.int32) for _ in range(nim)]
    ms_tim = timed(torch, lambda i: torch._int_mm(im[i % nim][0], im[i % nim][1]), K, W, SET)

    def own_i32(i):
        C(lib.xpuint8_int8_gemm_stream, L._ptr(im[i % nim][0]), L._ptr(imw[i % nim]),
          L._ptr(imo[i % nim]), M, N, Kd)
    ms_oim = timed(torch, own_i32, K, W, SET)
    extra["config3_torch_int_mm"] = {
        "torch_int_mm_ms_cold": round(ms_tim, 5),
        "torch_int_mm_TOP/s_cold": round(ops3 / (ms_tim * 1e-3) / 1e12, 1),
        "xpuint8_int32_gemm_ms_cold": round(ms_oim, 5),
        "xpuint8_int32_gemm_TOP/s_cold": round(ops3 / (ms_oim * 1e-3) / 1e12, 1),
        "sets": nim}
    if "config3_quantize" in extra:
        extra["config3_torch_int_mm"]["unfused_step_ms_cold"] = round(
            extra["config3_quantize"]["ms_cold"] + ms_tim + extra["config3_dequant"]["ms_cold"], 5)
    log(f"[bench] torch._int_mm {ms_tim:.4f} ms cold, this library's int32 GEMM {ms_oim:.4f} ms")
    del im, imw, imo
    Nq, Nqkv = 3072, 9216
    bytes_sl = 6 * M * Nq + 4 * M + 8 * Nq
    nsl = n_sets(bytes_sl)
    sl = [(torch.randint(-2 ** 20, 2 ** 20, (M, Nqkv), device=dev, generator=dev_gen(960 + i),
                         dtype=torch.int32),
           torch.empty((M, Nq), device=dev, dtype=torch.bfloat16)) for i in range(nsl)]

    def deq_slice(i):
        a, o = sl[i % nsl]
        C(lib.xpuint8_dequant_epilogue_slice_stream, L._ptr(a), L._ptr(o), L._ptr(xs32),
                                                  L._ptr(ws32), L._ptr(b32), M, Nq, Nqkv)
    extra["qkv_dequant_slice_m4096_n3072"] = hbm_line(
        bytes_sl, timed(torch, deq_slice, K, W, SET), timed(torch, lambda i: deq_slice(0), K, W, SET),
        sets=nsl)
    del sl

    # quantize_act: GELU-erf on [4096, 5120], GEGLU-erf on [4096, 2*5120]
    Mr, Kr = 4096, 5120
    for name, aid, width in (("gelu_erf", 5, Kr), ("geglu_erf", 4, 2 * Kr)):
        bytes_a = 2 * Mr * width + Mr * Kr + 4 * Mr
        na = n_sets(bytes_a)
        sa = [(dev_act(Mr, width, 1000 + 50 * aid + i),
               torch.empty((Mr, Kr), device=dev, dtype=torch.int8),
               torch.empty(Mr, device=dev, dtype=torch.float32)) for i in range(na)]

        def qa(i, sa=sa, na=na, aid=aid):
            xi, qi, si = sa[i % na]
            C(lib.xpuint8_convrot_quantize_act_stream, L._ptr(xi), L._ptr(qi), L._ptr(si),
                                                    Mr, Kr, aid)
        extra[f"quantize_act_{name}_m4096_k5120"] = hbm_line(
            bytes_a, timed(torch, qa, K, W, SET), timed(torch, lambda i: qa(0), K, W, SET), sets=na)
        del sa

    # dequant_act_quantize (the reference's FFN middle step): GEGLU on an int32
    # [4096, 2*5120] accumulator
    bytes_daq = 4 * Mr * 2 * Kr + Mr * Kr + 4 * Mr + 8 * Kr + 4 * Mr
    ndaq = n_sets(bytes_daq)
    xsd = torch.rand(Mr, device=dev, generator=dev_gen(1300)) * 1e-3
    wsd = torch.rand(2 * Kr, device=dev, generator=dev_gen(1301)) * 1e-3
    sd = [(torch.randint(-2 ** 20, 2 ** 20, (Mr, 2 * Kr), device=dev, generator=dev_gen(1310 + i),
                         dtype=torch.int32),
           torch.empty((Mr, Kr), device=dev, dtype=torch.int8),
           torch.empty(Mr, device=dev, dtype=torch.float32)) for i in range(ndaq)]

    def daq(i):
        a, qi, si = sd[i % ndaq]
        C(lib.xpuint8_dequant_act_quantize_stream, L._ptr(a), L._ptr(qi), L._ptr(si), L._ptr(xsd),
                                                L._ptr(wsd), Mr, Kr, 4)
    extra["dequant_act_quantize_geglu_m4096_k5120"] = hbm_line(
        bytes_daq, timed(torch, daq, K, W, SET), timed(torch, lambda i: daq(0), K, W, SET),
        sets=ndaq)
    del sd

    # dequant_weight of a config-2 weight [10240, 1280]
    bytes_dw = 3 * 10240 * 1280 + 4 * 10240
    ndw = n_sets(bytes_dw)
    sw = [int8.prepare_weight(dev_weight(10240, 1280, 1400 + i)) for i in range(ndw)]
    ow = [torch.empty((10240, 1280), device=dev, dtype=torch.bfloat16) for _ in range(ndw)]

    def dqw(i):
        w_i, s_i = sw[i % ndw]
        C(lib.xpuint8_dequant_weight_stream, L._ptr(w_i), L._ptr(s_i), L._ptr(ow[i % ndw]),
                                          10240, 1280)
    extra["dequant_weight_n10240_k1280"] = hbm_line(
        bytes_dw, timed(torch, dqw, K, W, SET), timed(torch, lambda i: dqw(0), K, W, SET), sets=ndw)
    del sw, ow

    # the reference's SDXL shape table (docs/sdxl.md:40-47, batch 1 at
    # 1024x1024, M = 4096 tokens): int8.linear end to end and torch's bf16
    # F.linear on the same (cold) inputs, with the reference's published
    # device time on its GPU (Arc B580) beside them
    sdxl = {}
    for Ks, Ns, ref_ms in ((5120, 1280, 0.647), (2048, 1280, 0.366), (1280, 1280, 0.289),
                           (1280, 10240, 1.980)):
        Ms = 4096
        nss = n_sets(2 * Ms * Ks + 3 * Ns * Ks + 2 * Ms * Ns)
        ss = []
        for i in range(nss):
            wb = dev_weight(Ns, Ks, 1600 + i)
            ss.append((dev_act(Ms, Ks, 1700 + i), *int8.prepare_weight(wb),
                       dev_weight(1, Ns, 1800 + i, 0.01)[0], wb))
        t_i8 = timed(torch, lambda i: int8.linear(*ss[i % nss][:4]), K, W, SET)
        t_bf = timed(torch, lambda i: torch.nn.functional.linear(ss[i % nss][0], ss[i % nss][4],
                                                                 ss[i % nss][3]), K, W, SET)
        # the same calls replayed from HIP graphs (one launch sequence per
        # call, each call on its own set): the GPU's time per call without the
        # Python host cost of either API (int8.linear's is ~16 us per call)
        g_i8 = timed_graph(torch, lambda i, s: int8.linear(*ss[i % nss][:4]), nss, settle_s=SET)
        g_bf = timed_graph(torch, lambda i, s: torch.nn.functional.linear(
            ss[i % nss][0], ss[i % nss][4], ss[i % nss][3]), nss, settle_s=SET)
        sdxl[f"K{Ks}_N{Ns}_M{Ms}"] = {
            "int8_linear_ms_cold": round(t_i8, 5),
            "int8_TOP/s": round(2.0 * Ms * Ns * Ks / (t_i8 * 1e-3) / 1e12, 1),
            "torch_bf16_linear_ms_cold": round(t_bf, 5),
            "int8_over_bf16": round(t_i8 / t_bf, 3),
            "graph_int8_linear_ms_cold": round(g_i8, 5),
            "graph_torch_bf16_linear_ms_cold": round(g_bf, 5),
            "graph_int8_over_bf16": round(g_i8 / g_bf, 3),
            "reference_b580_int8_ms": ref_ms}
        del ss
    extra["sdxl_shapes"] = sdxl
    log("[bench] SDXL shapes: " + ", ".join(f"{k} {v['int8_linear_ms_cold'] * 1e3:.1f} us "
                                            f"(bf16 {v['torch_bf16_linear_ms_cold'] * 1e3:.1f}; "
                                            f"graphs {v['graph_int8_linear_ms_cold'] * 1e3:.1f} / "
                                            f"{v['graph_torch_bf16_linear_ms_cold'] * 1e3:.1f})"
                                            for k, v in sdxl.items()))

    # int8_linear training step at config 5 shapes: forward, then backward
    # (dx, dbias; the weight is frozen int8), for both backward modes
    x5 = dev_act(4096, 1280, 1500).requires_grad_(True)
    w5_8, w5_s = int8.prepare_weight(dev_weight(5120, 1280, 1501))
    b5 = dev_weight(1, 5120, 1502, 0.01)[0].requires_grad_(True)
    dy5 = (torch.randn(4096, 5120, device=dev, generator=dev_gen(1503)) * 1e-3).to(torch.bfloat16)
    ops_step = 2 * (2.0 * 4096 * 5120 * 1280)
    for mode in ("int8", "dense"):
        def step(i, mode=mode):
            x5.grad = None
            b5.grad = None
            int8.int8_linear(x5, w5_8, w5_s, b5, mode=mode).backward(dy5)
        ms_st = timed(torch, step, K, W, SET)
        extra[f"config5_int8_linear_step_{mode}"] = {
            "ms": round(ms_st, 5), "TOP/s": round(ops_step / (ms_st * 1e-3) / 1e12, 1)}
        log(f"[bench] int8_linear step ({mode} backward): {ms_st:.4f} ms")


def measure_small_batch(torch, int8, lib, L, st, dev, K, W, SET, extra, dev_act, dev_weight,
                        ops):
    """Small batches (batched decode) at config 4's widths, weights cold
    (rotating sets of > 640 MB): the whole FFN (x [M,1280] -> GEGLU [M,5120]
    -> [M,1280], bf16 bias) as one ``xpuint8_ffn_packed_stream`` call and the
    linear of its down-projection shape (K=5120, N=1280) as one
    ``xpuint8_linear_packed_stream`` call (the weights' packed copies, as
    ``prepare_weight`` makes them), both on preallocated buffers, the FFN
    reading the row-major weights (``xpuint8_ffn_stream``), and the
    ``int8.ffn`` API call (host work included) beside them, at M = 1, 64, 128,
    200.
    At these sizes the weights are most of the traffic (19.66 MB per FFN,
    6.55 MB per linear); ``weights_GB/s`` is that over the call's time."""
    k, f = 1280, 5120
    nf = n_sets(3 * f * k)
    ffw = [int8.prepare_weight(dev_weight(2 * f, k, 2000 + i)) + int8.prepare_weight(
        dev_weight(k, f, 2100 + i)) for i in range(nf)]
    ffp = [(ops._packed_for(up8), ops._packed_for(dn8)) for up8, _, dn8, _ in ffw]
    assert all(a is not None and b is not None for a, b in ffp)
    bias = dev_weight(1, k, 2200, 0.01)[0]
    res = {}
    for m in (1, 64, 128, 200):
        x = dev_act(m, k, 2300 + m)
        y = torch.empty((m, k), dtype=torch.bfloat16, device=dev)
        need = lib.xpuint8_ffn_workspace_size(m, f, k, 4)
        work = torch.empty(max(1, need), dtype=torch.uint8, device=dev)

        def ffn(i):
            up8, ups, dn8, dns = ffw[i % nf]
            up_p, dn_p = ffp[i % nf]
            rc = lib.xpuint8_ffn_packed_stream(st, L._ptr(x), L._ptr(up8), L._ptr(up_p),
                                               L._ptr(ups), L._ptr(dn8), L._ptr(dn_p),
                                               L._ptr(dns), L._ptr(bias), 1, L._ptr(y), m, f, k,
                                               4, L._ptr(work), need)
            if rc != 0:
                raise RuntimeError(lib.xpuint8_last_error().decode())

        def ffn_rowmajor(i):
            up8, ups, dn8, dns = ffw[i % nf]
            rc = lib.xpuint8_ffn_stream(st, L._ptr(x), L._ptr(up8), L._ptr(ups), L._ptr(dn8),
                                        L._ptr(dns), L._ptr(bias), 1, L._ptr(y), m, f, k, 4,
                                        L._ptr(work), need)
            if rc != 0:
                raise RuntimeError(lib.xpuint8_last_error().decode())
        ffn(0)
        y_p = y.clone()
        ffn_rowmajor(0)
        assert torch.equal(y_p, y), f"small-batch FFN M={m}: packed and row-major differ"
        ms_ffn = timed(torch, ffn, K, W, SET)
        ms_ffn_rm = timed(torch, ffn_rowmajor, K, W, SET)
        ms_api = timed(torch, lambda i: int8.ffn(x, *ffw[i % nf], bias, act="geglu_erf"),
                       K, W, SET)
        xd = dev_act(m, f, 2400 + m)
        yd = torch.empty((m, k), dtype=torch.bfloat16, device=dev)
        needl = lib.xpuint8_linear_workspace_size(m, k, f)
        workl = torch.empty(max(1, needl), dtype=torch.uint8, device=dev)

        def down(i):
            dn8, dns = ffw[i % nf][2:]
            rc = lib.xpuint8_linear_packed_stream(st, L._ptr(xd), L._ptr(dn8),
                                                  L._ptr(ffp[i % nf][1]), L._ptr(dns),
                                                  L._ptr(bias), 1, L._ptr(yd), m, k, f,
                                                  L._ptr(workl), needl)
            if rc != 0:
                raise RuntimeError(lib.xpuint8_last_error().decode())
        ms_lin = timed(torch, down, K, W, SET)
        res[f"M{m}"] = {"ffn_ms_cold": round(ms_ffn, 5),
                        "ffn_weights_GB/s": round(3 * f * k / (ms_ffn * 1e-3) / 1e9, 1),
                        "ffn_rowmajor_weights_ms_cold": round(ms_ffn_rm, 5),
                        "ffn_api_ms_cold": round(ms_api, 5),
                        "linear_k5120_n1280_ms_cold": round(ms_lin, 5),
                        "linear_weights_GB/s": round(f * k / (ms_lin * 1e-3) / 1e9, 1)}
        del work, workl
    extra["small_batch_c4_widths"] = res
    log("[bench] small batches: " + ", ".join(
        f"M={m[1:]} ffn {v['ffn_ms_cold'] * 1e3:.1f} us (API {v['ffn_api_ms_cold'] * 1e3:.1f}), "
        f"linear {v['linear_k5120_n1280_ms_cold'] * 1e3:.1f} us" for m, v in res.items()))
    del ffw


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="untimed run-in before each measurement, seconds (GPU clock ramp)")
    ap.add_argument("--only-main", action="store_true", help="config 3 only (for profiling)")
    ap.add_argument("--only-rowquant", action="store_true",
                    help="config 2 rotate+quantize only, cold then warm (for profiling)")
    ap.add_argument("--only-gemm", action="store_true",
                    help="the config-3 GEMM alone, cold, and nothing else (for profiling: its "
                         "launches are then the only ones of that kernel in the run)")
    ap.add_argument("--only-c45", action="store_true",
                    help="only configs 4 and 5 (FFN, backward, skinny), for profiling")
    ap.add_argument("--only-side", action="store_true",
                    help="only the entry points beside the path (linear_acc, residual, dequant, "
                         "dequant_slice, quantize_act, dequant_act_quantize, dequant_weight, "
                         "int8_linear step), for profiling")
    ap.add_argument("--only-small", action="store_true",
                    help="only the small-batch FFN and linear lines (M = 1, 64, 128, 200 at "
                         "config 4's widths), for profiling")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain copy kernel (torch neg over 256 MiB in and out, "
                         "exactly 256 MiB) so counter runs can scale FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch
    from xpu_kernels import int8
    from xpu_kernels.int8 import _lib as L
    from xpu_kernels.int8 import ops
    if not int8.available():
        raise SystemExit(f"libxpuint8 unavailable: {L._ERR}")
    dev = torch.device("cuda", 0)
    K, W, SET = args.steps, args.warmup, args.settle
    lib = L._lib()
    st = L._stream(dev)
    if args.calibrate_copy:
        src = torch.ones(CALIB_BYTES, dtype=torch.int8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    def gbs(nbytes, ms):
        return nbytes / (ms * 1e-3) / 1e9

    def hbm_line(nbytes, ms_cold, ms_warm, graph_ms_cold=None, **more):
        d = {"ms_cold": round(ms_cold, 5), "GB/s_cold": round(gbs(nbytes, ms_cold), 1),
             "frac_hbm_peak_cold": round(gbs(nbytes, ms_cold) / PEAK_HBM_GBPS, 4),
             "ms_warm": round(ms_warm, 5), "GB/s_warm": round(gbs(nbytes, ms_warm), 1),
             "bytes": int(nbytes)}
        if graph_ms_cold is not None:
            # the same cold launches replayed from a HIP graph (no host cost)
            d["graph_ms_cold"] = round(graph_ms_cold, 5)
            d["graph_frac_hbm_peak_cold"] = round(gbs(nbytes, graph_ms_cold) / PEAK_HBM_GBPS, 4)
        d.update(more)
        return d

    def dev_gen(seed):
        return torch.Generator(device=dev).manual_seed(seed)

    def dev_act(m, k, seed):
        """activation() drawn on the device (extra buffer sets of a cold run)"""
        x = torch.randn(m, k, device=dev, generator=dev_gen(seed))
        cols = torch.randperm(k, device=dev, generator=dev_gen(seed + 7))[:max(1, round(0.01 * k))]
        x[:, cols] *= 30
        return x.to(torch.bfloat16)

    def dev_weight(n, k, seed, std=0.02):
        return (torch.randn(n, k, device=dev, generator=dev_gen(seed)) * std).to(torch.bfloat16)

    extra = {}
    # ---------------------------------------------------------- config 3
    M, Kd, N = 4096, 1280, 10240
    ops3 = 2.0 * M * N * Kd
    x = activation(torch, M, Kd).to(dev)
    w8, ws = int8.prepare_weight(weight(torch, N, Kd).to(dev))
    bias = weight(torch, 1, N, seed=2, std=0.01)[0].to(dev)
    if args.only_small:
        measure_small_batch(torch, int8, lib, L, st, dev, K, W, SET, extra, dev_act, dev_weight,
                            ops)
        print(json.dumps({"only_small": True, "steps": K, "warmup": W, "extra": extra}),
              flush=True)
        return
    if args.only_side:
        measure_side_rows(torch, int8, lib, L, st, dev, K, W, SET, extra, hbm_line, dev_gen,
                          dev_act, dev_weight, x, w8, ws, bias)
        print(json.dumps({"only_side": True, "steps": K, "warmup": W, "extra": extra}), flush=True)
        return
    # cold: distinct (x, w8, ws, bias) per call, set 0 the recipe's own inputs
    n3 = n_sets(2 * M * Kd + N * Kd + 6 * N)
    sets3 = [(x, w8, ws, bias)]
    for i in range(1, n3):
        wi8, wis = int8.prepare_weight(dev_weight(N, Kd, 100 + i))
        sets3.append((dev_act(M, Kd, 200 + i), wi8, wis, dev_weight(1, N, 300 + i, 0.01)[0]))
    log(f"[bench] config 3 linear {M}x{Kd}x{N}: {W} warm-up + {K} timed steps, "
        f"cold over {n3} input sets")
    # prepare_weight gave each weight its packed copy (the MFMA block layout,
    # read by the GEMM instead of the row-major codes; same bits): int8.linear
    # takes it, as it does for any caller of prepare_weight
    assert all(ops._packed_for(s[1]) is not None for s in sets3)
    if args.only_gemm or args.only_rowquant or args.only_c45:
        ms = ms_warm = float("nan")
    else:
        ms = timed(torch, lambda i: int8.linear(*sets3[i % n3]), K, W, SET)
        ms_warm = timed(torch, lambda i: int8.linear(x, w8, ws, bias), K, W, SET)
    value = ops3 / (ms * 1e-3) / 1e12

    # the dominant kernel alone: the GEMM with the fused epilogue, each call on
    # its own operands and output; x quantized in the MFMA block layout, as
    # the one-call linear keeps it for this shape
    ng = n_sets(M * Kd + N * Kd + 2 * M * N + 8 * N + 4 * M)
    tiled_bytes = ((M + 15) // 16) * ((Kd + 63) // 64) * 1024

    def quantize_tiled(xi, qi, si):
        rc = lib.xpuint8_convrot_quantize_tiled_stream(st, L._ptr(xi), L._ptr(qi), L._ptr(si), M, Kd)
        if rc != 0:
            raise RuntimeError(lib.xpuint8_last_error())
    gsets = []
    for i in range(ng):
        xi, wi8, wis, bi = sets3[i % n3]
        xq = torch.empty(tiled_bytes, device=dev, dtype=torch.int8)
        xs = torch.empty(M, device=dev, dtype=torch.float32)
        quantize_tiled(xi, xq, xs)
        gsets.append((xq, xs, wi8, wis, bi, torch.empty((M, N), device=dev, dtype=torch.bfloat16)))

    def gemm(i):
        xq, xs, wi8, wis, bi, out = gsets[i % ng]
        lib.xpuint8_linear_gemm_packed_stream(st, L._ptr(xq), L._ptr(xs),
                                              L._ptr(ops._packed_for(wi8)), L._ptr(wis),
                                              L._ptr(bi), 1, L._ptr(out), M, N, Kd)

    def gemm_rowmajor(i):
        xq, xs, wi8, wis, bi, out = gsets[i % ng]
        lib.xpuint8_linear_gemm_tiled_stream(st, L._ptr(xq), L._ptr(xs), L._ptr(wi8), L._ptr(wis),
                                             L._ptr(bi), 1, L._ptr(out), M, N, Kd)
    ms_gemm = ms_gemm_warm = ms_gemm_rm = float("nan")
    if not (args.only_rowquant or args.only_c45):
        ms_gemm = timed(torch, gemm, K, W, SET)
        ms_gemm_rm = timed(torch, gemm_rowmajor, K, W, SET)
    if args.only_gemm:
        print(json.dumps({"only_gemm": True, "gemm_ms_cold": round(ms_gemm, 5),
                          "TOP/s": round(ops3 / (ms_gemm * 1e-3) / 1e12, 1),
                          "gemm_rowmajor_weight_ms_cold": round(ms_gemm_rm, 5),
                          "steps": K, "warmup": W, "sets": ng}), flush=True)
        return
    if not (args.only_rowquant or args.only_c45):
        ms_gemm_warm = timed(torch, lambda i: gemm(0), K, W, SET)
    gemm_tops = ops3 / (ms_gemm * 1e-3) / 1e12
    q3 = [(torch.empty(tiled_bytes, device=dev, dtype=torch.int8),
           torch.empty(M, device=dev, dtype=torch.float32)) for _ in range(n3)]

    def quant3(i, s=st):
        xi = sets3[i % n3][0]
        qi, si = q3[i % n3]
        lib.xpuint8_convrot_quantize_tiled_stream(s, L._ptr(xi), L._ptr(qi), L._ptr(si), M, Kd)
    bytes_q3 = 3 * M * Kd + 4 * M
    ms_q3 = ms_q3_warm = ms_q3_graph = float("nan")
    if not (args.only_rowquant or args.only_c45):
        ms_q3 = timed(torch, quant3, K, W, SET)
        ms_q3_warm = timed(torch, lambda i: quant3(0), K, W, SET)
        ms_q3_graph = timed_graph(torch, quant3, K, settle_s=SET)
    log(f"[bench] step {ms:.4f} ms cold / {ms_warm:.4f} warm = {value:.1f} TOP/s; GEMM "
        f"{ms_gemm:.4f} / {ms_gemm_warm:.4f} ms = {gemm_tops:.1f} TOP/s; quantize "
        f"{ms_q3:.4f} / {ms_q3_warm:.4f} ms (graph, cold {ms_q3_graph:.4f})")
    extra["config3_step_ms_warm"] = round(ms_warm, 5)
    extra["config3_TOP/s_warm"] = round(ops3 / (ms_warm * 1e-3) / 1e12, 2)
    extra["config3_gemm"] = {"ms_cold": round(ms_gemm, 5), "ms_warm": round(ms_gemm_warm, 5),
                             "TOP/s_cold": round(gemm_tops, 1),
                             "TOP/s_warm": round(ops3 / (ms_gemm_warm * 1e-3) / 1e12, 1),
                             "weight": "packed (MFMA block layout)",
                             "rowmajor_weight_ms_cold": round(ms_gemm_rm, 5)}
    if not (args.only_rowquant or args.only_c45):
        # the same step with the weights as the reference stores them
        # (row-major codes, no packed copy: clones are new storages)
        sets3r = [(xi, wi8.clone(), wis, bi) for (xi, wi8, wis, bi) in sets3]
        ms_rm = timed(torch, lambda i: int8.linear(*sets3r[i % n3]), K, W, SET)
        extra["config3_rowmajor_weight"] = {"step_ms_cold": round(ms_rm, 5),
                                            "TOP/s_cold": round(ops3 / (ms_rm * 1e-3) / 1e12, 1)}
        del sets3r
    extra["config3_quantize"] = hbm_line(bytes_q3, ms_q3, ms_q3_warm, graph_ms_cold=ms_q3_graph)
    del gsets

    if not (args.only_main or args.only_c45):
        # ------------------------------------------------------ config 2
        # kernel throughput: the C entry points on preallocated outputs (the
        # python wrapper's own host cost, ~10 us per call, would otherwise
        # bound these ~10 us kernels); the API-level time is reported beside it
        Mr, Kr = 4096, 5120
        bytes_q = 2 * Mr * Kr + Mr * Kr + 4 * Mr
        n2 = n_sets(bytes_q)
        x2 = activation(torch, Mr, Kr).to(dev)
        sets2 = [(x2 if i == 0 else dev_act(Mr, Kr, 400 + i),
                  torch.empty((Mr, Kr), device=dev, dtype=torch.int8),
                  torch.empty(Mr, device=dev, dtype=torch.float32)) for i in range(n2)]

        def rq(i, s=st):
            xi, qi, si = sets2[i % n2]
            lib.xpuint8_convrot_quantize_stream(s, L._ptr(xi), L._ptr(qi), L._ptr(si), Mr, Kr)
        ms_q = timed(torch, rq, K, W, SET)
        if args.only_rowquant:
            print(json.dumps({"only_rowquant": True, "rotate_quant_ms_cold": round(ms_q, 5),
                              "GB/s": round(gbs(bytes_q, ms_q), 1), "steps": K, "warmup": W,
                              "sets": n2}), flush=True)
            return
        ms_q_warm = timed(torch, lambda i: rq(0), K, W, SET)
        ms_q_graph = timed_graph(torch, rq, K, settle_s=SET)
        ms_q_api = timed(torch, lambda i: int8.quantize(x2), K, W, SET)
        # the same traffic through torch's vectorized elementwise kernel (read
        # the bf16 tensor, write one byte per element: x != 0 into a bool
        # tensor), on the same cold sets: what a plain streaming kernel
        # reaches for this pattern on this box
        ne_out = [torch.empty((Mr, Kr), device=dev, dtype=torch.bool) for _ in range(n2)]
        ms_copy = timed(torch, lambda i: torch.ne(sets2[i % n2][0], 0, out=ne_out[i % n2]), K, W, SET)
        extra["config2_rotate_quant"] = hbm_line(
            bytes_q, ms_q, ms_q_warm, graph_ms_cold=ms_q_graph, api_ms_warm=round(ms_q_api, 5), sets=n2,
            streaming_ceiling_ms_cold=round(ms_copy, 5),
            streaming_ceiling_frac_hbm_peak_cold=round(gbs(3 * Mr * Kr, ms_copy) / PEAK_HBM_GBPS, 4))
        del sets2, ne_out
        bytes_p = 3 * 10240 * 1280 + 4 * 10240
        npw = n_sets(bytes_p)
        w2 = weight(torch, 10240, 1280).to(dev)
        setsp = [(w2 if i == 0 else dev_weight(10240, 1280, 500 + i),
                  torch.empty((10240, 1280), device=dev, dtype=torch.int8),
                  torch.empty(10240, device=dev, dtype=torch.float32)) for i in range(npw)]

        def pw(i, s=st):
            wi, qi, si = setsp[i % npw]
            lib.xpuint8_prepare_weight_stream(s, L._ptr(wi), L._ptr(qi), L._ptr(si), 10240, 1280)
        ms_p = timed(torch, pw, K, W, SET)
        ms_p_warm = timed(torch, lambda i: pw(0), K, W, SET)
        ms_p_graph = timed_graph(torch, pw, K, settle_s=SET)
        extra["config2_prepare_weight"] = hbm_line(bytes_p, ms_p, ms_p_warm, graph_ms_cold=ms_p_graph,
                                                   sets=npw)
        del setsp
        log(f"[bench] config 2: rotate+quant {ms_q:.4f} ms cold / {ms_q_warm:.4f} warm "
            f"(API {ms_q_api:.4f}), prepare_weight {ms_p:.4f} / {ms_p_warm:.4f} ms")
    if not (args.only_main or args.only_rowquant):
        # ------------------------------------------------------ config 4
        xf = activation(torch, 4096, 1280, seed=3).to(dev)
        up8, ups = int8.prepare_weight(weight(torch, 10240, 1280, seed=4).to(dev))
        dn8, dns = int8.prepare_weight(weight(torch, 1280, 5120, seed=5).to(dev))
        db = weight(torch, 1, 1280, seed=6, std=0.01)[0].to(dev)
        ms_f = timed(torch, lambda i: int8.ffn(xf, up8, ups, dn8, dns, db, act="geglu_erf"), K, W, SET)
        # cold: each call its own (x, up, down, bias) set, > 640 MB between reuses
        n4 = n_sets(2 * 4096 * 1280 + 10240 * 1280 + 1280 * 5120 + 2 * 4096 * 1280)
        sets4 = [(xf, up8, ups, dn8, dns, db)]
        for i in range(1, n4):
            u8, us = int8.prepare_weight(dev_weight(10240, 1280, 900 + i))
            d8, ds = int8.prepare_weight(dev_weight(1280, 5120, 950 + i))
            sets4.append((dev_act(4096, 1280, 1000 + i), u8, us, d8, ds,
                          dev_weight(1, 1280, 1050 + i, 0.01)[0]))
        ms_f_cold = timed(torch, lambda i: int8.ffn(*sets4[i % n4], act="geglu_erf"), K, W, SET)
        del sets4
        ops4 = 2.0 * 4096 * 1280 * 10240 + 2.0 * 4096 * 5120 * 1280
        extra["config4_ffn"] = {"ms_cold": round(ms_f_cold, 5),
                                "TOP/s_cold": round(ops4 / (ms_f_cold * 1e-3) / 1e12, 1),
                                "ms_warm": round(ms_f, 5),
                                "TOP/s_warm": round(ops4 / (ms_f * 1e-3) / 1e12, 1), "sets": n4}
        log(f"[bench] config 4: ffn {ms_f_cold:.4f} ms cold / {ms_f:.4f} warm")
        # ------------------------------------------------------ config 5
        w5_8, w5_s = int8.prepare_weight(weight(torch, 5120, 1280, seed=7).to(dev))
        dy = (torch.randn(4096, 5120, generator=torch.Generator().manual_seed(8)) * 1e-3
              ).to(torch.bfloat16).to(dev)
        x5 = activation(torch, 4096, 1280, seed=9).to(dev)
        ms_dx = timed(torch, lambda i: int8.linear_dx_int8(dy, w5_8, w5_s), K, W, SET)
        ms_dw = timed(torch, lambda i: int8.linear_dw(dy, x5), K, W, SET)
        w5d = int8.dequant_weight(w5_8, w5_s)
        ms_dxd = timed(torch, lambda i: int8.linear_dx(dy, w5d), K, W, SET)
        # cold: each call its own (dy, w8, w_scale, x, w) set, > 640 MB between reuses
        n5 = n_sets(2 * 4096 * 5120 + 5120 * 1280 + 2 * 4096 * 1280 + 2 * 5120 * 1280)
        sets5 = [(dy, w5_8, w5_s, x5, w5d)]
        for i in range(1, n5):
            wi8, wis = int8.prepare_weight(dev_weight(5120, 1280, 1100 + i))
            sets5.append(((torch.randn(4096, 5120, device=dev, generator=dev_gen(1150 + i)) * 1e-3)
                          .to(torch.bfloat16), wi8, wis, dev_act(4096, 1280, 1200 + i),
                          int8.dequant_weight(wi8, wis)))
        ms_dx_c = timed(torch, lambda i: int8.linear_dx_int8(*sets5[i % n5][:3]), K, W, SET)
        ms_dw_c = timed(torch, lambda i: int8.linear_dw(sets5[i % n5][0], sets5[i % n5][3]), K, W, SET)
        ms_dxd_c = timed(torch, lambda i: int8.linear_dx(sets5[i % n5][0], sets5[i % n5][4]), K, W, SET)
        del sets5
        ops5 = 2.0 * 4096 * 5120 * 1280

        def ops_line(unit, cold, warm):
            return {"ms_cold": round(cold, 5), f"{unit}_cold": round(ops5 / (cold * 1e-3) / 1e12, 1),
                    "ms_warm": round(warm, 5), f"{unit}_warm": round(ops5 / (warm * 1e-3) / 1e12, 1),
                    "sets": n5}
        extra["config5_dx_int8"] = ops_line("TOP/s", ms_dx_c, ms_dx)
        extra["config5_dw"] = ops_line("TFLOP/s", ms_dw_c, ms_dw)
        extra["config5_dx_dense"] = ops_line("TFLOP/s", ms_dxd_c, ms_dxd)
        bytes_rq = 3 * 4096 * 5120 + 4 * 4096
        nrq = n_sets(bytes_rq)
        setsr = [(dy if i == 0 else (torch.randn(4096, 5120, device=dev, generator=dev_gen(600 + i))
                                     * 1e-3).to(torch.bfloat16),
                  torch.empty((4096, 5120), device=dev, dtype=torch.int8),
                  torch.empty(4096, device=dev, dtype=torch.float32)) for i in range(nrq)]

        def qrow(i, s=st):
            di, qi, si = setsr[i % nrq]
            lib.xpuint8_quantize_row_stream(s, L._ptr(di), L._ptr(w5_s), L._ptr(qi), L._ptr(si),
                                            4096, 5120)
        ms_rq = timed(torch, qrow, K, W, SET)
        ms_rq_warm = timed(torch, lambda i: qrow(0), K, W, SET)
        ms_rq_graph = timed_graph(torch, qrow, K, settle_s=SET)
        extra["config5_quantize_row"] = hbm_line(bytes_rq, ms_rq, ms_rq_warm,
                                                 graph_ms_cold=ms_rq_graph, sets=nrq)
        del setsr
        # skinny M=16: the weight streamed once per call
        bytes_sk = 4096 * 4096 + 16 * 4096 + 2 * 16 * 4096 + 4 * 4096 + 4 * 16
        nsk = n_sets(bytes_sk)
        xs16 = activation(torch, 16, 4096, seed=10).to(dev)
        sk = [int8.prepare_weight(weight(torch, 4096, 4096, seed=11).to(dev))]
        sk += [int8.prepare_weight(dev_weight(4096, 4096, 700 + i)) for i in range(1, nsk)]
        q16, s16 = int8.quantize(xs16)
        o16 = [torch.empty((16, 4096), device=dev, dtype=torch.bfloat16) for _ in range(nsk)]
        # what linear runs on a prepared (packed) weight: q in the MFMA block
        # layout, the weight's packed copy
        q16t = torch.empty(4096 * 16, device=dev, dtype=torch.int8)
        s16t = torch.empty(16, device=dev, dtype=torch.float32)
        assert lib.xpuint8_convrot_quantize_tiled_stream(st, L._ptr(xs16), L._ptr(q16t),
                                                         L._ptr(s16t), 16, 4096) == 0
        assert torch.equal(s16t, s16)
        sk_p = [ops._packed_for(w_i) for w_i, _ in sk]
        assert all(p is not None for p in sk_p)

        def skinny(i, s=st):
            j = i % nsk
            lib.xpuint8_linear_gemm_packed_stream(s, L._ptr(q16t), L._ptr(s16t), L._ptr(sk_p[j]),
                                                  L._ptr(sk[j][1]), None, 0, L._ptr(o16[j]), 16,
                                                  4096, 4096)

        def skinny_rowmajor(i):
            w_i, s_i = sk[i % nsk]
            lib.xpuint8_linear_gemm_stream(st, L._ptr(q16), L._ptr(s16), L._ptr(w_i), L._ptr(s_i),
                                           None, 0, L._ptr(o16[i % nsk]), 16, 4096, 4096)
        skinny(0)
        o_p = o16[0].clone()
        skinny_rowmajor(0)
        assert torch.equal(o_p, o16[0]), "skinny: packed and row-major differ"
        ms_sk = timed(torch, skinny, K, W, SET)
        ms_sk_warm = timed(torch, lambda i: skinny(0), K, W, SET)
        ms_sk_kgraph = timed_graph(torch, skinny, K, settle_s=SET)
        ms_sk_rm = timed(torch, skinny_rowmajor, K, W, SET)
        ms_sk_rm_warm = timed(torch, lambda i: skinny_rowmajor(0), K, W, SET)
        ms_sk_api = timed(torch, lambda i: int8.linear(xs16, *sk[0]), K, W, SET)
        # the same API call captured once in a HIP graph and replayed: what a
        # serving loop pays per call without the Python host cost
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                int8.linear(xs16, *sk[0])
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            int8.linear(xs16, *sk[0])
        ms_sk_graph = timed(torch, lambda i: graph.replay(), K, W, SET)
        extra["config5_skinny_m16"] = hbm_line(bytes_sk, ms_sk, ms_sk_warm, graph_ms_cold=ms_sk_kgraph,
                                               sets=nsk,
                                               api_ms=round(ms_sk_api, 5),
                                               api_graph_replay_ms=round(ms_sk_graph, 5),
                                               rowmajor_ms_cold=round(ms_sk_rm, 5),
                                               rowmajor_ms_warm=round(ms_sk_rm_warm, 5))
        del sk, sk_p, graph
        log(f"[bench] config 5: dx {ms_dx_c:.4f} / {ms_dx:.4f} ms, dW {ms_dw_c:.4f} / {ms_dw:.4f} ms, "
            f"dense dx {ms_dxd_c:.4f} / {ms_dxd:.4f} ms (cold / warm), "
            f"quantize_row {ms_rq:.4f} / {ms_rq_warm:.4f} ms, skinny {ms_sk:.4f} / "
            f"{ms_sk_warm:.4f} ms (graph, cold {ms_sk_kgraph:.4f}; API {ms_sk_api:.4f}, graph replay {ms_sk_graph:.4f})")

        # ------------------------------------ accumulator consumer: rms + rope
        # q slice [1, 4096, 24, 128] of a qkv accumulator [4096, 3*3072]
        from xpu_kernels import rope
        S_r, H_r, D_r = 4096, 24, 128
        g_r = torch.Generator().manual_seed(12)
        bytes_rope = S_r * H_r * D_r * (4 + 2) + 4 * S_r + 4 * H_r * D_r
        nro = n_sets(S_r * 3 * H_r * D_r * 4)
        accs = [torch.randint(-2 ** 17, 2 ** 17, (1, S_r, 3 * H_r * D_r), generator=g_r,
                              dtype=torch.int32).to(dev)]
        accs += [torch.randint(-2 ** 17, 2 ** 17, (1, S_r, 3 * H_r * D_r), device=dev,
                               generator=dev_gen(800 + i), dtype=torch.int32) for i in range(1, nro)]
        xs_r = (torch.rand(1, S_r, generator=g_r) * 0.05).to(dev)
        ws_r = (torch.rand(H_r * D_r, generator=g_r) * 1e-4).to(dev)
        th = torch.rand(1, S_r, 1, D_r // 2, generator=g_r) * 6.28
        f_r = torch.stack([torch.stack([th.cos(), -th.sin()], -1),
                           torch.stack([th.sin(), th.cos()], -1)], -2).to(dev)
        sc_r = torch.ones(D_r, device=dev)
        qsl = [a[..., : H_r * D_r].unflatten(-1, (H_r, D_r)) for a in accs]
        ms_rope = timed(torch, lambda i: rope.rows_dq(qsl[i % nro], f_r, sc_r, 1e-6, xs_r, ws_r),
                        K, W, SET)
        ms_rope_warm = timed(torch, lambda i: rope.rows_dq(qsl[0], f_r, sc_r, 1e-6, xs_r, ws_r),
                             K, W, SET)
        extra["rms_rope_dequant_s4096_h24_d128"] = hbm_line(bytes_rope, ms_rope, ms_rope_warm,
                                                            sets=nro)
        del accs, qsl
        log(f"[bench] rms+rope dequant: {ms_rope:.4f} / {ms_rope_warm:.4f} ms")
        if args.only_c45:
            print(json.dumps({"only_c45": True, "steps": K, "warmup": W, "extra": extra}),
                  flush=True)
            return
        measure_side_rows(torch, int8, lib, L, st, dev, K, W, SET, extra, hbm_line, dev_gen,
                          dev_act, dev_weight, x, w8, ws, bias)
        measure_small_batch(torch, int8, lib, L, st, dev, K, W, SET, extra, dev_act, dev_weight,
                            ops)

    line = {
        "metric": "int8_linear TOPS (M=4096,K=1280,N=10240); rotate+quant HBM GB/s",
        "value": round(value, 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "settle_s": SET,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic (BASELINE.json config 3 recipe, torch CPU generator seed 0; "
                f"cold: {n3} input sets, > 640 MB between reuses)",
        "config": {"workload": "config 3: int8_linear forward M=4096 K=1280 N=10240 "
                               "(rotate+quantize + int8 MFMA GEMM with fused dequant+bias), "
                               "inputs cold in HBM",
                   "M": M, "K": Kd, "N": N, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "gemm_i8_pp_kernel (persistent 256x320 ping-pong, x and the "
                               "weight's packed copy in the MFMA block layout) with dequant "
                               "epilogue (2*M*N*K int ops per launch, cold operands)"},
        "extra": extra,
    }
    if not args.no_cpu:
        log(f"[bench] CPU baseline ({args.cpu_seconds:.0f} s)")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
