#!/usr/bin/env python3
"""Benchmark of the ConvRot INT8 linear path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle S] [--no-cpu]

A *step* is one ``xpu_kernels.int8.linear`` at config 3 of BASELINE.json
(x bf16 [4096,1280] with 1% outlier channels x30, W prepared from bf16
[10240,1280], bias bf16 [10240]): rotate+quantize of x, then the int8 MFMA
GEMM with the dequant+bias epilogue fused into its store.  Inputs are resident
in HBM before the timed region; W is prepared once, untimed.  An untimed run-in
of S seconds (default 0.25, so the GPU clock reaches its sustained level), W
warm-up steps, then exactly K steps between two ``torch.cuda.synchronize()`` calls, timed with
HIP events on the stream the kernels run on (torch's current stream).

``value`` is end-to-end TOP/s at config 3 (2*M*N*K = 107.37 GOP per step).
The other configurations are measured after it and reported under ``extra``.
``roofline`` is the GEMM kernel's own average duration against the dense INT8
MFMA peak; ``cpu_baseline`` times the oracle (a numpy port of the reference
chain) on a bounded row sample of config 3 on this host.  One JSON line on
stdout; progress goes to stderr.
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
    """Average ms per call of ``fn`` over ``steps`` calls (HIP events on the
    current stream, after a ``settle_s`` run-in and ``warmup`` untimed calls)."""
    settle(torch, fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def cpu_baseline(seconds):
    """The oracle's chain (rotate+quantize, int_mm, dequant) on a row sample
    of config 3, on this host's cores."""
    import numpy as np
    import oracle as O
    rng = np.random.default_rng(0)
    m, k, n = 256, 1280, 10240
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, rng.permutation(k)[:13]] *= 30
    xb = O.f32_to_bf16(x)
    w8 = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) * 0.01
    O.linear(xb, w8, ws, bias)                       # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.linear(xb, w8, ws, bias)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(2.0 * m * n * k / med / 1e12, 5),
        "unit": "TOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle.linear (numpy: Hadamard+quantize, exact float64 BLAS int_mm, "
                  f"dequant) on {m} of config 3's 4096 rows, K=1280, N=10240; median of "
                  f"{len(times)} runs ({med * 1e3:.1f} ms each)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="untimed run-in (seconds) before each measurement's warm-up, so the "
                         "GPU clock has reached its sustained level (0 = none)")
    ap.add_argument("--only-main", action="store_true", help="config 3 only (for profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run an elementwise int8 kernel over 256 MiB (reads and writes "
                         "exactly 256 MiB) so counter runs can scale FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch
    from xpu_kernels import int8
    from xpu_kernels.int8 import _lib as L
    if not int8.available():
        raise SystemExit(f"libxpuint8 unavailable: {L._ERR}")
    dev = torch.device("cuda", 0)
    K, W, SET = args.steps, args.warmup, args.settle
    if args.calibrate_copy:
        src = torch.ones(CALIB_BYTES, dtype=torch.int8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    # ---------------------------------------------------------- config 3
    M, Kd, N = 4096, 1280, 10240
    x = activation(torch, M, Kd).to(dev)
    w8, ws = int8.prepare_weight(weight(torch, N, Kd).to(dev))
    bias = weight(torch, 1, N, seed=2, std=0.01)[0].to(dev)
    ops3 = 2.0 * M * N * Kd
    log(f"[bench] config 3 linear {M}x{Kd}x{N}: {W} warm-up + {K} timed steps")
    ms = timed(torch, lambda: int8.linear(x, w8, ws, bias), K, W, SET)
    value = ops3 / (ms * 1e-3) / 1e12

    # the dominant kernel alone: the GEMM with the fused epilogue
    xq, xs = int8.quantize(x)
    out = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    lib = L._lib()

    def gemm():
        lib.xpuint8_linear_gemm_stream(L._stream(dev), L._ptr(xq), L._ptr(xs), L._ptr(w8),
                                       L._ptr(ws), L._ptr(bias), 1, L._ptr(out), M, N, Kd)
    ms_gemm = timed(torch, gemm, K, W, SET)
    gemm_tops = ops3 / (ms_gemm * 1e-3) / 1e12
    ms_q3 = timed(torch, lambda: int8.quantize(x), K, W, SET)
    log(f"[bench] step {ms:.4f} ms = {value:.1f} TOP/s; GEMM {ms_gemm:.4f} ms = "
        f"{gemm_tops:.1f} TOP/s; quantize {ms_q3:.4f} ms")

    extra = {"config3_gemm_ms": round(ms_gemm, 5), "config3_quantize_ms": round(ms_q3, 5)}
    if not args.only_main:
        # ------------------------------------------------------ config 2
        # kernel throughput: the C entry point on preallocated outputs (the
        # python wrapper's own host cost, ~10 us per call, would otherwise
        # bound these ~10 us kernels); the API-level time is reported beside it
        st = L._stream(dev)
        x2 = activation(torch, 4096, 5120).to(dev)
        q2 = torch.empty((4096, 5120), device=dev, dtype=torch.int8)
        s2 = torch.empty(4096, device=dev, dtype=torch.float32)
        ms_q = timed(torch, lambda: lib.xpuint8_convrot_quantize_stream(
            st, L._ptr(x2), L._ptr(q2), L._ptr(s2), 4096, 5120), K, W, SET)
        ms_q_api = timed(torch, lambda: int8.quantize(x2), K, W, SET)
        bytes_q = 2 * 4096 * 5120 + 4096 * 5120 + 4 * 4096
        w2 = weight(torch, 10240, 1280).to(dev)
        q2w = torch.empty((10240, 1280), device=dev, dtype=torch.int8)
        s2w = torch.empty(10240, device=dev, dtype=torch.float32)
        ms_p = timed(torch, lambda: lib.xpuint8_prepare_weight_stream(
            st, L._ptr(w2), L._ptr(q2w), L._ptr(s2w), 10240, 1280), K, W, SET)
        bytes_p = 3 * 10240 * 1280 + 4 * 10240
        extra["config2_rotate_quant"] = {
            "ms": round(ms_q, 5), "GB/s": round(bytes_q / (ms_q * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(bytes_q / (ms_q * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "api_ms": round(ms_q_api, 5)}
        extra["config2_prepare_weight"] = {
            "ms": round(ms_p, 5), "GB/s": round(bytes_p / (ms_p * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(bytes_p / (ms_p * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"[bench] config 2: rotate+quant {ms_q:.4f} ms (API {ms_q_api:.4f}), "
            f"prepare_weight {ms_p:.4f} ms")
        # ------------------------------------------------------ config 4
        xf = activation(torch, 4096, 1280, seed=3).to(dev)
        up8, ups = int8.prepare_weight(weight(torch, 10240, 1280, seed=4).to(dev))
        dn8, dns = int8.prepare_weight(weight(torch, 1280, 5120, seed=5).to(dev))
        db = weight(torch, 1, 1280, seed=6, std=0.01)[0].to(dev)
        ms_f = timed(torch, lambda: int8.ffn(xf, up8, ups, dn8, dns, db, act="geglu_erf"), K, W, SET)
        ops4 = 2.0 * 4096 * 1280 * 10240 + 2.0 * 4096 * 5120 * 1280
        extra["config4_ffn"] = {"ms": round(ms_f, 5), "TOP/s": round(ops4 / (ms_f * 1e-3) / 1e12, 1)}
        log(f"[bench] config 4: ffn {ms_f:.4f} ms")
        # ------------------------------------------------------ config 5
        w5_8, w5_s = int8.prepare_weight(weight(torch, 5120, 1280, seed=7).to(dev))
        dy = (torch.randn(4096, 5120, generator=torch.Generator().manual_seed(8)) * 1e-3
              ).to(torch.bfloat16).to(dev)
        x5 = activation(torch, 4096, 1280, seed=9).to(dev)
        ms_dx = timed(torch, lambda: int8.linear_dx_int8(dy, w5_8, w5_s), K, W, SET)
        ms_dw = timed(torch, lambda: int8.linear_dw(dy, x5), K, W, SET)
        q5 = torch.empty((4096, 5120), device=dev, dtype=torch.int8)
        s5 = torch.empty(4096, device=dev, dtype=torch.float32)
        ms_rq = timed(torch, lambda: lib.xpuint8_quantize_row_stream(
            st, L._ptr(dy), L._ptr(w5_s), L._ptr(q5), L._ptr(s5), 4096, 5120), K, W, SET)
        ops5 = 2.0 * 4096 * 5120 * 1280
        bytes_rq = 3 * 4096 * 5120 + 4 * 4096
        extra["config5_dx_int8"] = {"ms": round(ms_dx, 5), "TOP/s": round(ops5 / (ms_dx * 1e-3) / 1e12, 1)}
        extra["config5_dw"] = {"ms": round(ms_dw, 5), "TFLOP/s": round(ops5 / (ms_dw * 1e-3) / 1e12, 1)}
        extra["config5_quantize_row"] = {"ms": round(ms_rq, 5),
                                         "GB/s": round(bytes_rq / (ms_rq * 1e-3) / 1e9, 1)}
        xs16 = activation(torch, 16, 4096, seed=10).to(dev)
        sk8, sks = int8.prepare_weight(weight(torch, 4096, 4096, seed=11).to(dev))
        ms_sk_api = timed(torch, lambda: int8.linear(xs16, sk8, sks), K, W, SET)
        # the weight-streaming GEMM itself (quantized x resident, preallocated out)
        q16, s16 = int8.quantize(xs16)
        o16 = torch.empty((16, 4096), device=dev, dtype=torch.bfloat16)
        ms_sk = timed(torch, lambda: lib.xpuint8_linear_gemm_stream(
            st, L._ptr(q16), L._ptr(s16), L._ptr(sk8), L._ptr(sks), None, 0, L._ptr(o16),
            16, 4096, 4096), K, W, SET)
        bytes_sk = 4096 * 4096 + 16 * 4096 + 2 * 16 * 4096 + 4 * 4096 + 4 * 16
        extra["config5_skinny_m16"] = {
            "ms": round(ms_sk, 5), "GB/s": round(bytes_sk / (ms_sk * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(bytes_sk / (ms_sk * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "api_ms": round(ms_sk_api, 5)}
        log(f"[bench] config 5: dx {ms_dx:.4f} ms, dW {ms_dw:.4f} ms, quantize_row {ms_rq:.4f} ms, "
            f"skinny {ms_sk:.4f} ms")

        # ------------------------------------ accumulator consumer: rms + rope
        # q slice [1, 4096, 24, 128] of a qkv accumulator [4096, 3*3072]
        from xpu_kernels import rope
        S_r, H_r, D_r = 4096, 24, 128
        g_r = torch.Generator().manual_seed(12)
        acc_r = torch.randint(-2 ** 17, 2 ** 17, (1, S_r, 3 * H_r * D_r), generator=g_r,
                              dtype=torch.int32).to(dev)
        q_acc = acc_r[..., : H_r * D_r].unflatten(-1, (H_r, D_r))
        xs_r = (torch.rand(1, S_r, generator=g_r) * 0.05).to(dev)
        ws_r = (torch.rand(H_r * D_r, generator=g_r) * 1e-4).to(dev)
        th = torch.rand(1, S_r, 1, D_r // 2, generator=g_r) * 6.28
        f_r = torch.stack([torch.stack([th.cos(), -th.sin()], -1),
                           torch.stack([th.sin(), th.cos()], -1)], -2).to(dev)
        sc_r = torch.ones(D_r, device=dev)
        ms_rope = timed(torch, lambda: rope.rows_dq(q_acc, f_r, sc_r, 1e-6, xs_r, ws_r), K, W, SET)
        bytes_rope = S_r * H_r * D_r * (4 + 2) + 4 * S_r + 4 * H_r * D_r
        extra["rms_rope_dequant_s4096_h24_d128"] = {
            "ms": round(ms_rope, 5), "GB/s": round(bytes_rope / (ms_rope * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(bytes_rope / (ms_rope * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"[bench] rms+rope dequant: {ms_rope:.4f} ms")

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
        "data": "synthetic (BASELINE.json config 3 recipe, torch CPU generator seed 0)",
        "config": {"workload": "config 3: int8_linear forward M=4096 K=1280 N=10240 "
                               "(rotate+quantize + int8 MFMA GEMM with fused dequant+bias)",
                   "M": M, "K": Kd, "N": N, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "gemm_i8_pp_kernel (persistent 256x320 ping-pong) with dequant epilogue "
                               "(2*M*N*K int ops per launch)"},
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
