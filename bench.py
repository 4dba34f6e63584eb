#!/usr/bin/env python3
"""Benchmark of the MI355X BF16 transformer kernel path (one GPU).

Prints ONE JSON line. The headline workload is BASELINE config C2, RMSNorm forward+backward on
x[16384,4096] BF16 / weight F32 / eps 1e-6 (configs[1]; configs[0] is the reference's small
CPU-runnable Linear). A step is one forward plus one backward over that batch; `value` is
algorithmic HBM bytes per step / wall time per step. The BF16 GEMM (C3), RoPE (C4's Q/K), the
C1 Linear, fused attention (C4) and one decoder layer forward+backward (C5) are measured in the
same run and reported under "secondary", the kernels each with its own roofline. Inputs are synthetic, seeded and resident in
HBM before timing starts. Kernel durations come from HIP events recorded on the stream the
kernels run on (torch's current stream, which libhk.so is bound to for every call).

  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-secondary]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "rust-ascend_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "BF16 GEMM & attention TFLOP/s (% MI355X MFMA peak); RMSNorm HBM GB/s"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense BF16 MFMA
C2_ROWS, C2_WIDTH = 16384, 4096
# Algorithmic bytes (BF16 x/y/dy/dx, F32 w/rstd/dw):
C2_FWD_BYTES = 2 * C2_ROWS * C2_WIDTH * 2 + C2_WIDTH * 4 + C2_ROWS * 4           # x, y, w, rstd = 268,517,376
C2_BWD_BYTES = 3 * C2_ROWS * C2_WIDTH * 2 + 2 * C2_WIDTH * 4 + C2_ROWS * 4       # x, dy, dx, w, dw, rstd = 402,751,488


# C1/C3 GEMM workloads: name -> (M, N, K, transpose A, transpose B, label)
GEMMS = {
    "gemm8192_nt": (8192, 8192, 8192, 0, 1, "C3 8192^3 NT"),
    "gemm8192_nn": (8192, 8192, 8192, 0, 0, "C3 8192^3 NN"),
    "llama_up": (8192, 14336, 4096, 0, 1, "C3 Llama 8192x4096->14336 NT"),
    "llama_down": (8192, 4096, 14336, 0, 1, "C3 Llama 8192x14336->4096 NT"),
    "gemm4096_nt": (4096, 4096, 4096, 0, 1, "C3 4096^3 NT"),
    "gemm1024_nt": (1024, 1024, 1024, 0, 1, "C3 1024^3 NT"),
    "c1": (512, 1024, 1024, 0, 1, "C1 Linear 512x1024 by 1024x1024^T"),
}
# CPU-baseline sample rows per GEMM workload (None: the whole product)
CPU_ROWS = {"gemm8192_nt": 256, "gemm8192_nn": 16, "llama_up": 256, "llama_down": 256}
KERNELS = sorted(list(GEMMS) + ["c2", "attn_fwd", "attn_bwd", "rope", "c5"])


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-secondary", action="store_true", help="headline workload only")
    p.add_argument("--copy-calibration", action="store_true",
                   help="also run a 1 GiB device copy (for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    p.add_argument("--only-c5", action="store_true",
                   help="only run the C5 decoder layer (forward + backward, --warmup and --steps) and print its line")
    p.add_argument("--only-widened", action="store_true",
                   help="only run the lines of the rows widened around the path (grouped and padded GEMM, "
                        "softmax, cross entropy, SwiGLU, bias add, embedding) and print them, one JSON line each")
    p.add_argument("--kernel", choices=sorted(KERNELS),
                   help="only run one workload's kernels --steps times (after --warmup) and print its timing: "
                        "the unit that rocprofv3 profiles")
    p.add_argument("--vendor", action="store_true",
                   help="only time the vendor libraries on the same data (hipBLASLt through torch.matmul for C1/C3, "
                        "PyTorch SDPA for C4) next to this library and print one JSON line each")
    p.add_argument("--stream-ceilings", action="store_true",
                   help="only measure plain HBM streams (read, write, copy, 2 reads + 1 write) on 1 GiB "
                        "buffers with PyTorch's kernels and print them")
    return p.parse_args()


def stream_ceilings(gib=1, iters=10):
    """Plain HBM streaming rates on buffers far larger than the 256 MB on-package cache, with
    PyTorch's own kernels: sum (read), fill_ (write), copy_ (read + write), add (2 reads + 1
    write). They bound what an HBM-bound kernel with the same stream mix can reach here."""
    import torch
    n = gib * (1 << 30) // 4
    a = torch.ones(n, device="cuda")
    b = torch.ones(n, device="cuda")
    c = torch.empty(n, device="cuda")
    cases = [("read", 1, lambda: a.sum()), ("write", 1, lambda: c.fill_(1.0)),
             ("copy", 2, lambda: c.copy_(a)), ("2 reads + 1 write", 3, lambda: torch.add(a, b, out=c))]
    out = {}
    for name, streams, fn in cases:
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / iters
        out[name] = round(streams * n * 4 / (ms * 1e-3) / 1e9, 1)
    return out


def copy_calibration():
    """A 1 GiB device-to-device copy (reads 1 GiB, writes 1 GiB): the known-size launch against
    which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()


def warm(fn, seconds=0.3):
    """Run fn until `seconds` of wall time have passed: the GPU leaves its idle clocks only after
    sustained load, and a first timed launch otherwise measures the ramp (the first 8192^3 GEMM
    of a process measured ~15% slower after a 3-launch warmup than after this one)."""
    import torch
    t0 = time.perf_counter()
    while True:
        fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def event_ms(pairs):
    import torch
    torch.cuda.synchronize()
    vals = [a.elapsed_time(b) for a, b in pairs]
    return sum(vals) / len(vals)


def read_traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE and WRITE_SIZE, scaled by
    the same counters on a copy of known size), kept in profiles/hbm_traffic.txt as
    `<kernel> <bytes>` lines; None when not measured."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) == 2 and parts[0] == kernel:
            return int(float(parts[1]))
    return None


def read_counters(key: str):
    """Per-launch counters of an MFMA-bound workload from profiles/kernel_counters.txt
    (`<key> <traffic bytes> <MFMA utilisation> <executed flops>`), or None."""
    path = os.path.join(ROOT, "profiles", "kernel_counters.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) == 4 and parts[0] == key:
            return {"traffic": int(float(parts[1])), "mfma_util": float(parts[2]), "executed_flops": float(parts[3])}
    return None


def roofline(bound, algo, ms, kernel, key=None):
    if bound == "hbm":
        achieved = algo / (ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        achieved = algo / (ms * 1e-3) / 1e12
        peak, unit = BF16_PEAK_TFLOPS, "TFLOP/s"
    out = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": read_traffic(kernel), "kernel": kernel,
           "algorithmic_per_launch": algo, "avg_launch_ms": round(ms, 5)}
    counters = read_counters(key) if key else None
    if counters:  # measured per-launch traffic; for MFMA-bound workloads utilisation and executed work
        out["traffic"] = counters["traffic"]
        if bound == "mfma":
            out["mfma_util"] = counters["mfma_util"]
            out["executed_flops_per_launch"] = counters["executed_flops"]
    return out


def short_roofline(rl, kernel=True):
    """The roofline of a secondary line without what the line already states (value = achieved,
    ms = the average launch, unit and peak implied by the line's unit): the fraction of peak, the
    counter-measured HBM traffic per launch in MB, MFMA utilisation where measured."""
    out = {"kernel": rl["kernel"]} if kernel else {}
    out["frac"] = rl["frac"]
    out["traffic_MB"] = None if rl.get("traffic") is None else round(rl["traffic"] / 1e6)
    if "mfma_util" in rl:
        out["mfma_util"] = rl["mfma_util"]
    return out


def short_cpu(cpu):
    """A secondary line's CPU baseline without the unit it shares with the line."""
    return {k: cpu[k] for k in ("value", "cores", "kind", "sample")}


def bench_c2(steps, warmup):
    import ctypes
    import torch
    from rust_ascend_hip import HipRuntime, _lib, runtime
    from rust_ascend_hip._lib import check
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    x = torch.randn((C2_ROWS, C2_WIDTH), generator=g, device="cuda").to(torch.bfloat16)
    dy = torch.randn((C2_ROWS, C2_WIDTH), generator=g, device="cuda").to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn((C2_WIDTH,), generator=g, device="cuda")).float()
    y, rstd = HipRuntime.rms_norm(x, w, 1e-6)
    dx, dw = HipRuntime.rms_norm_backward(x, w, dy, rstd)
    # The step calls the C ABI directly with caller-owned outputs and descriptors built once, as
    # a native caller of hk_rms_norm / hk_rms_norm_backward would: the per-call Python
    # allocation and descriptor building of the HipRuntime mirror would otherwise leave the
    # GPU idle between the kernels.
    lib, ctx = _lib.load(), runtime._context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    d_x, d_w, d_dy = runtime.desc(x), runtime.desc(w), runtime.desc(dy)
    d_y, d_rstd, d_dx, d_dw = runtime.desc(y), runtime.desc(rstd), runtime.desc(dx), runtime.desc(dw)
    eps = ctypes.c_double(1e-6)

    def fwd():
        check(lib.hk_rms_norm(ctx, d_x, d_w, eps, d_y, d_rstd))

    def bwd():
        check(lib.hk_rms_norm_backward(ctx, d_x, d_w, d_dy, d_rstd, d_dx, d_dw))

    for _ in range(warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fwd()
        bwd()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    # The per-op split: each op alone, back to back, between one pair of events (its average
    # launch duration, launch gaps included). An event recorded between the two ops of every step
    # costs the GPU several microseconds of its own (~12 us per 123 us step), so the step loop above
    # has none. In the step the backward runs a few microseconds faster than alone: the forward
    # has just read x, and part of it is still in the on-package cache.
    split = []
    for op in (fwd, bwd):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            op()
        e1.record()
        torch.cuda.synchronize()
        split.append(e0.elapsed_time(e1) / steps)
    return wall_ms, split[0], split[1]


def cpu_baseline_c2(threads):
    """The oracle's restatement of the reference's FP32 row programs (row_programs.rs:144-151,
    200-217 plus the pairwise column sum of normalization.rs:95-114), timed on the host."""
    import numpy as np
    import oracle
    oracle.set_threads(threads)
    rng = np.random.default_rng(0)
    x = oracle.bf16_round(rng.standard_normal((C2_ROWS, C2_WIDTH), dtype=np.float32))
    dy = oracle.bf16_round(rng.standard_normal((C2_ROWS, C2_WIDTH), dtype=np.float32))
    w = (1 + 0.1 * rng.standard_normal(C2_WIDTH)).astype(np.float32)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        _, rstd = oracle.rms_norm_lanes_f32(x, w, 1e-6)
        oracle.rms_norm_backward_lanes_f32(x, w, dy, rstd)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    return {"value": round((C2_FWD_BYTES + C2_BWD_BYTES) / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "seconds_per_step": round(t, 3),
            "sample": "whole C2 step, FP32 row-program order on BF16-valued inputs, median of 3"}


def cpu_threads():
    """Host threads of the CPU baselines: OMP_NUM_THREADS (16 on the GPU box, its CPU share for
    one GPU), else the visible cores."""
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def cpu_baseline_gemm(m, n, k, ta, tb, rows=None):
    """The oracle's restatement of the reference's host GEMM (deepgemm_validate.rs:19-21: f32
    products summed over k in order, no FMA) on BF16-valued inputs of the workload's shape. With
    `rows`, only that many output rows are computed (the rate is theirs; `seconds` projects it to
    the full M)."""
    import numpy as np
    import oracle
    threads = cpu_threads()
    oracle.set_threads(threads)
    rng = np.random.default_rng(m + n + k)
    mr = rows or m
    a = oracle.bf16_round(rng.standard_normal((k, mr) if ta else (mr, k), dtype=np.float32) / np.float32(k ** 0.5))
    b = oracle.bf16_round(rng.standard_normal((n, k) if tb else (k, n), dtype=np.float32) / np.float32(k ** 0.5))
    reps = 3 if mr * n * k <= (1 << 31) else 1
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle.gemm_f32(a, b, ta, tb)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    return {"value": round(2 * mr * n * k / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": ("all rows" if mr == m else f"{mr}/{m} rows") + (", median of 3" if reps == 3 else "")}


def cpu_baseline_attention():
    """The oracle's restatement of the reference's host attention (grouped_attention_tensor.rs:
    14-44, f64 with its BF16 rounding points), forward and backward, on a sample of C4: batch 0,
    all 32 query / 8 KV heads, the first 1024 positions (1/64 of the causal work; the oracle is
    parallel over the 8 (batch, KV head) pairs). The rate is the sample's causal-useful flops over
    its time; `seconds` projects it to the whole config."""
    import numpy as np
    import oracle
    threads = cpu_threads()
    oracle.set_threads(threads)
    rng = np.random.default_rng(4)
    S, D = 1024, 128
    q, do = (oracle.bf16_round(rng.standard_normal((1, 32, S, D), dtype=np.float32)) for _ in range(2))
    k, v = (oracle.bf16_round(rng.standard_normal((1, 8, S, D), dtype=np.float32)) for _ in range(2))
    t0 = time.perf_counter()
    oracle.attention_f64(q, k, v, do, scale=D ** -0.5, causal=True)
    t = time.perf_counter() - t0
    flops = 3.5 * 2 * 32 * S * S * D  # forward + backward, causal-useful (the GPU lines' count)
    return {"value": round(flops / t / 1e12, 6), "unit": "TFLOP/s", "cores": min(threads, 8), "kind": "port",
            "sample": "batch 0, positions < 1024 (1/64 of the work)"}


def bench_gemm(m, n, k, ta, tb, iters=10, warmup=3, out=None):
    """Average GPU time of one GEMM over `iters` back-to-back calls of the C ABI (descriptors
    built once, as a native caller's would be), between one pair of events on the stream the
    kernels run on. Timing each call with its own event pair around the Python-level call would
    add the host's per-call work to small GEMMs (C1's 7 us kernel measured 16.6 us that way)."""
    import ctypes
    import torch
    from rust_ascend_hip import HipRuntime, Transpose, _lib, runtime
    from rust_ascend_hip._lib import check
    out = out or torch.bfloat16
    g = torch.Generator(device="cuda")
    g.manual_seed(m + n + k)
    a = (torch.randn((k, m) if ta else (m, k), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
    b = (torch.randn((n, k) if tb else (k, n), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
    c = torch.empty((m, n), device="cuda", dtype=out)
    for _ in range(warmup):
        HipRuntime.gemm_into(a, b, Transpose(ta), Transpose(tb), c)
    lib, ctx = _lib.load(), runtime._context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    d_a, d_b, d_c = runtime.desc(a), runtime.desc(b), runtime.desc(c)

    def call():
        check(lib.hk_gemm_into(ctx, d_a, d_b, int(ta), int(tb), d_c))

    warm(call)
    reps = max(iters, int(2e-3 / max(2 * m * n * k / 1.5e15, 1e-6)))  # >= ~2 ms of work
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        call()
    e1.record()
    return event_ms([(e0, e1)]) / reps


def run_kernel(name, steps, warmup):
    """One workload's kernels only, `warmup` then `steps` back-to-back calls through the C ABI
    with descriptors built once, timed by HIP events on the kernels' stream: the unit that
    rocprofv3 --pmc / --kernel-trace profiles (bench.py --kernel NAME)."""
    import ctypes
    import torch
    from rust_ascend_hip import HipRuntime, _lib, runtime
    from rust_ascend_hip._lib import check
    lib, ctx = _lib.load(), runtime._context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    if name in GEMMS:
        m, n, k, ta, tb, _ = GEMMS[name]
        a = (torch.randn((k, m) if ta else (m, k), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
        b = (torch.randn((n, k) if tb else (k, n), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
        c = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        d = (runtime.desc(a), runtime.desc(b), runtime.desc(c))
        calls = [lambda: check(lib.hk_gemm_into(ctx, d[0], d[1], int(ta), int(tb), d[2]))]
    elif name == "c2":
        x = torch.randn((C2_ROWS, C2_WIDTH), generator=g, device="cuda").to(torch.bfloat16)
        dy = torch.randn((C2_ROWS, C2_WIDTH), generator=g, device="cuda").to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn((C2_WIDTH,), generator=g, device="cuda")).float()
        y, rstd = HipRuntime.rms_norm(x, w, 1e-6)
        dx, dw = HipRuntime.rms_norm_backward(x, w, dy, rstd)
        d = [runtime.desc(t) for t in (x, w, dy, y, rstd, dx, dw)]
        eps = ctypes.c_double(1e-6)
        calls = [lambda: check(lib.hk_rms_norm(ctx, d[0], d[1], eps, d[3], d[4])),
                 lambda: check(lib.hk_rms_norm_backward(ctx, d[0], d[1], d[2], d[4], d[5], d[6]))]
    elif name in ("attn_fwd", "attn_bwd"):
        B, H, HKV, S, D = 4, 32, 8, 4096, 128
        q = torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16)
        k = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(torch.bfloat16)
        do = torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16)
        o, lse = HipRuntime.attention_forward(q, k, v, D ** -0.5, True)
        grads = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)]
        dq, dk, dv = (runtime.desc(t) for t in grads)
        dqkv = (runtime.desc(q), runtime.desc(k), runtime.desc(v), runtime.desc(o), runtime.desc(lse), runtime.desc(do))
        sc, z = ctypes.c_float(D ** -0.5), ctypes.c_uint64(0)
        if name == "attn_fwd":
            calls = [lambda: check(lib.hk_attention_forward(ctx, dqkv[0], dqkv[1], dqkv[2], sc, 1, z, z, dqkv[3],
                                                            dqkv[4]))]
        else:
            calls = [lambda: check(lib.hk_attention_backward(ctx, *dqkv, sc, 1, z, z, dq, dk, dv))]
    elif name == "c5":  # one decoder-layer step (forward + backward), as bench_decoder builds it
        from rust_ascend_hip import DecoderConfig, DecoderLayer
        cfg = DecoderConfig()
        layer = DecoderLayer(cfg, seed=5)
        layer.ids.copy_(torch.randint(0, cfg.vocab, (cfg.batch, cfg.seq), generator=g, device="cuda"))
        layer.dy.copy_(torch.randn(layer.dy.shape, generator=g, device="cuda").to(torch.bfloat16))
        calls = [layer.step]
    else:  # rope
        import numpy as np
        pos = np.arange(4096, dtype=np.float64)[:, None]
        ang = pos * (5e5 ** (-np.arange(0, 128, 2) / 128))[None, :]
        cos = torch.from_numpy(np.cos(ang).astype(np.float32)).cuda()[None, None]
        sin = torch.from_numpy(np.sin(ang).astype(np.float32)).cuda()[None, None]
        q = torch.randn((4, 32, 4096, 128), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty_like(q)
        d = (runtime.desc(q), runtime.desc(cos), runtime.desc(sin), runtime.desc(y))
        calls = [lambda: check(lib.hk_rotary_prefix(ctx, d[0], d[1], d[2], 128, 1, d[3]))]
    for _ in range(warmup):
        for c in calls:
            c()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        for c in calls:
            c()
    e1.record()
    torch.cuda.synchronize()
    return {"kernel": name, "steps": steps, "ms_per_step": round(e0.elapsed_time(e1) / max(steps, 1), 5)}


def bench_vendor():
    """The vendor libraries on the same shapes and data layout: hipBLASLt through torch.matmul
    for C1/C3 (the weight stored [N,K] and read transposed for NT), PyTorch's scaled_dot_product_
    attention for C4 (its K/V heads expanded to 32, which does not change its flop count). One
    JSON line per workload with both rates. Evidence for where the kernels stand, not the metric."""
    import torch
    import torch.nn.functional as F
    lines = []
    for key in ("gemm8192_nt", "gemm8192_nn", "llama_up", "llama_down", "gemm4096_nt", "gemm1024_nt", "c1"):
        m, n, k, ta, tb, label = GEMMS[key]
        g = torch.Generator(device="cuda")
        g.manual_seed(m + n + k)
        a = (torch.randn((m, k), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
        b = (torch.randn((n, k) if tb else (k, n), generator=g, device="cuda") / k ** 0.5).to(torch.bfloat16)
        bt = b.t() if tb else b
        vendor_ms = time_gpu(lambda: torch.matmul(a, bt), iters=max(10, int(2e-3 / (2 * m * n * k / 1.5e15))))
        ours_ms = bench_gemm(m, n, k, ta, tb)
        fl = 2 * m * n * k
        lines.append({"workload": label, "unit": "TFLOP/s", "hk": round(fl / ours_ms / 1e9, 1),
                      "hipblaslt_torch_matmul": round(fl / vendor_ms / 1e9, 1), "hk_ms": round(ours_ms, 5),
                      "vendor_ms": round(vendor_ms, 5)})
    B, H, HKV, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    q = torch.randn((B, H, S, D), generator=g, device="cuda", dtype=torch.bfloat16)
    k = torch.randn((B, HKV, S, D), generator=g, device="cuda", dtype=torch.bfloat16)
    v = torch.randn((B, HKV, S, D), generator=g, device="cuda", dtype=torch.bfloat16)
    kk = k.repeat_interleave(H // HKV, 1).contiguous()
    vv = v.repeat_interleave(H // HKV, 1).contiguous()
    f_ms, b_ms, ff, bf = bench_attention()
    entry = {"workload": "C4 causal GQA attention B4 S4096 Hq32 Hkv8 D128", "unit": "TFLOP/s",
             "hk_fwd": round(ff / f_ms / 1e9, 1), "hk_bwd": round(bf / b_ms / 1e9, 1)}
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for backend, tag in ((SDPBackend.FLASH_ATTENTION, "flash"), (SDPBackend.EFFICIENT_ATTENTION, "efficient")):
        try:
            with sdpa_kernel(backend):
                qg, kg, vg = (t.clone().requires_grad_() for t in (q, kk, vv))
                fwd = lambda: F.scaled_dot_product_attention(qg, kg, vg, is_causal=True)
                fms = time_gpu(fwd, iters=5)
                out = fwd()
                go = torch.randn_like(out)
                bms = time_gpu(lambda: torch.autograd.grad(out, (qg, kg, vg), go, retain_graph=True), iters=5)
            entry[f"sdpa_{tag}_fwd"] = round(ff / fms / 1e9, 1)
            entry[f"sdpa_{tag}_bwd"] = round(bf / bms / 1e9, 1)
        except Exception as exc:  # a backend this build lacks is reported, not replaced
            entry[f"sdpa_{tag}"] = f"unavailable: {str(exc)[:80]}"
    lines.append(entry)
    return lines


def gemm_kernel_name(m, n, k, ta, tb):
    """The kernel libhk.so runs for this shape (hk_gemm.hip's selection on 256 CUs)."""
    if ((m + 255) // 256) * ((n + 255) // 256) >= 256 and k % 64 == 0:
        return "gemm_nt_m16_kernel"
    return "gemm_nt_dma_kernel"


def c4_tables(S=4096, D=128, theta=5e5):
    """C4's RoPE tables [1, 1, S, D/2] F32: angle = position * theta^(-2i/D), in float64."""
    import numpy as np
    pos = np.arange(S, dtype=np.float64)[:, None]
    ang = pos * (theta ** (-np.arange(0, D, 2) / D))[None, :]
    return (np.cos(ang).astype(np.float32)[None, None], np.sin(ang).astype(np.float32)[None, None])


def bench_rope(iters=10):
    """C4's RoPE: split-half rotation of Q [4,32,4096,128] and K [4,8,4096,128] (two calls of the
    C ABI per step, descriptors built once)."""
    import ctypes
    import torch
    from rust_ascend_hip import _lib, runtime
    from rust_ascend_hip._lib import check
    cos, sin = (torch.from_numpy(t).cuda() for t in c4_tables())
    q = torch.randn((4, 32, 4096, 128), device="cuda").to(torch.bfloat16)
    k = torch.randn((4, 8, 4096, 128), device="cuda").to(torch.bfloat16)
    yq, yk = torch.empty_like(q), torch.empty_like(k)
    lib, ctx = _lib.load(), runtime._context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    d = [runtime.desc(t) for t in (q, k, cos, sin, yq, yk)]

    def step():
        check(lib.hk_rotary_prefix(ctx, d[0], d[2], d[3], 128, 1, d[4]))
        check(lib.hk_rotary_prefix(ctx, d[1], d[2], d[3], 128, 1, d[5]))
    # back-to-back steps between one pair of events (an event between every two calls costs the
    # GPU time of its own)
    ms = time_gpu(step, iters)
    algo = 2 * (q.numel() + k.numel()) * 2 + 2 * 2 * cos.numel() * 4
    return ms, algo


def cpu_baseline_rope():
    """The oracle's restatement of the reference's rotary program (rotary_programs.rs:47-97,
    101-156) on batch 0 of C4's Q and K (a quarter of the work), timed on the host."""
    import numpy as np
    import oracle
    threads = cpu_threads()
    oracle.set_threads(threads)
    rng = np.random.default_rng(6)
    cos, sin = c4_tables()
    q = oracle.bf16_round(rng.standard_normal((1, 32, 4096, 128), dtype=np.float32))
    k = oracle.bf16_round(rng.standard_normal((1, 8, 4096, 128), dtype=np.float32))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.rotary_prefix(q, cos, sin, 128, 1)
        oracle.rotary_prefix(k, cos, sin, 128, 1)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    algo = 2 * (q.size + k.size) * 2
    return {"value": round(algo / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": "batch 0 (1/4), median of 3"}


def bench_c4_step(iters=3):
    """BASELINE C4 as one step: RoPE (split-half, theta 5e5) on Q and K, the causal GQA attention
    forward and backward on the rotated Q/K, and the RoPE backward of dQ and dK (BF16 gradients),
    eight C-ABI calls with descriptors built once. Returns (step ms, attention flops per step)."""
    import ctypes
    import torch
    from rust_ascend_hip import _lib, runtime
    from rust_ascend_hip._lib import check
    B, H, HKV, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    bf = torch.bfloat16
    q = torch.randn((B, H, S, D), generator=g, device="cuda").to(bf)
    k = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(bf)
    v = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(bf)
    do = torch.randn((B, H, S, D), generator=g, device="cuda").to(bf)
    cos, sin = (torch.from_numpy(t).cuda() for t in c4_tables(S, D))
    qr, kr, o, dq, dk, dv, dq0, dk0 = (torch.empty_like(t) for t in (q, k, q, q, k, v, q, k))
    lse = torch.empty((B, H, S), device="cuda")
    lib, ctx = _lib.load(), runtime._context()
    check(lib.hk_set_stream(ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    t = {n: runtime.desc(x) for n, x in dict(q=q, k=k, v=v, do=do, cos=cos, sin=sin, qr=qr, kr=kr, o=o, lse=lse,
                                              dq=dq, dk=dk, dv=dv, dq0=dq0, dk0=dk0).items()}
    sc, z = ctypes.c_float(D ** -0.5), ctypes.c_uint64(0)

    def step():
        check(lib.hk_rotary_prefix(ctx, t["q"], t["cos"], t["sin"], D, 1, t["qr"]))
        check(lib.hk_rotary_prefix(ctx, t["k"], t["cos"], t["sin"], D, 1, t["kr"]))
        check(lib.hk_attention_forward(ctx, t["qr"], t["kr"], t["v"], sc, 1, z, z, t["o"], t["lse"]))
        check(lib.hk_attention_backward(ctx, t["qr"], t["kr"], t["v"], t["o"], t["lse"], t["do"], sc, 1, z, z,
                                        t["dq"], t["dk"], t["dv"]))
        check(lib.hk_rotary_prefix_backward(ctx, t["dq"], t["cos"], t["sin"], D, 1, t["dq0"]))
        check(lib.hk_rotary_prefix_backward(ctx, t["dk"], t["cos"], t["sin"], D, 1, t["dk0"]))
    ms = time_gpu(step, iters)
    return ms, 3.5 * 2 * B * H * S * S * D


def bench_attention(iters=5):
    import torch
    from rust_ascend_hip import HipRuntime
    B, H, HKV, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    q = torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, HKV, S, D), generator=g, device="cuda").to(torch.bfloat16)
    do = torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16)
    scale = D ** -0.5
    o, lse = HipRuntime.attention_forward(q, k, v, scale, True)
    warm(lambda: HipRuntime.attention_backward(q, k, v, o, lse, do, scale, True, grad_dtype=torch.bfloat16))
    fw, bw = [], []
    for _ in range(iters):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        HipRuntime.attention_forward(q, k, v, scale, True)
        e[1].record()
        HipRuntime.attention_backward(q, k, v, o, lse, do, scale, True, grad_dtype=torch.bfloat16)
        e[2].record()
        fw.append((e[0], e[1]))
        bw.append((e[1], e[2]))
    fwd_flops = 2 * B * H * S * S * D  # causal-useful (FlashAttention convention): 4*B*H*S^2*D/2
    return event_ms(fw), event_ms(bw), fwd_flops, 2.5 * fwd_flops


def time_gpu(fn, iters=10):
    """Average HIP-event time (ms) of fn() over iters back-to-back launches after a warm-up."""
    import torch
    warm(fn)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def bench_widened():
    """One line per widened row next to the path (M-grouped and padded GEMM, softmax rows, cross
    entropy, SwiGLU, bias/residual add, embedding), each at a Llama-sized shape with seeded data:
    TFLOP/s against the BF16 MFMA peak for the GEMMs, algorithmic HBM bytes against 8 TB/s for
    the row and elementwise kernels (every tensor read once and written once)."""
    import torch
    from rust_ascend_hip import HipRuntime, LossReduction
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    out = []

    def add(name, ms, bound, algo, kernel, unit, key):
        val = algo / ms / 1e9 if unit == "TFLOP/s" else algo / ms / 1e6
        out.append({"workload": name, "value": round(val, 1), "unit": unit, "ms": round(ms, 4),
                    "roofline": short_roofline(roofline(bound, algo, ms, kernel, key), kernel=False)})

    def guarded(name, fn):
        try:
            fn()
        except Exception as exc:  # reported, never silently replaced by another path
            out.append({"workload": name, "error": str(exc)[:200]})

    def grouped():
        E, rows, K, N = 8, 1024, 4096, 14336
        a = torch.randn((E * rows, K), generator=g, device="cuda").to(torch.bfloat16)
        w = torch.randn((E, N, K), generator=g, device="cuda").to(torch.bfloat16)
        ends = HipRuntime.upload_group_ends([rows * (i + 1) for i in range(E)])
        y = HipRuntime.grouped_nt(a, w, ends)
        ms = time_gpu(lambda: HipRuntime.grouped_nt_into(a, w, ends, y))
        add(f"(f) MoE grouped NT GEMM {E}x{rows} rows, K {K}, N {N}", ms, "mfma",
            2 * E * rows * N * K, "gemm_nt_m16_kernel", "TFLOP/s", "grouped")
    guarded("(f) M-grouped NT GEMM", grouped)

    def padded():
        M = N = K = 4000
        a = torch.randn((M, K), generator=g, device="cuda")
        b = torch.randn((K, N), generator=g, device="cuda")
        ms = time_gpu(lambda: HipRuntime.gemm_padded_bf16_fp32(a, b))
        add(f"(f) padded GEMM F32 {M}^3 (pad+GEMM+crop)", ms, "mfma", 2 * M * N * K,
            "pad_bf16+gemm+crop_f32", "TFLOP/s", "padded")
    guarded("(f) padded GEMM", padded)

    R, C = 8192, 32000
    x = torch.randn((R, C), generator=g, device="cuda")

    def softmax():
        y = HipRuntime.softmax(x)
        ms = time_gpu(lambda: HipRuntime.softmax(x))
        add(f"(f) softmax F32 [{R},{C}]", ms, "hbm", 2 * 4 * R * C, "softmax", "GB/s", "softmax")
        dy = torch.randn((R, C), generator=g, device="cuda")
        ms = time_gpu(lambda: HipRuntime.softmax_backward(y, dy))
        add(f"(f) softmax bwd F32 [{R},{C}]", ms, "hbm", 3 * 4 * R * C, "softmax_backward", "GB/s",
            "softmax_bwd")
    guarded("(f) softmax rows", softmax)

    def cross_entropy():
        labels = torch.randint(0, C, (R,), generator=g, device="cuda", dtype=torch.int64)
        wt = torch.ones((C,), device="cuda")

        def ce():
            lp = HipRuntime.log_softmax(x)
            return HipRuntime.nll_loss(lp, labels, wt, LossReduction.Mean)
        ms = time_gpu(ce)
        add(f"(f) cross entropy F32 [{R},{C}]", ms, "hbm",
            2 * 4 * R * C + 8 * R + 4 * C, "softmax+nll_loss", "GB/s", "cross_entropy")
    guarded("(f) cross entropy", cross_entropy)

    def swiglu():
        T, F = 4096, 14336
        gate = torch.randn((T, F), generator=g, device="cuda").to(torch.bfloat16)
        up = torch.randn((T, F), generator=g, device="cuda").to(torch.bfloat16)
        ms = time_gpu(lambda: HipRuntime.silu_mul(gate, up))
        add(f"(f) silu_mul BF16 [{T},{F}]", ms, "hbm", 3 * 2 * T * F, "silu_mul_kernel", "GB/s", "silu_mul")
        gr = torch.randn((T, F), generator=g, device="cuda").to(torch.bfloat16)
        ms = time_gpu(lambda: HipRuntime.silu_mul_backward(gate, up, gr))
        add(f"(f) silu_mul bwd BF16 [{T},{F}]", ms, "hbm", 5 * 2 * T * F, "silu_mul_bwd_kernel", "GB/s",
            "silu_mul_bwd")
    guarded("(f) SwiGLU", swiglu)

    def bias():
        T, H = 4096, 4096
        xb = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
        res = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
        bb = torch.randn((H,), generator=g, device="cuda")
        ms = time_gpu(lambda: HipRuntime.bias_add(xb, bb, res))
        add(f"(f) bias+residual add BF16 [{T},{H}]", ms, "hbm", 3 * 2 * T * H + 4 * H, "bias_add_kernel",
            "GB/s", "bias_add")
    guarded("(f) bias add", bias)

    def embedding():
        V, H, T = 32000, 4096, 4096
        table = torch.randn((V, H), generator=g, device="cuda").to(torch.bfloat16)
        ids = torch.randint(0, V, (T,), generator=g, device="cuda", dtype=torch.int64)
        ms = time_gpu(lambda: HipRuntime.embedding(table, ids))
        add(f"(f) embedding gather [{V},{H}] BF16, {T} IDs", ms, "hbm", 2 * 2 * T * H + 8 * T,
            "embedding_gather_kernel", "GB/s", "embedding")
    guarded("(f) embedding", embedding)
    return out


def bench_decoder(steps=5, warmup=2):
    """C5: one Llama-style decoder layer forward + backward (hidden 4096, 32/8 heads, SwiGLU 14336,
    batch 2 x seq 2048, token IDs uniform in [0, 32000), N(0, 0.02) BF16 weights)."""
    import torch
    from rust_ascend_hip import DecoderConfig, DecoderLayer
    cfg = DecoderConfig()
    layer = DecoderLayer(cfg, seed=5)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    layer.ids.copy_(torch.randint(0, cfg.vocab, (cfg.batch, cfg.seq), generator=g, device="cuda"))
    layer.dy.copy_(torch.randn(layer.dy.shape, generator=g, device="cuda").to(torch.bfloat16))
    for _ in range(warmup):
        layer.step()
    warm(layer.step)
    fw, bw = [], []
    for _ in range(steps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        layer._run(layer._forward)
        e[1].record()
        layer._run(layer._backward)
        e[2].record()
        fw.append((e[0], e[1]))
        bw.append((e[1], e[2]))
    return cfg, event_ms(fw), event_ms(bw)


def cpu_baseline_decoder(tokens=32):
    """The C5 layer forward + backward composed from the oracle's restatements of the reference's
    host loops (embedding, the FP32 row programs of RMSNorm, the f32 sequential-k GEMM, the
    rotary program, the f64 attention with BF16 rounding points, SiLU-mul, the dense embedding
    gradient) on one sequence of `tokens` positions with C5's widths and N(0, 0.02) weights,
    timed on the host. The rate is tokens per second of that sample (the layer's cost is nearly
    linear in tokens: 96 % of its flops are the projections)."""
    import numpy as np
    import oracle
    from rust_ascend_hip import DecoderConfig
    threads = cpu_threads()
    oracle.set_threads(threads)
    c = DecoderConfig()
    T, Hd, F, D, hq, hkv = tokens, c.hidden, c.ffn, c.head_dim, c.heads, c.kv_heads
    W = (hq + 2 * hkv) * D
    rng = np.random.default_rng(5)

    block = oracle.bf16_round(rng.standard_normal(1 << 20, dtype=np.float32) * np.float32(c.init_std))

    def init(*shape):  # N(0, 0.02) BF16 values, a 1M-value block repeated (the timing does not depend on them)
        return np.resize(block, shape)
    table, wqkv, wo = init(c.vocab, Hd), init(W, Hd), init(Hd, Hd)
    wg, wu, wd = init(F, Hd), init(F, Hd), init(Hd, F)
    w1 = w2 = np.ones(Hd, np.float32)
    ids = rng.integers(0, c.vocab, T)
    dy = oracle.bf16_round(rng.standard_normal((T, Hd), dtype=np.float32))
    cos, sin = oracle.rope_tables(np.arange(T), D, c.theta)
    cos, sin = cos[None, None], sin[None, None]
    heads = lambda x, n: np.ascontiguousarray(x.reshape(1, T, n, D).transpose(0, 2, 1, 3))
    rows = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3).reshape(T, -1))
    t0 = time.perf_counter()
    x0 = oracle.embedding(table, ids)
    n1, r1 = oracle.rms_norm_lanes_f32(x0, w1, c.eps)
    qkv = oracle.gemm_f32(n1, wqkv, 0, 1)
    q = oracle.rotary_prefix(heads(qkv[:, :hq * D], hq), cos, sin, D, 1)
    k = oracle.rotary_prefix(heads(qkv[:, hq * D:(hq + hkv) * D], hkv), cos, sin, D, 1)
    v = heads(qkv[:, (hq + hkv) * D:], hkv)
    o = rows(oracle.attention_f64(q, k, v, scale=D ** -0.5, causal=True, want_grads=False)["out"]).astype(np.float32)
    h1 = x0 + oracle.gemm_f32(o, wo, 0, 1)
    n2, r2 = oracle.rms_norm_lanes_f32(h1, w2, c.eps)
    gt, up = oracle.gemm_f32(n2, wg, 0, 1), oracle.gemm_f32(n2, wu, 0, 1)
    m = oracle.silu_mul_f64(gt, up).astype(np.float32)
    oracle.gemm_f32(m, wd, 0, 1)  # y = h1 + this
    dm = oracle.gemm_f32(dy, wd, 0, 0)
    oracle.gemm_f32(dy, m, 1, 0)                                   # dWd
    dgt, dup = (x.astype(np.float32) for x in oracle.silu_mul_backward_f64(gt, up, dm))
    dn2 = oracle.gemm_f32(dgt, wg, 0, 0) + oracle.gemm_f32(dup, wu, 0, 0)
    oracle.gemm_f32(dgt, n2, 1, 0), oracle.gemm_f32(dup, n2, 1, 0)  # dWg, dWu
    dh1 = oracle.rms_norm_backward_lanes_f32(h1, w2, dn2, r2)[0] + dy
    do = oracle.gemm_f32(dh1, wo, 0, 0)
    oracle.gemm_f32(dh1, o, 1, 0)                                   # dWo
    g = oracle.attention_f64(q, k, v, heads(do, hq), scale=D ** -0.5, causal=True)
    dq = oracle.rotary_prefix(g["dq"], cos, sin, D, 1, backward=True)
    dk = oracle.rotary_prefix(g["dk"], cos, sin, D, 1, backward=True)
    dqkv = np.concatenate([rows(dq), rows(dk), rows(g["dv"].astype(np.float32))], axis=1)
    dn1 = oracle.gemm_f32(dqkv, wqkv, 0, 0)
    oracle.gemm_f32(dqkv, n1, 1, 0)                                 # dWqkv
    dx0 = oracle.rms_norm_backward_lanes_f32(x0, w1, dn1, r1)[0] + dh1
    oracle.embedding_backward_f64(dx0, ids, c.vocab)                # dtable (dense)
    t = time.perf_counter() - t0
    return {"value": round(T / t, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"1 x {T} tokens"}


def c5_line(steps=5, warmup=2, cpu=True):
    cfg, f_ms, b_ms = bench_decoder(steps, warmup)
    step_ms = f_ms + b_ms
    fl = cfg.flops_per_step()
    tflops = fl["total"] / (step_ms * 1e-3) / 1e12
    line = {"workload": "C5 decoder layer fwd+bwd",
            "value": round(cfg.tokens / (step_ms * 1e-3), 1), "unit": "tokens/s",
            "ms": round(step_ms, 4), "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4),
            "model_TFLOPs": round(tflops, 1),
            # the layer is GEMM-dominated (96 % of its model flops are the projections): its
            # roofline is the model flops over the step against the BF16 MFMA peak; traffic and
            # MFMA utilisation are the step's counters (all its kernels) when measured
            "roofline": {"kernel": "gemm_nt_m16_kernel (96 % of the flops)", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                         "traffic_MB": None}}
    counters = read_counters("c5")
    if counters:
        line["roofline"]["traffic_MB"] = round(counters["traffic"] / 1e6)
        line["roofline"]["mfma_util"] = counters["mfma_util"]
    if cpu:
        line["cpu_baseline"] = short_cpu(cpu_baseline_decoder())
    return line


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from rust_ascend_hip import HipRuntime
    torch.cuda.set_device(0)
    if args.stream_ceilings:
        print(json.dumps({"hbm_stream_GBps_1GiB_buffers": {"torch": stream_ceilings()}}))
        return
    HipRuntime.initialize_exclusive()
    HipRuntime.set_async(True)
    if args.kernel:
        print(json.dumps(run_kernel(args.kernel, args.steps, args.warmup)), flush=True)
        if args.copy_calibration:
            copy_calibration()
        return
    if args.vendor:
        for entry in bench_vendor():
            print(json.dumps(entry), flush=True)
        return
    if args.only_c5:
        print(json.dumps(c5_line(args.steps, args.warmup)), flush=True)
        return
    if args.only_widened:
        for entry in bench_widened():
            print(json.dumps(entry), flush=True)
        if args.copy_calibration:
            copy_calibration()
        return

    wall_ms, fwd_ms, bwd_ms = bench_c2(args.steps, args.warmup)
    step_bytes = C2_FWD_BYTES + C2_BWD_BYTES
    value = step_bytes / (wall_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic, seeded, resident in HBM (x, dy N(0,1) BF16; weight 1+N(0,0.1) F32)",
        "config": {"workload": "C2 RMSNorm fwd+bwd: x[16384,4096] BF16, weight F32, eps 1e-6, dX BF16, dW F32",
                   "rows": C2_ROWS, "width": C2_WIDTH, "bytes_per_step": step_bytes,
                   "fwd_ms": round(fwd_ms, 5), "bwd_ms": round(bwd_ms, 5),
                   "fwd_GBps": round(C2_FWD_BYTES / fwd_ms / 1e6, 1),
                   "bwd_GBps": round(C2_BWD_BYTES / bwd_ms / 1e6, 1)},
        # the backward call is two kernels (the row kernel and the dγ partial sum); the events
        # time the call, so the roofline is the call's
        "roofline": roofline("hbm", C2_BWD_BYTES, bwd_ms, "rms_bwd_split+sum_partials8"),
    }
    sec = None
    if not args.no_secondary:
        sec = bench_widened()
        try:
            sec.append(c5_line(cpu=not args.no_cpu))
        except Exception as exc:  # reported, never silently replaced by another path
            sec.append({"workload": "C5 decoder layer", "error": str(exc)[:200]})
        ms, algo = bench_rope()
        sec.append({"workload": "C4 RoPE Q and K",
                    "value": round(algo / ms / 1e6, 1), "unit": "GB/s", "ms": round(ms, 4),
                    "roofline": short_roofline(roofline("hbm", algo, ms, "rope_rows", "rope"))})
        if not args.no_cpu:
            sec[-1]["cpu_baseline"] = short_cpu(cpu_baseline_rope())
        try:
            f_ms, b_ms, ff, bf = bench_attention()
            sec.append({"workload": "C4 attention fwd", "value": round(ff / f_ms / 1e9, 1), "unit": "TFLOP/s",
                        "ms": round(f_ms, 4),
                        "roofline": short_roofline(roofline("mfma", ff, f_ms, "attn_fwd_pp16", "attn_fwd"))})
            sec.append({"workload": "C4 attention bwd", "value": round(bf / b_ms / 1e9, 1), "unit": "TFLOP/s",
                        "ms": round(b_ms, 4),
                        "roofline": short_roofline(roofline("mfma", bf, b_ms, "attn_bwd_dkdv+attn_bwd_dq_ds",
                                                            "attn_bwd"))})
            st_ms, st_fl = bench_c4_step()
            sec.append({"workload": "C4 step: RoPE Q,K + attention fwd+bwd + RoPE bwd", "value": round(st_fl / st_ms / 1e9, 1), "unit": "TFLOP/s",
                        "ms": round(st_ms, 4), "frac": round(st_fl / st_ms / 1e9 / BF16_PEAK_TFLOPS, 4)})
            if not args.no_cpu:
                sec[-1]["cpu_baseline"] = short_cpu(cpu_baseline_attention())
        except Exception as exc:  # reported, never silently replaced by another path
            sec.append({"workload": "C4 causal GQA attention", "error": str(exc)[:200]})
        for key in ("c1", "gemm1024_nt", "gemm4096_nt", "llama_down", "llama_up", "gemm8192_nn", "gemm8192_nt"):
            m, n, k, ta, tb, name = GEMMS[key]
            ms = bench_gemm(m, n, k, ta, tb)
            flops = 2 * m * n * k
            sec.append({"workload": name, "value": round(flops / ms / 1e9, 1), "unit": "TFLOP/s",
                        "ms": round(ms, 4),
                        "roofline": short_roofline(roofline("mfma", flops, ms, gemm_kernel_name(m, n, k, ta, tb),
                                                            key))})
            if not args.no_cpu:
                sec[-1]["cpu_baseline"] = short_cpu(cpu_baseline_gemm(m, n, k, ta, tb, CPU_ROWS.get(key)))
    if args.copy_calibration:
        copy_calibration()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_c2(cpu_threads())
    if sec is not None:
        # "secondary" is the line's last key and the lines of the north-star targets are its last
        # entries, so a reader that keeps only the end of the line still sees them
        line["secondary"] = sorted(sec, key=lambda e: secondary_rank(e["workload"]))
    print(json.dumps(line), flush=True)


SECONDARY_LAST = ("C3 Llama 8192x14336->4096", "C3 Llama 8192x4096->14336", "C4 RoPE", "C4 step", "C4 attention bwd",
                  "C5", "C3 8192^3 NN", "C3 8192^3 NT", "C4 attention fwd")


def secondary_rank(workload):
    """Position class of a secondary line: 0 for the widened rows and the small GEMMs (in their
    measured order: the sort is stable), then SECONDARY_LAST's order."""
    for i, prefix in enumerate(SECONDARY_LAST):
        if workload.startswith(prefix):
            return i + 1
    return 0


if __name__ == "__main__":
    main()
