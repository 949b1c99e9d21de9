#!/usr/bin/env python3
"""Benchmark of the Clove Compute GEMM hot path on one MI355X.

Headline workload (the step): one FP16 GEMM C = A @ B at M = N = K = 4096,
row-major, A ~ N(0,1) activations and B ~ N(0,0.02) weights from a fixed
seed, fp32 accumulation, fp16 output, through the C ABI (clove_gemm_fp16).
`value` is TFLOP/s = 2*M*N*K / (time per step), inputs resident in HBM, W
untimed warm-up steps then exactly K timed steps between device syncs, HIP
events on the stream every call is launched on (torch's current stream).

The same JSON line also carries:
  roofline      the headline kernel against MI355X dense FP16 MFMA peak, with
                the HBM traffic per launch from the committed rocprof counters
  cpu_baseline  the oracle's restatement of the reference's naive GEMM
                (fp32 sequential-k FMA) on a bounded row sample: all usable
                cores (`value`, `cores`) and one thread (`value_1_thread`),
                with the host's nproc and CPU model
  shapes        every other shape of the five named configurations: FP16 512^3
                and M = 1/32/128 at 4096x4096, INT8 M = 1/128, INT4 W4A4
                (11008x4096 and 4096x11008, N = 1/16/128), the W4A16 Llama-1B
                layer at T = 1 and 512 as the reference runtime sequences it and
                with gate / up / SwiGLU fused, the FP16 Llama-1B MLP gate / up +
                SwiGLU (swiglu_fused) at T = 1 and 512, plus the reference benchmark's
                other FP16 shapes (512x4096^2, 1x11008x4096, 1x4096x11008,
                128x11008x4096, 128x4096x11008, 1024^3, 2048^3); each with
                t_roof = max(flops / MFMA peak, bytes / 8 TB/s) and
                frac_roofline = t_roof / time
The shapes are timed as HIP-graph replays of one call per operand copy: the
copies rotate through >= 512 MiB so that no call finds its weights in the
256 MB Infinity Cache (cold), and the graph removes the per-call host launch
cost, which exceeds most of these kernels' run time.  Each graph is checked
once against the same calls run eagerly.  `us` is graph time per call (kernel
plus the inter-kernel gap); `us_hot` replays one copy.  INT4 W4A4 is priced
at the INT8 MFMA peak (its integer products fit i8 operands).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 flop/clk/CU (dense, no sparsity)
PEAK_INT8_TOPS = 5033.2
PEAK_HBM_GBS = 8000.0
ROTATE_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the CPU-baseline sample (0 disables it)")
    ap.add_argument("--skip-extra", action="store_true", help="headline only")
    ap.add_argument("--floor", action="store_true",
                    help="only measure the cold HBM streaming-read floor (lib/libclove_diag.so) at the "
                         "weight sizes of the memory-bound shapes and print one JSON line")
    ap.add_argument("--compare-lib", action="store_true",
                    help="also time torch.matmul (hipBLASLt) on the headline operands, in blocks "
                         "alternating with clove_gemm_fp16, and report both")
    return ap.parse_args()


class Timer:
    """HIP events on torch's current stream, which is the stream every clove
    call below is launched on."""

    def __init__(self):
        import torch
        self.torch = torch
        self.s = torch.cuda.Event(enable_timing=True)
        self.e = torch.cuda.Event(enable_timing=True)

    def run(self, fn, steps, warmup):
        t = self.torch
        for i in range(warmup):
            fn(i)
        t.cuda.synchronize()
        self.s.record()
        for i in range(steps):
            fn(i)
        self.e.record()
        t.cuda.synchronize()
        return self.s.elapsed_time(self.e) / steps  # ms per call


def graph_time(calls, outputs, replays=5):
    """Captures calls[0..n) into one HIP graph on a private stream (after an
    eager pass on that stream, which also allocates any split-K scratch for it)
    and returns the mean time per call in microseconds over `replays` replays.
    The first replay's outputs must equal the eager ones bit for bit (the
    kernels are deterministic)."""
    import torch
    s = torch.cuda.Stream()
    torch.cuda.synchronize()  # operands were generated on the default stream
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outputs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for c in calls:
            c()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        for o in outputs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outputs, eager):
            if not torch.equal(o.view(torch.int16), e.view(torch.int16)):
                raise RuntimeError("graph replay differs from the eager calls")
        g.replay()
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * len(calls))
    del g
    return us


def headline(args, timer):
    import numpy as np
    import torch

    import clove_compute_amd as cg
    from tests._util import to_dev

    M = N = K = 4096
    g = np.random.default_rng(20261201)
    A_h = g.standard_normal((M, K)).astype(np.float16)
    B_h = (g.standard_normal((K, N)) * 0.02).astype(np.float16)
    A, B = to_dev(A_h), to_dev(B_h)
    C = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ms = timer.run(lambda i: cg.gemm_fp16(A, B, C, M, N, K), args.steps, args.warmup)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return dict(ms=ms, tflops=tflops, A=A_h, B=B_h, C=C, dA=A, dB=B)


def compare_library(h, timer, steps, warmup, rounds=3):
    """torch.matmul (hipBLASLt on ROCm) and clove_gemm_fp16 on the headline's
    device operands, timed the same way in alternating blocks (the clock drifts
    with sustained load, so neither side gets a cooler GPU).  TFLOP/s per block."""
    import torch

    import clove_compute_amd as cg

    A, B, C = h["dA"], h["dB"], h["C"]
    M, K = A.shape
    N = B.shape[1]
    C2 = torch.empty_like(C)
    tf = lambda ms: 2.0 * M * N * K / (ms * 1e-3) / 1e12
    out = {"torch_matmul": [], "clove_gemm_fp16": []}
    for _ in range(rounds):
        out["torch_matmul"].append(round(tf(timer.run(lambda i: torch.matmul(A, B, out=C2), steps, warmup)), 1))
        out["clove_gemm_fp16"].append(round(tf(timer.run(lambda i: cg.gemm_fp16(A, B, C, M, N, K), steps, warmup)), 1))
    return out


def cpu_threads():
    """Threads for the all-cores CPU baseline: the cores this process may run
    on, capped by OMP_NUM_THREADS when the host sets it (the GPU host's share of
    its CPUs for one GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(h, seconds):
    """Times the oracle's naive-arithmetic FP16 GEMM on rows of the same
    4096^3 problem: about half of `seconds` on one thread and half on all usable
    cores (rows spread over POSIX threads).  Each leg is one call over a row
    range sized from a short calibration, so B is widened to fp32 once per leg.
    `value` is the all-cores figure."""
    import numpy as np

    import oracle
    from tests._util import to_host, within_tol

    A, B = h["A"], h["B"]
    M, K = A.shape
    N = B.shape[1]
    out = np.zeros((M, N), np.float16)

    def leg(r0, r1, nthreads):
        t0 = time.perf_counter()
        if nthreads == 1:
            out[r0:r1] = oracle.gemm_fp16(A[r0:r1], B)
        else:
            out[r0:r1] = oracle.gemm_fp16_mt(A[r0:r1], B, (0, r1 - r0), nthreads)
        return time.perf_counter() - t0

    nt = cpu_threads()
    # calibration on one thread: the difference of 12 and 4 rows leaves out
    # the per-call widening of B
    per_row = max((leg(0, 12, 1) - leg(0, 4, 1)) / 8, 1e-4)
    rows1 = int(min(M // 2, max(8, seconds / 2 / per_row)))
    dt1 = leg(0, rows1, 1)
    rowsn = int(min(M - rows1, max(nt, seconds / 2 / (dt1 / rows1) * nt * 0.8)))
    dtn = leg(rows1, rows1 + rowsn, nt)
    tf1 = 2.0 * rows1 * N * K / dt1 / 1e12
    tfn = 2.0 * rowsn * N * K / dtn / 1e12
    # the sampled rows double as a parity check of the timed GPU output
    done = rows1 + rowsn
    pick = sorted({0, 1, rows1 - 1, rows1, done - 1})
    ok, _ = within_tol(to_host(h["C"])[pick], oracle.gemm_fp16_f64(A[pick], B))
    return dict(value=tfn, unit="TFLOP/s", cores=nt, kind="port",
                value_1_thread=tf1, nproc=os.cpu_count(), cpu_model=cpu_model(),
                sample=f"rows of the 4096x4096x4096 FP16 GEMM: rows 0..{rows1 - 1} on one thread "
                       f"({rows1} rows, {dt1:.1f} s, {tf1 * 1e3:.2f} GFLOP/s), rows {rows1}..{done - 1} "
                       f"on {nt} threads ({rowsn} rows, {dtn:.1f} s); oracle/clove_oracle.c restatement of "
                       f"gemm_fp16_naive_kernel (fp32 sequential-k fmaf)",
                parity_rows_ok=bool(ok))


def device_info():
    """Compute units and the maximum shader clock the runtime reports (the
    peaks above assume 256 CUs at 2.4 GHz; under sustained MFMA load the clock
    runs lower, which is why the measured fraction of peak is a clock-bound
    figure, not a per-cycle one)."""
    import ctypes

    import torch
    props = torch.cuda.get_device_properties(0)
    info = {"name": props.name, "arch": getattr(props, "gcnArchName", None), "cus": props.multi_processor_count}
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        v = ctypes.c_int(0)
        # hipDeviceAttributeClockRate (kHz)
        if hip.hipDeviceGetAttribute(ctypes.byref(v), 5, 0) == 0 and v.value > 0:
            info["max_sclk_mhz"] = v.value // 1000
    except OSError:
        pass
    return info


def copies_for(nbytes):
    return max(2, -(-ROTATE_BYTES // max(1, nbytes)))


def extras():
    """Every shape of the five named configurations except the headline, each
    timed as graph replays with cold weights.  Returns {name: figures}."""
    import torch

    import clove_compute_amd as cg

    gen = torch.Generator(device="cuda")

    def f16(shape, scale, seed):
        gen.manual_seed(seed)
        return (torch.randn(shape, generator=gen, device="cuda") * scale).half()

    def u16(shape, seed):  # fp16 ~U[-1, 1]
        gen.manual_seed(seed)
        return (torch.rand(shape, generator=gen, device="cuda") * 2 - 1).half()

    def u8(shape, seed, hi=256):
        gen.manual_seed(seed)
        return torch.randint(0, hi, shape, generator=gen, device="cuda", dtype=torch.uint8)

    def i8(shape, seed):
        gen.manual_seed(seed)
        return torch.randint(-127, 128, shape, generator=gen, device="cuda", dtype=torch.int8)

    def uni16(shape, lo, hi, seed):
        gen.manual_seed(seed)
        return (torch.rand(shape, generator=gen, device="cuda") * (hi - lo) + lo).half()

    def zeros16(shape, seed):
        gen.manual_seed(seed)
        return torch.randint(0, 16, shape, generator=gen, device="cuda").half()

    out = {}

    def record(name, calls, outputs, flops, nbytes, peak, hot_calls=None, replays=5):
        us = graph_time(calls, outputs, replays)
        t_mfma = flops / (peak * 1e6)
        t_hbm = nbytes / (PEAK_HBM_GBS * 1e3)
        t_roof = max(t_mfma, t_hbm)
        d = dict(us=us, TFLOPs=flops / us / 1e6, GBs=nbytes / us / 1e3,
                 bound="mfma" if t_mfma >= t_hbm else "hbm", t_roof_us=t_roof, frac_roofline=t_roof / us)
        if hot_calls is not None:
            d["us_hot"] = graph_time(hot_calls, outputs[:1], replays)
        out[name] = d
        print(f"[bench] {name}: {us:.2f} us", file=sys.stderr, flush=True)

    # ---- FP16: 512^3 (U[-1,1]) and the decode/prefill rows of the LLM shapes ----
    A5, B5 = u16((512, 512), 1), u16((512, 512), 2)
    C5 = torch.empty(512, 512, dtype=torch.float16, device="cuda")
    c = [lambda: cg.gemm_fp16(A5, B5, C5, 512, 512, 512)] * 16
    record("fp16_512x512x512", c, [C5], 2 * 512 ** 3, 2 * 3 * 512 * 512, PEAK_FP16_TFLOPS)
    for M in (1, 32, 128):
        N = K = 4096
        x = f16((M, K), 1.0, 3 + M)
        Bs = [f16((K, N), 0.02, 100 + i) for i in range(copies_for(K * N * 2))]
        Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in Bs]
        calls = [lambda B=B, C=C, M=M: cg.gemm_fp16(x, B, C, M, N, K) for B, C in zip(Bs, Cs)]
        record(f"fp16_{M}x4096x4096", calls, Cs, 2 * M * N * K, 2 * (M * K + K * N + M * N),
               PEAK_FP16_TFLOPS, hot_calls=calls[:1] * 16 if M == 1 else None)
        del Bs, Cs, calls

    # ---- the reference benchmark's other FP16 shapes (bench/bench_gemm.cu:20-37):
    # (M, N, K) with activations ~N(0,1) and weights ~N(0,0.02), weights cold ----
    for (M, N, K) in ((512, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (128, 11008, 4096),
                      (128, 4096, 11008), (1024, 1024, 1024), (2048, 2048, 2048)):
        x = f16((M, K), 1.0, 40 + M)
        Bs = [f16((K, N), 0.02, 140 + i) for i in range(copies_for(K * N * 2))]
        Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in Bs]
        calls = [lambda B=B, C=C, M=M, N=N, K=K: cg.gemm_fp16(x, B, C, M, N, K) for B, C in zip(Bs, Cs)]
        record(f"ref_bench_fp16_{M}x{N}x{K}", calls, Cs, 2 * M * N * K, 2 * (M * K + K * N + M * N),
               PEAK_FP16_TFLOPS)
        del Bs, Cs, calls

    # ---- INT8 W8A8 with per-row / per-column fp16 scales: the decode / small
    # batch rows of config 3 (weights cold), and the prefill square 4096^3 ----
    for M in (1, 128, 4096):
        N = K = 4096
        a8 = i8((M, K), 8 + M)
        sa = uni16((M,), 0.001, 0.02, 9)
        sb = uni16((N,), 0.001, 0.02, 10)
        Bs = [i8((K, N), 500 + i) for i in range(copies_for(K * N))]
        Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in Bs]
        calls = [lambda B=B, C=C, M=M: cg.gemm_int8_rowcol(a8, B, sa, sb, C, M, N, K) for B, C in zip(Bs, Cs)]
        record(f"int8_{M}x4096x4096", calls, Cs, 2 * M * N * K, M * K + K * N + 2 * M * N + 2 * M + 2 * N,
               PEAK_INT8_TOPS)
        del Bs, Cs, calls

    # ---- INT4 W4A4 group-wise: weights A_q [M, K/2], activations B_q [K, ceil(N/2)] ----
    for (M, K) in ((11008, 4096), (4096, 11008)):
        G = -(-K // 128)
        wbytes = M * K // 2 + 4 * M * G
        sets = [(u8((M, K // 2), 200 + i), uni16((M, G), 0.001, 0.02, 300 + i), zeros16((M, G), 400 + i))
                for i in range(copies_for(wbytes))]
        for N in (1, 16, 128):
            Bq = u8((K, 1), 5, 16) << 4 if N == 1 else u8((K, (N + 1) // 2), 5)
            Bsc = uni16((G, N), 0.001, 0.02, 6)
            Bz = zeros16((G, N), 7)
            Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in sets]
            calls = [lambda s=s, C=C, Bq=Bq, Bsc=Bsc, Bz=Bz, N=N: cg.gemm_int4(*s, Bq, Bsc, Bz, C, M, N, K)
                     for s, C in zip(sets, Cs)]
            nb = wbytes + K * ((N + 1) // 2) + 4 * G * N + 2 * M * N
            record(f"int4_w4a4_{M}x{K}_n{N}", calls, Cs, 2 * M * N * K, nb, PEAK_INT8_TOPS,
                   hot_calls=calls[:1] * 16 if N == 1 else None)
            del Cs, calls
        del sets

    # ---- W4A16 Llama-1B decoder-layer GEMM sequence, as the reference runtime
    # runs its linear layers (src/runtime/inference.cu:139-194): QKV, O +
    # residual, gate, up, SwiGLU, down + residual; and the same layer with the
    # gate / up projections and SwiGLU fused into one pass over a [2I, K/2]
    # weight (clove_w4a16_swiglu) ----
    hid, inter = 2048, 8192
    layer = [(3072, hid, 0.0), (hid, hid, 1.0), (inter, hid, 0.0), (inter, hid, 0.0), (hid, inter, 1.0)]
    wbytes = sum(O * K // 2 + 4 * O * (-(-K // 128)) for O, K, _ in layer)

    def make_layer(i):
        return [(u8((O, K // 2), 600 + 10 * i + j), uni16((O, -(-K // 128)), 0.001, 0.02, 700 + 10 * i + j),
                 zeros16((O, -(-K // 128)), 800 + 10 * i + j)) for j, (O, K, _) in enumerate(layer)]

    def fuse_gate_up(L):
        # [gate rows; up rows] as one weight: the same numbers as L[2], L[3]
        return [L[0], L[1], tuple(torch.cat([L[2][k], L[3][k]], 0) for k in range(3)), L[4]]

    for T in (1, 512):
        layers = [make_layer(i) for i in range(copies_for(wbytes) if T == 1 else 2)]
        x = f16((T, hid), 1.0, 900)
        attn = f16((T, hid), 1.0, 901)
        q = torch.empty(T, 3072, dtype=torch.float16, device="cuda")
        res = f16((T, hid), 1.0, 902)
        gate = torch.empty(T, inter, dtype=torch.float16, device="cuda")
        up = torch.empty_like(gate)
        h = torch.empty_like(gate)

        def step(L, T=T):
            cg.gemm_w4a16(x, *L[0], q, T, 3072, hid, 1.0, 0.0)
            cg.gemm_w4a16(attn, *L[1], res, T, hid, hid, 1.0, 1.0)
            cg.gemm_w4a16(x, *L[2], gate, T, inter, hid, 1.0, 0.0)
            cg.gemm_w4a16(x, *L[3], up, T, inter, hid, 1.0, 0.0)
            cg.swiglu(gate, up, h, T * inter)
            cg.gemm_w4a16(h, *L[4], res, T, hid, inter, 1.0, 1.0)

        def step_fused(L, T=T):
            cg.gemm_w4a16(x, *L[0], q, T, 3072, hid, 1.0, 0.0)
            cg.gemm_w4a16(attn, *L[1], res, T, hid, hid, 1.0, 1.0)
            cg.w4a16_swiglu(x, *L[2], h, T, inter, hid)
            cg.gemm_w4a16(h, *L[3], res, T, hid, inter, 1.0, 1.0)

        flops = sum(2 * T * O * K for O, K, _ in layer)
        lin = sum(2 * T * K + 2 * T * O * (2 if b else 1) for O, K, b in layer)
        # the residual projections accumulate into res across calls: compare the
        # other outputs only
        calls = [lambda L=L: step(L) for L in layers]
        record(f"w4a16_llama1b_layer_T{T}", calls, [q, gate, up, h], flops,
               wbytes + lin + 3 * 2 * T * inter, PEAK_FP16_TFLOPS, replays=5 if T == 1 else 3)
        fused = [fuse_gate_up(L) for L in layers]
        del layers, calls
        calls = [lambda L=L: step_fused(L) for L in fused]
        lin_f = lin - 2 * (2 * T * hid + 2 * T * inter) + (2 * T * hid + 2 * T * inter)
        record(f"w4a16_llama1b_layer_fused_T{T}", calls, [q, h], flops, wbytes + lin_f,
               PEAK_FP16_TFLOPS, replays=5 if T == 1 else 3)
        del fused, calls

    # ---- FP16 Llama-1B MLP: gate / up projections and SwiGLU on FP16 weights
    # [2048, 8192] (the reference's declared swiglu_fused), one fused launch,
    # and the same as two gemm_fp16 calls and swiglu for comparison ----
    H, I = 2048, 8192
    wb = 2 * H * I * 2
    for T in (1, 512):
        x = f16((T, H), 1.0, 950)
        pairs = [(f16((H, I), 0.02, 960 + 2 * i), f16((H, I), 0.02, 961 + 2 * i)) for i in range(copies_for(wb))]
        outs = [torch.empty(T, I, dtype=torch.float16, device="cuda") for _ in pairs]
        flops = 2 * 2 * T * H * I
        calls = [lambda w=w, o=o, T=T: cg.swiglu_fused(x, w[0], w[1], o, T, H, I) for w, o in zip(pairs, outs)]
        record(f"fp16_llama1b_mlp_swiglu_fused_T{T}", calls, outs, flops, wb + 2 * T * H + 2 * T * I,
               PEAK_FP16_TFLOPS)
        gate = torch.empty(T, I, dtype=torch.float16, device="cuda")
        up = torch.empty_like(gate)

        def unfused(w, o, T=T):
            cg.gemm_fp16(x, w[0], gate, T, I, H)
            cg.gemm_fp16(x, w[1], up, T, I, H)
            cg.swiglu(gate, up, o, T * I)
        calls = [lambda w=w, o=o: unfused(w, o) for w, o in zip(pairs, outs)]
        record(f"fp16_llama1b_mlp_unfused_T{T}", calls, outs, flops,
               wb + 2 * 2 * T * H + 3 * 2 * 2 * T * I, PEAK_FP16_TFLOPS)
        del pairs, outs, calls
    return out


def floor():
    """Cold read floor: a read-only streaming kernel (16-byte lane-contiguous
    loads, 32 KB per workgroup) over the weight sizes of the decode and
    memory-bound shapes, each timed as graph replays that rotate through
    >= 512 MiB of copies (no replay finds its bytes in the 256 MB Infinity
    Cache), and hot (one copy replayed)."""
    import ctypes

    import torch
    path = os.path.join(ROOT, "clove_compute_amd", "lib", "libclove_diag.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    lib.clove_diag_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.clove_diag_stream_read.restype = ctypes.c_int
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    out = {}
    for name, nbytes in (("int8_4096x4096_weight", 4096 * 4096),
                         ("int4_11008x4096_weight", 11008 * 4096 // 2),
                         ("fp16_4096x4096_weight", 4096 * 4096 * 2)):
        bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(copies_for(nbytes))]

        def call(b):
            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            if lib.clove_diag_stream_read(b.data_ptr(), nbytes, sink.data_ptr(), stream) <= 0:
                raise RuntimeError("clove_diag_stream_read failed")
        calls = [lambda b=b: call(b) for b in bufs]
        us = graph_time(calls, [], 5)
        hot = graph_time(calls[:1] * 16, [], 5)
        out[name] = {"MB": round(nbytes / 1e6, 3), "copies": len(bufs), "us_cold": round(us, 3),
                     "GBs_cold": round(nbytes / us / 1e3, 1), "us_hot": round(hot, 3),
                     "GBs_hot": round(nbytes / hot / 1e3, 1)}
        print(f"[floor] {name}: cold {us:.2f} us, hot {hot:.2f} us", file=sys.stderr, flush=True)
        del bufs, calls
    # one CU's pull rate: 32 workgroups, each streaming 1 MB of a 32 MB buffer
    # (at most one workgroup per CU) with 32 KB or 128 KB in flight, cold and hot
    lib.clove_diag_stream_read_chunked.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.clove_diag_stream_read_chunked.restype = ctypes.c_int
    nbytes, chunk = 32 << 20, 1 << 20
    bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(copies_for(nbytes))]
    for depth in (1, 4):
        def call_chunk(b, depth=depth):
            stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            if lib.clove_diag_stream_read_chunked(b.data_ptr(), nbytes, chunk, depth, sink.data_ptr(), stream) <= 0:
                raise RuntimeError("clove_diag_stream_read_chunked failed")
        calls = [lambda b=b: call_chunk(b) for b in bufs]
        us = graph_time(calls, [], 5)
        hot = graph_time(calls[:1] * 16, [], 5)
        out[f"per_cu_32x1MB_inflight_{32 * depth}KB"] = {
            "workgroups": nbytes // chunk, "MB_per_workgroup": 1.049, "us_cold": round(us, 3),
            "GBs_per_workgroup_cold": round(chunk / us / 1e3, 1), "us_hot": round(hot, 3),
            "GBs_per_workgroup_hot": round(chunk / hot / 1e3, 1)}
        print(f"[floor] per CU (32 x 1 MB, {32 * depth} KB in flight): cold {us:.2f} us, hot {hot:.2f} us",
              file=sys.stderr, flush=True)
    # the same pull by load kind: 32 workgroups on their own 1 MB (cold, the
    # copies rotated), and 256 workgroups (one per CU) all reading one 1 MB
    # chunk that then sits in every XCD's L2
    lib.clove_diag_pull.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p]
    lib.clove_diag_pull.restype = ctypes.c_int
    for kind, kname in ((0, "nontemporal"), (1, "cached"), (2, "lds_dma")):
        for shared, grid in ((0, nbytes // chunk), (1, 256)):
            def call_pull(b, kind=kind, shared=shared, grid=grid):
                stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                if lib.clove_diag_pull(b.data_ptr(), chunk, grid, shared, kind, sink.data_ptr(), stream) != grid:
                    raise RuntimeError("clove_diag_pull failed")
            calls = [lambda b=b: call_pull(b) for b in bufs]
            us = graph_time(calls if not shared else calls[:1] * 16, [], 5)
            key = f"pull_{kname}_{'l2_shared_256x1MB' if shared else 'cold_32x1MB'}"
            out[key] = {"workgroups": grid, "us": round(us, 3), "GBs_per_workgroup": round(chunk / us / 1e3, 1),
                        "GBs_total": round(grid * chunk / us / 1e3, 1)}
            print(f"[floor] {key}: {us:.2f} us, {chunk / us / 1e3:.1f} GB/s per workgroup",
                  file=sys.stderr, flush=True)
    del bufs, calls
    print(json.dumps({"floor": out, "device": device_info()}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the GEMM path has no "
              "multi-GPU component in this build. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    from clove_compute_amd import _lib
    _lib.lib()  # fails loudly when the HIP library is not built
    if args.floor:
        floor()
        return

    timer = Timer()
    h = headline(args, timer)
    print(f"[bench] headline: {h['ms'] * 1e3:.1f} us per call", file=sys.stderr, flush=True)
    flops = 2.0 * 4096 ** 3
    achieved = h["tflops"]
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_fp16_gemm_4096.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    line = {
        "metric": "TFLOP/s + % roofline (MFMA or HBM) for gemm_fp16/int4 at 1x4096x4096 & 4096^3",
        "value": round(achieved, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded numpy PCG64: A ~ N(0,1), B ~ N(0,0.02), fp16)",
        "config": {"workload": "fp16_gemm_4096x4096x4096", "M": 4096, "N": 4096, "K": 4096,
                   "layout": "row-major A[M,K] B[K,N] C[M,N]", "accumulate": "fp32"},
        "device": device_info(),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic, "flops_per_launch": flops,
                     "kernel": "dma::gemm_f16_big<Big>"},
    }
    if args.compare_lib:
        line["library_comparison"] = compare_library(h, timer, args.steps, args.warmup)
    if not args.skip_extra:
        line["shapes"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                          for k, v in extras().items()}
    if args.cpu_seconds > 0:
        cb = cpu_baseline(h, args.cpu_seconds)
        cb["value"] = round(cb["value"], 6)
        cb["value_1_thread"] = round(cb["value_1_thread"], 6)
        line["cpu_baseline"] = cb
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    # leave nothing behind on the GPU: the library's split-K scratch is freed and
    # every stream drained before the interpreter tears the runtime down
    import torch
    import clove_compute_amd as cg
    torch.cuda.synchronize()
    cg.release_scratch()
    torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
