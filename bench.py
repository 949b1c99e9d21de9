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
once against the same calls run eagerly, and the first call's output on a few
rows against the oracle (`parity`: bit-exact for INT8, the tolerance of the
GPU tests otherwise; a mismatch stops the run).  `us` is graph time per call
(kernel plus the inter-kernel gap); `us_hot` replays one copy.  INT4 W4A4 is
priced at the INT8 MFMA peak (its integer products fit i8 operands).  With
--compare-lib every FP16 shape is also timed through torch.matmul (hipBLASLt)
and INT8 M > 16 through torch._int_mm on the same operands (`lib_us`).

`device.sclk_mhz_measured` is the shader clock under the headline's load (a
probe wave after each launch counts shader cycles against the 100 MHz
constant counter), and `roofline.frac_at_measured_sclk` the headline against
the dense peak at that clock.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]
                       [--skip-extra] [--compare-lib] [--floor]
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
    ap.add_argument("--phases", action="store_true",
                    help="only measure the headline kernel's phases (prologue, K loop, epilogue, the spread "
                         "and gaps between launches) from per-workgroup timestamps (lib/libclove_diag.so) and "
                         "print one JSON line")
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


def graph_time(calls, outputs, replays=5, compare=True):
    """Captures calls[0..n) into one HIP graph on a private stream (after an
    eager pass on that stream, which also allocates any split-K scratch for it)
    and returns the mean time per call in microseconds over `replays` replays.
    The first replay's outputs must equal the eager ones bit for bit (the
    kernels are deterministic; `compare=False` for a library's calls)."""
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
        for o, e in zip(outputs if compare else [], eager):
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


def diag_lib():
    import ctypes
    path = os.path.join(ROOT, "clove_compute_amd", "lib", "libclove_diag.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    return ctypes.CDLL(path)


def measure_sclk(h, steps, ticks=200):
    """The shader clock under the headline's load: `steps` launches of the
    headline GEMM on torch's current stream, each followed by a probe wave
    (libclove_diag.so sclk_probe) that counts shader cycles over `ticks` of
    the 100 MHz constant counter (2 us), right after the GEMM drains.  Returns
    the median, min and max in MHz over the probes."""
    import ctypes

    import torch

    import clove_compute_amd as cg
    lib = diag_lib()
    lib.clove_diag_sclk.argtypes = [ctypes.c_void_p, ctypes.c_uint, ctypes.c_void_p]
    lib.clove_diag_sclk.restype = ctypes.c_int
    A, B, C = h["dA"], h["dB"], h["C"]
    n = 4096
    buf = torch.zeros(steps, 4, dtype=torch.int64, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in range(steps):
        cg.gemm_fp16(A, B, C, n, n, n)
        if lib.clove_diag_sclk(ctypes.c_void_p(buf[i].data_ptr()), ticks, stream) != 0:
            raise RuntimeError("clove_diag_sclk failed")
    torch.cuda.synchronize()
    v = buf.cpu().tolist()
    mhz = sorted(100.0 * (c1 - c0) / (r1 - r0) for c0, r0, c1, r1 in v if r1 > r0)
    if not mhz:
        return None
    return {"median": round(mhz[len(mhz) // 2], 1), "min": round(mhz[0], 1), "max": round(mhz[-1], 1),
            "probes": len(mhz)}


def phases(args, timer, rounds=3, series=300):
    """The headline kernel phase by phase.  dma::gemm_f16_big_ts is the
    product kernel's body with shader-cycle (s_memtime) and 100 MHz
    (s_memrealtime) timestamps at its phase boundaries, one record per
    workgroup (libclove_diag.so clove_diag_fp16_big_phases).
      1. `series` timestamped launches back to back from this process's
         first GEMM launch: per launch the K loop's clock, the span of its
         workgroups and the gap to the next launch (the shader clock's
         response to the sustained load, launch by launch);
      2. blocks of `steps` back-to-back launches of the product call and of
         the timestamped kernel, alternating `rounds` times (per-launch event
         time of each: the cost of the timestamps);
      3. from the last timestamped block, per workgroup: the time from entry
         until its first K tile has landed, the first two K tiles, the shader
         cycles per K tile and the clock over the remaining K tiles, and the
         output stores; per launch, the spread of the workgroups' starts and
         ends and the gap to the next launch."""
    import ctypes

    import numpy as np
    import torch

    import clove_compute_amd as cg
    from tests._util import to_dev
    lib = diag_lib()
    lib.clove_diag_fp16_big_phases.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_void_p] * 2
    lib.clove_diag_fp16_big_phases.restype = ctypes.c_int
    n = 4096
    g = np.random.default_rng(20261201)  # the headline's operands
    A = to_dev(g.standard_normal((n, n)).astype(np.float16))
    B = to_dev((g.standard_normal((n, n)) * 0.02).astype(np.float16))
    C = torch.empty(n, n, dtype=torch.float16, device="cuda")
    ref = torch.empty_like(C)
    grid, words = 256, 16
    steps = args.steps
    nts = max(series, steps)
    ts = torch.zeros(nts, grid, words, dtype=torch.int64, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    def product(i):
        cg.gemm_fp16(A, B, C, n, n, n)

    def stamped(i):
        if lib.clove_diag_fp16_big_phases(A.data_ptr(), B.data_ptr(), C.data_ptr(), n, n, n,
                                          ctypes.c_void_p(ts[i % nts].data_ptr()), stream) != grid:
            raise RuntimeError("clove_diag_fp16_big_phases failed")

    def records(count):
        t = ts[:count].cpu().numpy().astype(np.int64)
        if not (t[:, :, 10] == n // 64).all():
            raise RuntimeError("a workgroup wrote no record")
        return t[:, :, 0:10:2], t[:, :, 1:10:2].astype(np.float64) * 0.01, t[:, :, 12]  # cycles, us, XCC

    # 1. the series from the first launch
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(series // 10 + 1)]
    ev[0].record()
    for i in range(series):
        stamped(i)
        if (i + 1) % 10 == 0:
            ev[(i + 1) // 10].record()
    torch.cuda.synchronize()
    cyc, rt, _ = records(series)
    lmhz = np.median((cyc[:, :, 3] - cyc[:, :, 2]) / (rt[:, :, 3] - rt[:, :, 2]), axis=1)
    sgap = rt[1:, :, 0].min(1) - rt[:-1, :, 4].max(1)
    ser = [{"launches": f"{10 * j}-{10 * j + 9}",
            "us_per_launch": round(ev[j].elapsed_time(ev[j + 1]) * 100.0, 1),
            "k_loop_sclk_mhz": round(float(np.median(lmhz[10 * j:10 * j + 10])), 0),
            "span_us": round(float(np.median(rt[10 * j:10 * j + 10, :, 4].max(1) - rt[10 * j:10 * j + 10, :, 0].min(1))), 1),
            "gap_us": round(float(np.median(sgap[10 * j:min(10 * j + 10, series - 1)])), 2)}
           for j in range(series // 10)]
    cg.gemm_fp16(A, B, ref, n, n, n)
    torch.cuda.synchronize()
    if not torch.equal(C.view(torch.int16), ref.view(torch.int16)):
        raise RuntimeError("the timestamped kernel's output differs from clove_gemm_fp16's")

    # 2. alternating blocks
    prod_us, ts_us = [], []
    for _ in range(rounds):
        prod_us.append(timer.run(product, steps, args.warmup) * 1e3)
        ts_us.append(timer.run(stamped, steps, args.warmup) * 1e3)
    torch.cuda.synchronize()
    if not torch.equal(C.view(torch.int16), ref.view(torch.int16)):
        raise RuntimeError("the timestamped kernel's output differs from clove_gemm_fp16's")

    # 3. the last timestamped block
    cyc, rt, xcc = records(steps)

    def pct(v):
        v = np.asarray(v, dtype=np.float64).ravel()
        return {"p10": round(float(np.percentile(v, 10)), 3), "median": round(float(np.median(v)), 3),
                "p90": round(float(np.percentile(v, 90)), 3)}

    loop_cyc = (cyc[:, :, 3] - cyc[:, :, 2]) / (n // 64 - 2)
    loop_us = rt[:, :, 3] - rt[:, :, 2]
    loop_mhz = (cyc[:, :, 3] - cyc[:, :, 2]) / loop_us
    first_mhz = (cyc[:, :, 1] - cyc[:, :, 0]) / np.maximum(rt[:, :, 1] - rt[:, :, 0], 0.01)
    starts, ends = rt[:, :, 0], rt[:, :, 4]
    span = ends.max(1) - starts.min(1)
    gap = starts.min(1)[1:] - ends.max(1)[:-1]
    out = {
        "workload": "fp16_gemm_4096x4096x4096", "launches": steps, "workgroups": grid,
        "series_from_first_launch": ser,
        "us_per_launch_event": {"product": [round(x, 2) for x in prod_us], "timestamped": [round(x, 2) for x in ts_us]},
        "per_workgroup_us": {
            "entry_to_first_tile_landed": pct(rt[:, :, 1] - rt[:, :, 0]),
            "first_two_k_tiles": pct(rt[:, :, 2] - rt[:, :, 1]),
            "k_tiles_3_to_64": pct(loop_us),
            "epilogue_to_stores_done": pct(rt[:, :, 4] - rt[:, :, 3]),
            "workgroup_total": pct(ends - starts),
        },
        "k_loop_cycles_per_tile": pct(loop_cyc),
        "k_loop_sclk_mhz": pct(loop_mhz),
        "prologue_sclk_mhz": pct(first_mhz),
        "k_loop_sclk_mhz_by_xcc": {int(x): round(float(np.median(loop_mhz[xcc == x])), 1)
                                   for x in np.unique(xcc)},
        "per_launch_us": {"start_spread": pct(starts.max(1) - starts.min(1)),
                          "end_spread": pct(ends.max(1) - ends.min(1)),
                          "span_first_start_to_last_end": pct(span),
                          "gap_to_next_launch": pct(gap) if gap.size else None},
        "mfma_bound_cycles_per_tile": 2048,
        "device": device_info(),
    }
    print(json.dumps({"phases": out}), flush=True)


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


def pick_rows(n, count=4):
    """A few row indices spread over [0, n): the first, the last and some between."""
    return sorted({0, n - 1, n // 3, (2 * n) // 3, n // 2}) if n > 1 else [0]


def extras(compare_lib=False):
    """Every shape of the five named configurations except the headline, each
    timed as graph replays with cold weights and its first call's output
    checked on a few rows against the oracle.  Returns {name: figures}."""
    import numpy as np
    import torch

    import clove_compute_amd as cg
    import oracle
    from tests._util import f16bits, to_host, within_tol

    def host(t):
        return to_host(t) if t.dtype == torch.float16 else t.cpu().numpy()

    def tol(got, ref64):
        ok, rep = within_tol(got, ref64)
        if not ok:
            raise RuntimeError(f"parity check failed: {rep}")
        return f"ok: max rel err {rep['max_rel_err_floored']:.2e} (bound 1e-2)"

    def chk_fp16(x, B, C, M):
        rows = pick_rows(M)
        return lambda: tol(host(C)[rows], oracle.gemm_fp16_f64(host(x)[rows], host(B)))

    def chk_int8(a8, B, sa, sb, C, M):
        rows = pick_rows(M)

        def f():
            ref, _ = oracle.gemm_int8_rowcol(host(a8)[rows], host(B), host(sa)[rows], host(sb))
            if not np.array_equal(f16bits(host(C)[rows]), f16bits(ref)):
                raise RuntimeError("parity check failed: INT8 output differs from the oracle")
            return "ok: bit-exact"
        return f

    def chk_int4(s, Bq, Bsc, Bz, C, M, N, K):
        rows = pick_rows(M)

        def f():
            Aq, sA, zA = (host(t)[rows] for t in s)
            _, ref, _ = oracle.gemm_int4_groupwise(Aq, sA, zA, host(Bq), host(Bsc), host(Bz), len(rows), N, K)
            return tol(host(C)[rows], ref)
        return f

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

    def record(name, calls, outputs, flops, nbytes, peak, hot_calls=None, replays=5, check=None,
               lib_calls=None, lib_outputs=None):
        """Times `calls`, then checks the outputs of the first call against the
        oracle (`check()` raises on a mismatch, so no wrong kernel yields a
        timed number) and, with --compare-lib, times the library's calls on the
        same operands the same way."""
        us = graph_time(calls, outputs, replays)
        t_mfma = flops / (peak * 1e6)
        t_hbm = nbytes / (PEAK_HBM_GBS * 1e3)
        t_roof = max(t_mfma, t_hbm)
        d = dict(us=us, TFLOPs=flops / us / 1e6, GBs=nbytes / us / 1e3,
                 bound="mfma" if t_mfma >= t_hbm else "hbm", t_roof_us=t_roof, frac_roofline=t_roof / us)
        if hot_calls is not None:
            d["us_hot"] = graph_time(hot_calls, outputs[:1], replays)
        if check is not None:
            d["parity"] = check()
        if lib_calls is not None and compare_lib:
            try:
                lus = graph_time(lib_calls, lib_outputs or [], replays, compare=False)
                d["lib_us"] = lus
                d["lib_vs_clove"] = lus / us
            except Exception as e:  # a library without this shape
                d["lib_us"] = None
                d["lib_error"] = str(e).splitlines()[0][:120]
        out[name] = d
        print(f"[bench] {name}: {us:.2f} us" + (f" (library {d['lib_us']:.2f} us)" if d.get("lib_us") else ""),
              file=sys.stderr, flush=True)

    # ---- FP16: 512^3 (U[-1,1]) and the decode/prefill rows of the LLM shapes ----
    A5, B5 = u16((512, 512), 1), u16((512, 512), 2)
    C5 = torch.empty(512, 512, dtype=torch.float16, device="cuda")
    L5 = torch.empty_like(C5)
    c = [lambda: cg.gemm_fp16(A5, B5, C5, 512, 512, 512)] * 16
    record("fp16_512x512x512", c, [C5], 2 * 512 ** 3, 2 * 3 * 512 * 512, PEAK_FP16_TFLOPS,
           check=chk_fp16(A5, B5, C5, 512), lib_calls=[lambda: torch.matmul(A5, B5, out=L5)] * 16)
    for M in (1, 32, 128):
        N = K = 4096
        x = f16((M, K), 1.0, 3 + M)
        Bs = [f16((K, N), 0.02, 100 + i) for i in range(copies_for(K * N * 2))]
        Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in Bs]
        calls = [lambda B=B, C=C, M=M: cg.gemm_fp16(x, B, C, M, N, K) for B, C in zip(Bs, Cs)]
        Ls = [torch.empty_like(C) for C in Cs] if compare_lib else []
        lcalls = [lambda B=B, L=L: torch.matmul(x, B, out=L) for B, L in zip(Bs, Ls)]
        record(f"fp16_{M}x4096x4096", calls, Cs, 2 * M * N * K, 2 * (M * K + K * N + M * N),
               PEAK_FP16_TFLOPS, hot_calls=calls[:1] * 16 if M == 1 else None,
               check=chk_fp16(x, Bs[0], Cs[0], M), lib_calls=lcalls)
        del Bs, Cs, calls, Ls, lcalls

    # ---- the reference benchmark's other FP16 shapes (bench/bench_gemm.cu:20-37):
    # (M, N, K) with activations ~N(0,1) and weights ~N(0,0.02), weights cold ----
    for (M, N, K) in ((512, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (128, 11008, 4096),
                      (128, 4096, 11008), (1024, 1024, 1024), (2048, 2048, 2048)):
        x = f16((M, K), 1.0, 40 + M)
        Bs = [f16((K, N), 0.02, 140 + i) for i in range(copies_for(K * N * 2))]
        Cs = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in Bs]
        calls = [lambda B=B, C=C, M=M, N=N, K=K: cg.gemm_fp16(x, B, C, M, N, K) for B, C in zip(Bs, Cs)]
        Ls = [torch.empty_like(C) for C in Cs] if compare_lib else []
        lcalls = [lambda B=B, L=L: torch.matmul(x, B, out=L) for B, L in zip(Bs, Ls)]
        record(f"ref_bench_fp16_{M}x{N}x{K}", calls, Cs, 2 * M * N * K, 2 * (M * K + K * N + M * N),
               PEAK_FP16_TFLOPS, check=chk_fp16(x, Bs[0], Cs[0], M), lib_calls=lcalls)
        del Bs, Cs, calls, Ls, lcalls

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
        # the library's int8 GEMM (int32 out, no scale epilogue; hipBLASLt
        # takes M > 16 only)
        Ls = [torch.empty(M, N, dtype=torch.int32, device="cuda") for _ in Bs] if compare_lib and M > 16 else []
        lcalls = [lambda B=B, L=L: torch._int_mm(a8, B, out=L) for B, L in zip(Bs, Ls)] if Ls else None
        record(f"int8_{M}x4096x4096", calls, Cs, 2 * M * N * K, M * K + K * N + 2 * M * N + 2 * M + 2 * N,
               PEAK_INT8_TOPS, check=chk_int8(a8, Bs[0], sa, sb, Cs[0], M), lib_calls=lcalls)
        del Bs, Cs, calls, Ls, lcalls

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
                   hot_calls=calls[:1] * 16 if N == 1 else None,
                   check=chk_int4(sets[0], Bq, Bsc, Bz, Cs[0], M, N, K))
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

        def chk_layer(L, fused, T=T):
            # one eager step on the first copy, then the QKV output and the MLP
            # activation h on a few tokens against the oracle (the residual
            # outputs accumulate across calls and are not compared)
            rows = pick_rows(T)

            def f():
                (step_fused if fused else step)(L)
                torch.cuda.synchronize()
                xr = host(x)[rows]
                _, q64 = oracle.w4a16(xr, *(host(t) for t in L[0]))
                r = [tol(host(q)[rows], q64)]
                if fused:
                    href = oracle.w4a16_swiglu(xr, *(host(t) for t in L[2]))
                else:
                    g_, _ = oracle.w4a16(xr, *(host(t) for t in L[2]))
                    u_, _ = oracle.w4a16(xr, *(host(t) for t in L[3]))
                    href = oracle.swiglu(g_, u_)
                r.append(tol(host(h)[rows], href.astype(np.float64)))
                return "; ".join(r)
            return f

        flops = sum(2 * T * O * K for O, K, _ in layer)
        lin = sum(2 * T * K + 2 * T * O * (2 if b else 1) for O, K, b in layer)
        # the residual projections accumulate into res across calls: compare the
        # other outputs only
        calls = [lambda L=L: step(L) for L in layers]
        record(f"w4a16_llama1b_layer_T{T}", calls, [q, gate, up, h], flops,
               wbytes + lin + 3 * 2 * T * inter, PEAK_FP16_TFLOPS, replays=5 if T == 1 else 3,
               check=chk_layer(layers[0], False))
        fused = [fuse_gate_up(L) for L in layers]
        del layers, calls
        calls = [lambda L=L: step_fused(L) for L in fused]
        lin_f = lin - 2 * (2 * T * hid + 2 * T * inter) + (2 * T * hid + 2 * T * inter)
        record(f"w4a16_llama1b_layer_fused_T{T}", calls, [q, h], flops, wbytes + lin_f,
               PEAK_FP16_TFLOPS, replays=5 if T == 1 else 3, check=chk_layer(fused[0], True))
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

        def chk_mlp(w, o, T=T):
            rows = pick_rows(T)

            def f():
                xr = host(x)[rows]
                g_ = oracle.gemm_fp16_f64(xr, host(w[0])).astype(np.float16)
                u_ = oracle.gemm_fp16_f64(xr, host(w[1])).astype(np.float16)
                return tol(host(o)[rows], oracle.swiglu(g_, u_).astype(np.float64))
            return f
        calls = [lambda w=w, o=o, T=T: cg.swiglu_fused(x, w[0], w[1], o, T, H, I) for w, o in zip(pairs, outs)]
        record(f"fp16_llama1b_mlp_swiglu_fused_T{T}", calls, outs, flops, wb + 2 * T * H + 2 * T * I,
               PEAK_FP16_TFLOPS, check=chk_mlp(pairs[0], outs[0]))
        gate = torch.empty(T, I, dtype=torch.float16, device="cuda")
        up = torch.empty_like(gate)

        def unfused(w, o, T=T):
            cg.gemm_fp16(x, w[0], gate, T, I, H)
            cg.gemm_fp16(x, w[1], up, T, I, H)
            cg.swiglu(gate, up, o, T * I)
        calls = [lambda w=w, o=o: unfused(w, o) for w, o in zip(pairs, outs)]
        record(f"fp16_llama1b_mlp_unfused_T{T}", calls, outs, flops,
               wb + 2 * 2 * T * H + 3 * 2 * 2 * T * I, PEAK_FP16_TFLOPS, check=chk_mlp(pairs[0], outs[0]))
        del pairs, outs, calls

    # ---- large prefill MLP (T = 2048, hidden 4096, intermediate 11008): where
    # gemm_fp16 takes its 256x256 tile, swiglu_fused runs the two GEMMs and
    # swiglu; fused and unfused side by side ----
    T, H, I = 2048, 4096, 11008
    x = f16((T, H), 1.0, 970)
    w = (f16((H, I), 0.02, 971), f16((H, I), 0.02, 972))
    o = torch.empty(T, I, dtype=torch.float16, device="cuda")
    gate = torch.empty(T, I, dtype=torch.float16, device="cuda")
    up = torch.empty_like(gate)
    flops = 2 * 2 * T * H * I
    nb = 2 * H * I * 2 + 2 * T * H + 2 * T * I

    def chk_big():
        rows = pick_rows(T)
        xr = host(x)[rows]
        g_ = oracle.gemm_fp16_f64(xr, host(w[0])).astype(np.float16)
        u_ = oracle.gemm_fp16_f64(xr, host(w[1])).astype(np.float16)
        return tol(host(o)[rows], oracle.swiglu(g_, u_).astype(np.float64))
    record("fp16_mlp_swiglu_fused_2048x4096x11008", [lambda: cg.swiglu_fused(x, w[0], w[1], o, T, H, I)] * 4,
           [o], flops, nb, PEAK_FP16_TFLOPS, replays=3, check=chk_big)

    def unfused_big():
        cg.gemm_fp16(x, w[0], gate, T, I, H)
        cg.gemm_fp16(x, w[1], up, T, I, H)
        cg.swiglu(gate, up, o, T * I)
    record("fp16_mlp_unfused_2048x4096x11008", [unfused_big] * 4, [o], flops, nb + 3 * 2 * 2 * T * I,
           PEAK_FP16_TFLOPS, replays=3, check=chk_big)
    del x, w, o, gate, up
    return out


def floor():
    """Cold read floor: a read-only streaming kernel (16-byte lane-contiguous
    loads, 32 KB per workgroup) over the weight sizes of the decode and
    memory-bound shapes, each timed as graph replays that rotate through
    >= 512 MiB of copies (no replay finds its bytes in the 256 MB Infinity
    Cache), and hot (one copy replayed)."""
    import ctypes

    import torch
    lib = diag_lib()
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
        # the second design: persistent workgroups over contiguous slices
        lib.clove_diag_stream_read_persistent.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lib.clove_diag_stream_read_persistent.restype = ctypes.c_int
        for grid, depth in ((256, 4), (256, 8), (512, 4), (512, 8)):
            def pcall(b, grid=grid, depth=depth):
                stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                if lib.clove_diag_stream_read_persistent(b.data_ptr(), nbytes, grid, depth, sink.data_ptr(),
                                                         stream) != grid:
                    raise RuntimeError("clove_diag_stream_read_persistent failed")
            pcalls = [lambda b=b: pcall(b) for b in bufs]
            pus = graph_time(pcalls, [], 5)
            phot = graph_time(pcalls[:1] * 16, [], 5)
            out[f"{name}_persistent_{grid}x1024_{16 * depth}KB"] = {
                "us_cold": round(pus, 3), "GBs_cold": round(nbytes / pus / 1e3, 1), "us_hot": round(phot, 3),
                "GBs_hot": round(nbytes / phot / 1e3, 1)}
            print(f"[floor] {name} persistent {grid} x 1024, {16 * depth} KB in flight: cold {pus:.2f} us, "
                  f"hot {phot:.2f} us", file=sys.stderr, flush=True)
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
              "multi-GPU component (each call runs on one GPU). Run with --gpus 1.", file=sys.stderr)
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
    if args.phases:
        phases(args, Timer())
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
    # the clock the headline ran at, and its fraction of the dense peak at that
    # clock (256 CUs x 4096 flop/clk x the measured shader clock)
    clk = measure_sclk(h, max(args.steps, 20))
    if clk is not None:
        line["device"]["sclk_mhz_measured"] = clk
        line["device"]["sclk_method"] = ("s_memtime / s_memrealtime probe wave after each of the headline "
                                         "GEMM's launches (libclove_diag.so clove_diag_sclk)")
        peak_at = 256 * 4096 * clk["median"] * 1e6 / 1e12
        line["roofline"]["peak_at_measured_sclk"] = round(peak_at, 1)
        line["roofline"]["frac_at_measured_sclk"] = round(achieved / peak_at, 4)
    if args.compare_lib:
        line["library_comparison"] = compare_library(h, timer, args.steps, args.warmup)
    if not args.skip_extra:
        line["shapes"] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                          for k, v in extras(args.compare_lib).items()}
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
