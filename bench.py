#!/usr/bin/env python3
"""Benchmark of the Clove Compute GEMM hot path on one MI355X.

Headline workload (the step): one FP16 GEMM C = A @ B at M = N = K = 4096,
row-major, A ~ N(0,1) activations and B ~ N(0,0.02) weights from a fixed
seed, fp32 accumulation, fp16 output, through the C ABI (clove_gemm_fp16).
`value` is TFLOP/s = 2*M*N*K / (time per step), inputs resident in HBM, W
untimed warm-up steps then exactly K timed steps between device syncs.

The same JSON line also carries:
  roofline      the dominant kernel against MI355X dense FP16 MFMA peak
  cpu_baseline  the oracle's restatement of the reference's naive GEMM
                (fp32 sequential-k FMA), single thread, on a bounded row sample
  decode        the HBM-bound decode shapes (FP16 1x4096x4096, INT4 W4A4
                4096x11008 N=1, INT8 1x4096x4096, W4A16 Llama-1B layer at T=1),
                timed cold: operands rotate through >= 512 MiB of copies so no
                call finds its operands in the 256 MB Infinity Cache
  prefill       MFMA-bound companions (INT4 N=128, W4A16 layer at T=512)

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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bound on the CPU-baseline sample (0 disables it)")
    ap.add_argument("--skip-extra", action="store_true", help="headline only")
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
    return dict(ms=ms, tflops=tflops, A=A_h, B=B_h, C=C)


def cpu_baseline(h, seconds):
    """Times the oracle's naive-arithmetic FP16 GEMM on rows of the same
    4096^3 problem, 64 rows at a time until `seconds` have passed."""
    import numpy as np

    import oracle
    from tests._util import to_host, within_tol

    A, B = h["A"], h["B"]
    M, K = A.shape
    N = B.shape[1]
    out = np.zeros((M, N), np.float16)
    rows = 0
    t0 = time.perf_counter()
    while rows < M and time.perf_counter() - t0 < seconds:
        r1 = min(M, rows + 64)
        out[rows:r1] = oracle.gemm_fp16(A[rows:r1], B)
        rows = r1
    dt = time.perf_counter() - t0
    # the sampled rows double as a parity check of the timed GPU output
    r8 = min(rows, 8)
    ok, _ = within_tol(to_host(h["C"])[:r8], oracle.gemm_fp16_f64(A[:r8], B))
    return dict(value=2.0 * rows * N * K / dt / 1e12, unit="TFLOP/s", cores=1, kind="port",
                sample=f"rows 0..{rows - 1} of the 4096x4096x4096 FP16 GEMM ({rows} rows, "
                       f"{dt:.1f} s), single thread, oracle/clove_oracle.c restatement of "
                       f"gemm_fp16_naive_kernel",
                parity_rows_ok=bool(ok))


def rotating(make, nbytes_each, min_total=512 << 20):
    copies = max(2, -(-min_total // max(1, nbytes_each)))
    return [make(i) for i in range(copies)]


def extras(args, timer):
    import torch

    import clove_compute_amd as cg

    res = {}
    gen = torch.Generator(device="cuda")
    steps, warm = max(args.steps, 100), max(args.warmup, 10)

    def f16(shape, scale, seed):
        gen.manual_seed(seed)
        return (torch.randn(shape, generator=gen, device="cuda") * scale).half()

    def u8(shape, seed, hi=256):
        gen.manual_seed(seed)
        return torch.randint(0, hi, shape, generator=gen, device="cuda", dtype=torch.uint8)

    def uni16(shape, lo, hi, seed):
        gen.manual_seed(seed)
        return (torch.rand(shape, generator=gen, device="cuda") * (hi - lo) + lo).half()

    def zeros16(shape, seed):
        gen.manual_seed(seed)
        return torch.randint(0, 16, shape, generator=gen, device="cuda").half()

    # FP16 decode 1x4096x4096 (B is the 32 MiB weight)
    M, N, K = 1, 4096, 4096
    x = f16((M, K), 1.0, 1)
    Bs = rotating(lambda i: f16((K, N), 0.02, 100 + i), K * N * 2)
    C = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ms = timer.run(lambda i: cg.gemm_fp16(x, Bs[i % len(Bs)], C, M, N, K), steps, warm)
    by = 2 * (M * K + K * N + M * N)
    res["fp16_1x4096x4096"] = dict(us=ms * 1e3, GBs=by / ms / 1e6, frac_hbm=by / ms / 1e6 / PEAK_HBM_GBS,
                                   TFLOPs=2 * M * N * K / ms / 1e9)
    hot = timer.run(lambda i: cg.gemm_fp16(x, Bs[0], C, M, N, K), steps, warm)
    res["fp16_1x4096x4096"]["us_hot_cache"] = hot * 1e3
    del Bs

    # INT4 W4A4 decode: A_q [4096, 11008/2], N = 1
    for (M, K) in ((4096, 11008), (11008, 4096)):
        N, G = 1, -(-K // 128)
        sets = rotating(lambda i: (u8((M, K // 2), 200 + i), uni16((M, G), 0.001, 0.02, 300 + i),
                                   zeros16((M, G), 400 + i)), M * K // 2 + 4 * M * G)
        Bq = u8((K, 1), 5, 16) << 4
        Bsc = uni16((G, N), 0.001, 0.02, 6)
        Bz = zeros16((G, N), 7)
        C = torch.empty(M, N, dtype=torch.float16, device="cuda")
        ms = timer.run(lambda i: cg.gemm_int4(*sets[i % len(sets)], Bq, Bsc, Bz, C, M, N, K), steps, warm)
        by = M * K // 2 + 4 * M * G + K * 1 + 4 * G * N + 2 * M * N
        res[f"int4_w4a4_{M}x{K}_n1"] = dict(us=ms * 1e3, GBs=by / ms / 1e6,
                                             frac_hbm=by / ms / 1e6 / PEAK_HBM_GBS)
        hot = timer.run(lambda i: cg.gemm_int4(sets[0][0], sets[0][1], sets[0][2], Bq, Bsc, Bz, C, M, N, K),
                        steps, warm)
        res[f"int4_w4a4_{M}x{K}_n1"]["us_hot_cache"] = hot * 1e3
        del sets

    # INT8 W8A8 decode 1x4096x4096 with per-row / per-column scales
    M, N, K = 1, 4096, 4096
    a8 = u8((M, K), 8).view(torch.int8)
    Bs = rotating(lambda i: u8((K, N), 500 + i).view(torch.int8), K * N)
    sa = uni16((M,), 0.001, 0.02, 9)
    sb = uni16((N,), 0.001, 0.02, 10)
    C = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ms = timer.run(lambda i: cg.gemm_int8_rowcol(a8, Bs[i % len(Bs)], sa, sb, C, M, N, K), steps, warm)
    by = M * K + K * N + 2 * M * N + 2 * M + 2 * N
    res["int8_1x4096x4096"] = dict(us=ms * 1e3, GBs=by / ms / 1e6, frac_hbm=by / ms / 1e6 / PEAK_HBM_GBS)
    del Bs

    # W4A16 Llama-1B decoder-layer GEMM sequence (QKV, O+res, gate, up, down+res)
    layer = [(3072, 2048, 0.0), (2048, 2048, 1.0), (8192, 2048, 0.0), (8192, 2048, 0.0),
             (2048, 8192, 1.0)]

    def make_layer(i):
        return [(u8((O, K // 2), 600 + 10 * i + j), uni16((O, -(-K // 128)), 0.001, 0.02, 700 + 10 * i + j),
                 zeros16((O, -(-K // 128)), 800 + 10 * i + j)) for j, (O, K, _) in enumerate(layer)]

    wbytes = sum(O * K // 2 + 4 * O * (-(-K // 128)) for O, K, _ in layer)
    for T in (1, 512):
        layers = rotating(make_layer, wbytes) if T == 1 else [make_layer(0)]
        xs = [f16((T, K), 1.0, 900 + j) for j, (O, K, _) in enumerate(layer)]
        ys = [f16((T, O), 1.0, 950 + j) for j, (O, K, _) in enumerate(layer)]

        def step(i, layers=layers, xs=xs, ys=ys, T=T):
            L = layers[i % len(layers)]
            for j, (O, K, beta) in enumerate(layer):
                w, s, z = L[j]
                cg.gemm_w4a16(xs[j], w, s, z, ys[j], T, O, K, 1.0, beta)

        ms = timer.run(step, steps if T == 1 else max(20, args.steps // 2), warm)
        flops = sum(2 * T * O * K for O, K, _ in layer)
        by = wbytes + sum(2 * T * K + 2 * T * O * (2 if b else 1) for O, K, b in layer)
        key = f"w4a16_llama1b_layer_T{T}"
        res[key] = dict(us=ms * 1e3, TFLOPs=flops / ms / 1e9, GBs=by / ms / 1e6,
                        frac_hbm=by / ms / 1e6 / PEAK_HBM_GBS, frac_mfma=flops / ms / 1e9 / PEAK_FP16_TFLOPS)
        del layers

    # INT4 W4A4 N=128 (MFMA side of config 4)
    M, N, K = 4096, 128, 11008
    G = -(-K // 128)
    Aq, As, Az = u8((M, K // 2), 11), uni16((M, G), 0.001, 0.02, 12), zeros16((M, G), 13)
    Bq, Bsc, Bz = u8((K, N // 2), 14), uni16((G, N), 0.001, 0.02, 15), zeros16((G, N), 16)
    C = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ms = timer.run(lambda i: cg.gemm_int4(Aq, As, Az, Bq, Bsc, Bz, C, M, N, K), steps, warm)
    by = M * K // 2 + 4 * M * G + K * N // 2 + 4 * G * N + 2 * M * N
    res["int4_w4a4_4096x11008_n128"] = dict(us=ms * 1e3, TFLOPs=2 * M * N * K / ms / 1e9, GBs=by / ms / 1e6,
                                            frac_hbm=by / ms / 1e6 / PEAK_HBM_GBS)
    return res


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

    timer = Timer()
    h = headline(args, timer)
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
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic, "flops_per_launch": flops},
    }
    if not args.skip_extra:
        ex = extras(args, timer)
        line["decode"] = {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in ex.items()
                          if "n128" not in k and "T512" not in k}
        line["prefill"] = {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in ex.items()
                           if "n128" in k or "T512" in k}
    if args.cpu_seconds > 0:
        cb = cpu_baseline(h, args.cpu_seconds)
        cb["value"] = round(cb["value"], 6)
        line["cpu_baseline"] = cb
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
