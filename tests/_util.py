"""Shared helpers for the GPU parity tests (inputs, tolerance, transfers)."""
from __future__ import annotations

import numpy as np


def rng(*key) -> np.random.Generator:
    """Seeded PCG64 generator per (config, operand) key."""
    seed = np.frombuffer(repr(key).encode(), np.uint8).astype(np.uint64)
    s = int((seed * np.arange(1, seed.size + 1, dtype=np.uint64)).sum() % (2 ** 63))
    return np.random.default_rng(s + 20261201)


def to_dev(a: np.ndarray):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.float16)
    else:
        t = torch.from_numpy(a)
    return t.to("cuda")


def to_host(t) -> np.ndarray:
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.float16)
    return t.numpy()


def empty_f16(*shape, fill=None):
    import torch
    if fill is None:
        return torch.empty(*shape, dtype=torch.float16, device="cuda")
    return torch.full(shape, fill, dtype=torch.float16, device="cuda")


def f16bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def within_tol(got: np.ndarray, ref64: np.ndarray, rel: float = 1e-2):
    """Elementwise |got - ref| <= rel * max(|ref|, 1e-2 * rms(ref)).

    Returns (ok, report) with the max relative error, the normwise error and the
    reference test's own rule (fail iff rel_err > 0.05 and abs_err > 1e-3,
    tests/test_gemm.cu:22-58) for continuity."""
    g = got.astype(np.float64)
    r = np.asarray(ref64, np.float64)
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    floor = max(1e-2 * rms, 1e-30)
    err = np.abs(g - r)
    bound = rel * np.maximum(np.abs(r), floor)
    ok = bool(np.all(err <= bound)) and bool(np.all(np.isfinite(g)))
    ref_rule_fail = int(np.sum((err / (np.abs(r) + 1e-3) > 0.05) & (err > 1e-3)))
    report = {
        "max_rel_err_floored": float(np.max(err / np.maximum(np.abs(r), floor))) if r.size else 0.0,
        "normwise": float(np.max(err) / max(np.max(np.abs(r)), 1e-30)) if r.size else 0.0,
        "ref_rule_failures": ref_rule_fail,
    }
    return ok, report
