"""CPU-side checks of the C ABI (no GPU, no compute calls).

The library must load, export every entry point include/clove/gemm_c.h
declares, and reject bad arguments with the documented status codes before it
touches the GPU.  Pointers here are fake addresses that are never dereferenced.
"""
import os
import re
import subprocess

import pytest

from clove_compute_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "clove", "gemm_c.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clove_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        import clove_compute_amd.build as b
        b.build()
    return _lib.lib()


def test_every_declared_symbol_is_exported(L):
    syms = declared_symbols()
    assert len(syms) >= 11
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(\S+)$", out, flags=re.M))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    # the ctypes binding covers every declared entry point
    assert set(syms) == set(_lib.SIGNATURES)
    for s in syms:
        assert hasattr(L, s)


def test_status_strings_and_version(L):
    assert L.clove_abi_version() == 1
    for code in range(9):
        assert L.clove_status_string(code).decode().startswith("CLOVE_")
    assert b"UNKNOWN" in L.clove_status_string(99)


A, B, C = 0x100000, 0x200000, 0x300000  # fake, 16-byte aligned, disjoint


def test_fp16_validation(L):
    f = L.clove_gemm_fp16
    assert f(A, B, C, -1, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(A, B, C, 4, 4, -4, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(None, B, C, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, None, C, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, B, None, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A + 1, B, C, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, B, A + 8, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_ALIASING
    assert f(A, B, B, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_ALIASING
    # empty products are no-ops that never touch the device
    assert f(A, B, C, 0, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_OK
    assert f(None, None, None, 4, 0, 4, 1.0, 0.0, None) == _lib.CLOVE_OK
    g = L.clove_gemm_fp16_batched
    assert g(A, B, C, -2, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert g(A, B, C, 0, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_OK
    # batch 2 of C overlaps B when B sits right after C's first batch
    assert g(A, C + 32, C, 2, 4, 4, 4, 1.0, 0.0, None) == _lib.CLOVE_ERR_ALIASING


def test_int8_validation(L):
    f = L.clove_gemm_int8
    assert f(A, B, C, 4, -1, 4, 1.0, 0, 1.0, 0, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(None, B, C, 4, 4, 4, 1.0, 0, 1.0, 0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, B, C + 1, 4, 4, 4, 1.0, 0, 1.0, 0, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, B, A, 4, 4, 4, 1.0, 0, 1.0, 0, None) == _lib.CLOVE_ERR_ALIASING
    assert f(A, B, C, 0, 4, 4, 1.0, 0, 1.0, 0, None) == _lib.CLOVE_OK
    r = L.clove_gemm_int8_rowcol
    assert r(A, B, None, 0x400000, C, 4, 4, 4, 0, 0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert r(A, B, 0x400001, 0x400000, C, 4, 4, 4, 0, 0, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert r(A, B, C, 0x400000, C, 4, 4, 4, 0, 0, None) == _lib.CLOVE_ERR_ALIASING
    a = L.clove_gemm_int8_acc32
    assert a(A, B, C + 2, 4, 4, 4, 0, 0, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert a(A, B, None, 4, 4, 4, 0, 0, None) == _lib.CLOVE_ERR_NULL_POINTER


def test_int4_validation(L):
    S, Z, BS, BZ = 0x400000, 0x500000, 0x600000, 0x700000
    f = L.clove_gemm_int4
    assert f(A, S, Z, B, BS, BZ, C, 4, 4, 7, None) == _lib.CLOVE_ERR_INVALID_ARG  # odd K
    assert f(A, S, Z, B, BS, BZ, C, 4, -4, 8, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(A, S, None, B, BS, BZ, C, 4, 4, 8, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, S, Z, B, BS, BZ, S, 4, 4, 8, None) == _lib.CLOVE_ERR_ALIASING
    assert f(A, S + 1, Z, B, BS, BZ, C, 4, 4, 8, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, S, Z, B, BS, BZ, C, 0, 4, 8, None) == _lib.CLOVE_OK
    g = L.clove_gemm_int4_ex
    assert g(A, S, Z, B, BS, BZ, C, 4, 4, 8, 7, None) == _lib.CLOVE_ERR_INVALID_ARG  # bad mode
    # literal mode never reads zeros but needs B when N >= 2 (stride floor(N/2))
    lit = _lib.CLOVE_INT4_REFERENCE_LITERAL
    assert g(A, S, None, None, BS, None, C, 4, 4, 8, lit, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert g(A, S, None, B, BS, None, C, 4, 4, 7, lit, None) == _lib.CLOVE_ERR_INVALID_ARG


def test_int4_group_acc32_validation(L):
    Z, BZ, P = 0x500000, 0x700000, 0x800000
    f = L.clove_gemm_int4_group_acc32
    assert f(A, Z, B, BZ, P, 4, 4, 128, None) == _lib.CLOVE_ERR_INVALID_ARG  # K not a multiple of 256
    assert f(A + 8, Z, B, BZ, P, 4, 4, 256, None) == _lib.CLOVE_ERR_INVALID_ARG  # A not 16-byte aligned
    assert f(A, Z, B, BZ, P + 2, 4, 4, 256, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, Z, B, BZ, P, 4, -4, 256, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(A, None, B, BZ, P, 4, 4, 256, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, Z, B, BZ, None, 4, 4, 256, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, Z, B, BZ, Z, 4, 4, 256, None) == _lib.CLOVE_ERR_ALIASING
    assert f(A, Z, B, BZ, P, 0, 4, 256, None) == _lib.CLOVE_OK


def test_w4a16_validation(L):
    W, S, Z = 0x400000, 0x500000, 0x600000
    f = L.clove_gemm_w4a16
    assert f(A, W, S, Z, C, 4, 4, 9, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, W, S, Z, C, -1, 4, 8, 1.0, 0.0, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(A, W, None, Z, C, 4, 4, 8, 1.0, 0.0, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A, W, S, Z, W, 4, 4, 8, 1.0, 0.0, None) == _lib.CLOVE_ERR_ALIASING
    assert f(A, W, S, Z, C, 0, 4, 8, 1.0, 0.0, None) == _lib.CLOVE_OK


def test_swiglu_validation(L):
    f = L.clove_swiglu
    assert f(A, B, C, -1, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert f(A, B, C, 0, None) == _lib.CLOVE_OK
    assert f(None, B, C, 8, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert f(A + 1, B, C, 8, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert f(A, B, A + 2, 8, None) == _lib.CLOVE_ERR_ALIASING  # shifted against an input
    g = L.clove_swiglu_fused
    assert g(A, B, B, C, 4, -1, 8, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert g(A, B, B, C, 0, 4, 8, None) == _lib.CLOVE_OK
    assert g(A, None, B, C, 4, 4, 8, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert g(A, B, B, B, 4, 4, 8, None) == _lib.CLOVE_ERR_ALIASING
    W, S, Z = 0x400000, 0x500000, 0x600000
    h = L.clove_w4a16_swiglu
    assert h(A, W, S, Z, C, 4, 4, 9, None) == _lib.CLOVE_ERR_INVALID_ARG
    assert h(A, W, S, Z, C, 4, -4, 8, None) == _lib.CLOVE_ERR_INVALID_DIM
    assert h(A, W, S, None, C, 4, 4, 8, None) == _lib.CLOVE_ERR_NULL_POINTER
    assert h(A, W, S, Z, Z, 4, 4, 8, None) == _lib.CLOVE_ERR_ALIASING
    assert h(A, W, S, Z, C, 4, 0, 8, None) == _lib.CLOVE_OK
