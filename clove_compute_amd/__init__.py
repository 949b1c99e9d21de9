"""clove_compute_amd -- MI355X (gfx950) GEMM hot path of Clove Compute.

The product is the C ABI library ``lib/libclove_gemm.so`` (declared in
include/clove/gemm_c.h, C++ spelling in include/clove/gemm.h).  This package
is its Python host side: the ctypes binding, a mirror of the reference's
GEMM API over torch device tensors, and the INT4 packing/quantisation helpers.
"""
from ._lib import (  # noqa: F401
    CloveError, CLOVE_ERR_SCRATCH_LIMIT, CLOVE_ERR_WORKSPACE, CLOVE_INT4_GROUPWISE,
    CLOVE_INT4_REFERENCE_LITERAL, CLOVE_INT8_EXACT, CLOVE_INT8_REFERENCE_LITERAL, CLOVE_NOALLOC_SCRATCH_BYTES,
    CLOVE_WORKSPACE_MIN_BYTES,
)
from .gemm import (  # noqa: F401
    INT4_GROUP_SIZE,
    gemm_fp16,
    gemm_fp16_batched,
    gemm_fp16_noalloc,
    gemm_int4,
    gemm_int4_ex,
    gemm_int8,
    gemm_int8_ex,
    gemm_int8_acc32,
    gemm_int4_group_acc32,
    gemm_int8_rowcol,
    gemm_w4a16,
    release_scratch,
    swiglu,
    swiglu_fused,
    w4a16_swiglu,
    workspace_bind,
    workspace_query,
)
from . import quant  # noqa: F401
