"""Python mirror of the reference GEMM API (include/clove/kernels/gemm.cuh:41-101).

Same function names, argument order and defaults as the reference's C++ API;
buffers are torch tensors on a HIP device (or raw device addresses as int).
Every call goes through the C ABI of libclove_gemm.so and is asynchronous on
``stream`` (default: torch's current stream).  Where the reference prints the
error and exits (include/clove/common.cuh:11-21), these raise CloveError.
"""
from __future__ import annotations

from typing import Optional, Union

from . import _lib

INT4_GROUP_SIZE = 128  # include/clove/kernels/gemm.cuh:72

Buffer = Union["torch.Tensor", int, None]  # noqa: F821


def _ptr(x: Buffer) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if not x.is_cuda:
        raise ValueError("clove GEMM buffers must live on the GPU")
    if not x.is_contiguous():
        raise ValueError("clove GEMM buffers must be contiguous row-major")
    return x.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def gemm_fp16(A, B, C, M: int, N: int, K: int, alpha: float = 1.0, beta: float = 0.0,
              stream=None) -> None:
    """C = alpha * A @ B + beta * C (fp16, fp32 accumulate)."""
    _lib.check(_lib.lib().clove_gemm_fp16(_ptr(A), _ptr(B), _ptr(C), M, N, K, alpha, beta,
                                          _stream(stream)), "gemm_fp16")


def gemm_fp16_noalloc(A, B, C, M: int, N: int, K: int, alpha: float = 1.0, beta: float = 0.0,
                      stream=None) -> None:
    """gemm_fp16 that allocates nothing: split-K scratch from the library's fixed
    per-GPU array (CLOVE_NOALLOC_SCRATCH_BYTES); raises CloveError with
    CLOVE_ERR_SCRATCH_LIMIT when the call needs more.  Calls that overlap on one
    GPU share the array and must be serialised by the caller."""
    _lib.check(_lib.lib().clove_gemm_fp16_noalloc(_ptr(A), _ptr(B), _ptr(C), M, N, K, alpha, beta,
                                                  _stream(stream)), "gemm_fp16_noalloc")


def gemm_fp16_batched(A, B, C, batch: int, M: int, N: int, K: int, alpha: float = 1.0,
                      beta: float = 0.0, stream=None) -> None:
    _lib.check(_lib.lib().clove_gemm_fp16_batched(_ptr(A), _ptr(B), _ptr(C), batch, M, N, K,
                                                  alpha, beta, _stream(stream)),
               "gemm_fp16_batched")


def gemm_int8(A_q, B_q, C, M: int, N: int, K: int, A_scale: float, A_zero: int,
              B_scale: float, B_zero: int, stream=None) -> None:
    """C = fp16(float(sum (a - za)(b - zb)) * (A_scale * B_scale))."""
    _lib.check(_lib.lib().clove_gemm_int8(_ptr(A_q), _ptr(B_q), _ptr(C), M, N, K, A_scale,
                                          A_zero, B_scale, B_zero, _stream(stream)),
               "gemm_int8")


def gemm_int8_ex(A_q, B_q, C, M: int, N: int, K: int, A_scale: float, A_zero: int,
                 B_scale: float, B_zero: int, mode: int = 0, stream=None) -> None:
    """gemm_int8 with an arithmetic mode: CLOVE_INT8_EXACT (0), or
    CLOVE_INT8_REFERENCE_LITERAL (1), the reference kernel's accumulator at any K
    (each zero-padded k of its last 32-wide K tile adds A_zero * B_zero)."""
    _lib.check(_lib.lib().clove_gemm_int8_ex(_ptr(A_q), _ptr(B_q), _ptr(C), M, N, K, A_scale,
                                             A_zero, B_scale, B_zero, mode, _stream(stream)),
               "gemm_int8_ex")


def gemm_int8_rowcol(A_q, B_q, A_scale, B_scale, C, M: int, N: int, K: int,
                     A_zero: int = 0, B_zero: int = 0, stream=None) -> None:
    _lib.check(_lib.lib().clove_gemm_int8_rowcol(_ptr(A_q), _ptr(B_q), _ptr(A_scale),
                                                 _ptr(B_scale), _ptr(C), M, N, K, A_zero,
                                                 B_zero, _stream(stream)), "gemm_int8_rowcol")


def gemm_int8_acc32(A_q, B_q, acc, M: int, N: int, K: int, A_zero: int = 0, B_zero: int = 0,
                    stream=None) -> None:
    _lib.check(_lib.lib().clove_gemm_int8_acc32(_ptr(A_q), _ptr(B_q), _ptr(acc), M, N, K,
                                                A_zero, B_zero, _stream(stream)),
               "gemm_int8_acc32")


def gemm_int4(A_q, A_scale, A_zero, B_q, B_scale, B_zero, C, M: int, N: int, K: int,
              stream=None) -> None:
    """Group-wise W4A4 (group 128 along K); layouts as in include/clove/gemm_c.h."""
    _lib.check(_lib.lib().clove_gemm_int4(_ptr(A_q), _ptr(A_scale), _ptr(A_zero), _ptr(B_q),
                                          _ptr(B_scale), _ptr(B_zero), _ptr(C), M, N, K,
                                          _stream(stream)), "gemm_int4")


def gemm_int4_group_acc32(A_q, A_zero, B_q, B_zero, P, M: int, N: int, K: int, stream=None) -> None:
    """Test hook: the per-group int32 partials P [M, N, K // 128] of group-wise INT4."""
    _lib.check(_lib.lib().clove_gemm_int4_group_acc32(_ptr(A_q), _ptr(A_zero), _ptr(B_q), _ptr(B_zero),
                                                      _ptr(P), M, N, K, _stream(stream)),
               "gemm_int4_group_acc32")


def gemm_int4_ex(A_q, A_scale, A_zero, B_q, B_scale, B_zero, C, M: int, N: int, K: int,
                 mode: int = _lib.CLOVE_INT4_GROUPWISE, stream=None) -> None:
    _lib.check(_lib.lib().clove_gemm_int4_ex(_ptr(A_q), _ptr(A_scale), _ptr(A_zero),
                                             _ptr(B_q), _ptr(B_scale), _ptr(B_zero), _ptr(C),
                                             M, N, K, mode, _stream(stream)), "gemm_int4_ex")


def gemm_w4a16(X, W_q, W_scale, W_zero, Y, T: int, O: int, K: int, alpha: float = 1.0,
               beta: float = 0.0, stream=None) -> None:
    """Y = alpha * X @ dequant(W)^T + beta * Y with group-128 INT4 weights."""
    _lib.check(_lib.lib().clove_gemm_w4a16(_ptr(X), _ptr(W_q), _ptr(W_scale), _ptr(W_zero),
                                           _ptr(Y), T, O, K, alpha, beta, _stream(stream)),
               "gemm_w4a16")


def swiglu(gate, up, output, size: int, stream=None) -> None:
    """output = fp16(silu(gate) * up) elementwise (include/clove/kernels/activations.cuh:25-31);
    output may be gate or up."""
    _lib.check(_lib.lib().clove_swiglu(_ptr(gate), _ptr(up), _ptr(output), size, _stream(stream)),
               "swiglu")


def swiglu_fused(input, W_gate, W_up, output, batch_seq: int, hidden_dim: int,
                 intermediate_dim: int, stream=None) -> None:
    """output = swiglu(input @ W_gate, input @ W_up) on FP16 weights [hidden, intermediate]
    (declared in include/clove/kernels/activations.cuh:37-46)."""
    _lib.check(_lib.lib().clove_swiglu_fused(_ptr(input), _ptr(W_gate), _ptr(W_up), _ptr(output),
                                             batch_seq, hidden_dim, intermediate_dim,
                                             _stream(stream)), "swiglu_fused")


def w4a16_swiglu(X, W_q, W_scale, W_zero, H, T: int, I: int, K: int, stream=None) -> None:
    """H = swiglu(X @ dequant(W[:I])^T, X @ dequant(W[I:2I])^T): the MLP's gate and up
    projections and SwiGLU on one fused INT4 weight [2I, K/2] (gate rows first)."""
    _lib.check(_lib.lib().clove_w4a16_swiglu(_ptr(X), _ptr(W_q), _ptr(W_scale), _ptr(W_zero),
                                             _ptr(H), T, I, K, _stream(stream)), "w4a16_swiglu")


def workspace_bind(workspace=None, nbytes: int = 0) -> None:
    """Bind a caller-owned workspace (a device tensor or pointer; 256-byte aligned, its first
    CLOVE_WORKSPACE_MIN_BYTES zero) to the calling thread; ``workspace_bind()`` unbinds."""
    if workspace is not None and not isinstance(workspace, int) and nbytes == 0:
        nbytes = workspace.numel() * workspace.element_size()
    _lib.check(_lib.lib().clove_workspace_bind(_ptr(workspace), nbytes), "workspace_bind")


class workspace_query:
    """``with workspace_query() as q: <calls>`` plans the calls without launching them;
    ``q.bytes`` is then the largest workspace any of them needs (0: none)."""

    def __enter__(self):
        _lib.check(_lib.lib().clove_workspace_query_begin(), "workspace_query_begin")
        self.bytes = 0
        return self

    def __exit__(self, *exc):
        self.bytes = int(_lib.lib().clove_workspace_query_end())
        return False


def release_scratch() -> None:
    _lib.check(_lib.lib().clove_release_scratch(), "release_scratch")
