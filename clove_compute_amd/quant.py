"""INT4 weight/activation packing and group-wise quantisation (host side, numpy).

Byte layouts follow the reference kernel (src/kernels/gemm_int4.cu:27-34,
:88-92, :105-112): two nibbles per byte, the EVEN index in the HIGH nibble.

* rows  [R, K] nibbles -> [R, K/2]        (gemm_int4's A_q; W4A16 weights)
* cols  [K, N] nibbles -> [K, ceil(N/2)]  (gemm_int4's B_q; the pad nibble of
  an odd N is zero)

Group-wise quantisation (group 128 along K, asymmetric, unsigned 4-bit):
  scale = (max - min) / 15,  zero = round(-min / scale) clamped to [0, 15],
  q = clamp(round(x / scale) + zero, 0, 15),   x ~= (q - zero) * scale
Scales and zeros are stored as fp16 ([R, G] for rows, [G, N] for columns).
"""
from __future__ import annotations

import numpy as np

GROUP = 128


def pack_rows(q: np.ndarray) -> np.ndarray:
    """[R, K] values 0..15 -> [R, K/2] uint8, even k in the high nibble."""
    q = np.asarray(q)
    if q.shape[1] % 2:
        raise ValueError("K must be even to pack along rows")
    q = q.astype(np.uint8)
    return ((q[:, 0::2] << 4) | (q[:, 1::2] & 0x0F)).astype(np.uint8)


def unpack_rows(p: np.ndarray, K: int) -> np.ndarray:
    p = np.asarray(p, np.uint8)
    out = np.empty((p.shape[0], K), np.uint8)
    out[:, 0::2] = p[:, : K // 2] >> 4
    out[:, 1::2] = p[:, : K // 2] & 0x0F
    return out


def pack_cols(q: np.ndarray) -> np.ndarray:
    """[K, N] values 0..15 -> [K, ceil(N/2)] uint8, even n in the high nibble."""
    q = np.asarray(q).astype(np.uint8)
    K, N = q.shape
    if N % 2:
        q = np.concatenate([q, np.zeros((K, 1), np.uint8)], axis=1)
    return ((q[:, 0::2] << 4) | (q[:, 1::2] & 0x0F)).astype(np.uint8)


def unpack_cols(p: np.ndarray, N: int) -> np.ndarray:
    p = np.asarray(p, np.uint8)
    out = np.empty((p.shape[0], 2 * p.shape[1]), np.uint8)
    out[:, 0::2] = p >> 4
    out[:, 1::2] = p & 0x0F
    return out[:, :N]


def _groups(K: int) -> int:
    return (K + GROUP - 1) // GROUP


def quantize_rows(x: np.ndarray):
    """Quantise [R, K] floats group-wise along K.

    Returns (packed [R, K/2] uint8, scale [R, G] fp16, zero [R, G] fp16)."""
    x = np.asarray(x, np.float32)
    R, K = x.shape
    G = _groups(K)
    pad = G * GROUP - K
    xp = np.pad(x, ((0, 0), (0, pad)), mode="edge").reshape(R, G, GROUP)
    lo = np.minimum(xp.min(axis=2), 0.0)
    hi = np.maximum(xp.max(axis=2), 0.0)
    scale = ((hi - lo) / 15.0).astype(np.float16)
    s32 = scale.astype(np.float32)
    s32 = np.where(s32 == 0, 1.0, s32)
    zero = np.clip(np.rint(-lo / s32), 0, 15).astype(np.float16)
    q = np.clip(np.rint(xp / s32[:, :, None]) + zero.astype(np.float32)[:, :, None], 0, 15)
    q = q.reshape(R, G * GROUP)[:, :K].astype(np.uint8)
    return pack_rows(q), scale, zero


def quantize_cols(x: np.ndarray):
    """Quantise [K, N] floats group-wise along K (per column).

    Returns (packed [K, ceil(N/2)] uint8, scale [G, N] fp16, zero [G, N] fp16)."""
    packed_t, scale_t, zero_t = quantize_rows(np.asarray(x, np.float32).T)
    K = x.shape[0]
    q = unpack_rows(packed_t, K).T
    return pack_cols(q), np.ascontiguousarray(scale_t.T), np.ascontiguousarray(zero_t.T)


def dequantize_rows(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray, K: int) -> np.ndarray:
    """[R, K/2] + [R, G] scales/zeros -> float64 [R, K] = (q - rint(zero)) * scale."""
    q = unpack_rows(packed, K).astype(np.float64)
    g = np.arange(K) // GROUP
    s = np.asarray(scale, np.float16).astype(np.float64)[:, g]
    z = np.rint(np.asarray(zero, np.float16).astype(np.float64))[:, g]
    return (q - z) * s
