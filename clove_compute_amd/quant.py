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

On disk, INT4 linear weights are SafeTensors files (save_int4_linear /
load_int4_linear / quantize_linear_file below).
"""
from __future__ import annotations

import json as _json
import struct as _struct

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


# ---------------------------------------------------------------------------
# On-disk format: SafeTensors (8-byte little-endian header length, a JSON
# header {name: {"dtype", "shape", "data_offsets": [begin, end]}, optional
# "__metadata__": {str: str}}, then the raw little-endian tensor bytes).  The
# reference's loader (src/runtime/model_loader.cpp:57-91) reads the header
# length and stops; this reader parses the header and the tensors.
#
# An INT4 linear weight `name` is three tensors:
#   name.qweight  U8  [out, in/2]   two nibbles per byte, even k in the high nibble
#   name.scales   F16 [out, in/128] group scales
#   name.zeros    F16 [out, in/128] group zero points (integers 0..15)
# and the file's metadata records {"clove.format": "int4-g128-rows"}.
# ---------------------------------------------------------------------------


_ST_DTYPES = {"U8": np.uint8, "I8": np.int8, "F16": np.float16, "F32": np.float32, "I32": np.int32,
              "I64": np.int64, "F64": np.float64, "U16": np.uint16, "I16": np.int16, "BOOL": np.bool_}
_ST_NAMES = {np.dtype(v).str: k for k, v in _ST_DTYPES.items()}
INT4_FORMAT = "int4-g128-rows"


def save_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Writes {name: numpy array} (tensors sorted by name, data 8-byte aligned)."""
    header = {}
    offset = 0
    blobs = []
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        if a.dtype.str not in _ST_NAMES:
            raise ValueError(f"{name}: dtype {a.dtype} has no SafeTensors name here")
        b = a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": _ST_NAMES[a.dtype.str], "shape": list(a.shape),
                        "data_offsets": [offset, offset + len(b)]}
        blobs.append(b)
        offset += len(b)
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = _json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)  # keep the data 8-byte aligned
    with open(path, "wb") as f:
        f.write(_struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def read_safetensors_header(path: str):
    """Returns (header dict without __metadata__, metadata dict, data start offset)."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError("not a SafeTensors file (short header length)")
        n = _struct.unpack("<Q", raw)[0]
        if n > 100 << 20:
            raise ValueError("SafeTensors header longer than 100 MiB")
        header = _json.loads(f.read(n))
    meta = header.pop("__metadata__", {}) or {}
    return header, meta, 8 + n


def load_safetensors(path: str, names=None) -> dict:
    """Memory-maps the file and returns {name: numpy array} (read-only views)."""
    header, _, start = read_safetensors_header(path)
    mm = np.memmap(path, np.uint8, mode="r")
    out = {}
    for name, info in header.items():
        if names is not None and name not in names:
            continue
        dt = info["dtype"]
        if dt not in _ST_DTYPES:
            raise ValueError(f"{name}: unsupported dtype {dt}")
        b, e = info["data_offsets"]
        a = mm[start + b:start + e].view(_ST_DTYPES[dt])
        out[name] = a.reshape(info["shape"])
    return out


def save_int4_linear(path: str, weights: dict) -> None:
    """weights: {name: (qweight [out, in/2] uint8, scales [out, G] fp16, zeros [out, G] fp16)}."""
    t = {}
    for name, (q, s, z) in weights.items():
        q = np.asarray(q, np.uint8)
        s = np.asarray(s, np.float16)
        z = np.asarray(z, np.float16)
        if s.shape != z.shape or s.shape[0] != q.shape[0] or s.shape[1] != _groups(2 * q.shape[1]):
            raise ValueError(f"{name}: qweight {q.shape}, scales {s.shape}, zeros {z.shape} disagree")
        t[name + ".qweight"], t[name + ".scales"], t[name + ".zeros"] = q, s, z
    save_safetensors(path, t, {"clove.format": INT4_FORMAT})


def load_int4_linear(path: str) -> dict:
    """{name: (qweight, scales, zeros)} of a file written by save_int4_linear."""
    header, meta, _ = read_safetensors_header(path)
    if meta.get("clove.format") != INT4_FORMAT:
        raise ValueError(f"{path}: not an {INT4_FORMAT} file (metadata {meta})")
    arrays = load_safetensors(path)
    out = {}
    for key in header:
        if key.endswith(".qweight"):
            name = key[: -len(".qweight")]
            q, s, z = arrays[key], arrays[name + ".scales"], arrays[name + ".zeros"]
            if q.dtype != np.uint8 or s.dtype != np.float16 or z.dtype != np.float16:
                raise ValueError(f"{name}: wrong dtypes")
            out[name] = (q, s, z)
    return out


def quantize_linear_file(src: str, dst: str, names=None) -> list:
    """Reads fp16 / fp32 [out, in] linear weights from a SafeTensors file,
    quantises them group-wise (quantize_rows) and writes them with
    save_int4_linear.  Returns the names converted."""
    arrays = load_safetensors(src, names)
    done = {}
    for name, w in arrays.items():
        if w.ndim != 2 or w.dtype not in (np.float16, np.float32) or w.shape[1] % 2:
            continue
        done[name] = quantize_rows(np.asarray(w, np.float32))
    save_int4_linear(dst, done)
    return sorted(done)
