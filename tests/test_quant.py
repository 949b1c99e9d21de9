"""INT4 packing, group-wise quantisation and the SafeTensors weight format (CPU).

The nibble order and group size are the reference's (src/kernels/gemm_int4.cu:27-34:
even index in the high nibble; include/clove/kernels/gemm.cuh:72: groups of 128).
The SafeTensors reader/writer is checked against the `safetensors` package in
both directions, which pins the file format independently of this code.
"""
import os

import numpy as np
import pytest

from clove_compute_amd import quant

RNG = np.random.default_rng(20261202)


def test_pack_rows_nibble_order_and_round_trip():
    q = np.array([[1, 2, 3, 4, 15, 0]], np.uint8)
    p = quant.pack_rows(q)
    assert p.tolist() == [[0x12, 0x34, 0xF0]]  # even k high
    big = RNG.integers(0, 16, (7, 256)).astype(np.uint8)
    assert np.array_equal(quant.unpack_rows(quant.pack_rows(big), 256), big)
    with pytest.raises(ValueError):
        quant.pack_rows(np.zeros((2, 3), np.uint8))


def test_pack_cols_odd_n_pads_low_nibble():
    q = np.array([[1, 2, 3], [4, 5, 6]], np.uint8)
    p = quant.pack_cols(q)
    assert p.tolist() == [[0x12, 0x30], [0x45, 0x60]]
    assert np.array_equal(quant.unpack_cols(p, 3), q)


def test_quantize_rows_error_bound():
    W = RNG.standard_normal((16, 384)).astype(np.float32)
    q, s, z = quant.quantize_rows(W)
    deq = quant.dequantize_rows(q, s, z, 384)
    # asymmetric 4-bit: |w - deq| <= scale / 2 (+ fp16 rounding of the scale)
    g = np.arange(384) // 128
    bound = s.astype(np.float64)[:, g] * 0.5 * (1 + 2 ** -9) + 1e-6
    assert np.all(np.abs(W - deq) <= bound + np.abs(W) * 2e-3)
    assert np.all((z >= 0) & (z <= 15)) and np.all(z == np.rint(z))


def test_safetensors_round_trip_and_header(tmp_path):
    t = {"a": RNG.standard_normal((3, 5)).astype(np.float32),
         "b.qweight": RNG.integers(0, 256, (4, 64)).astype(np.uint8),
         "b.scales": RNG.standard_normal((4, 1)).astype(np.float16),
         "c": np.arange(7, dtype=np.int64)}
    p = str(tmp_path / "x.safetensors")
    quant.save_safetensors(p, t, {"k": "v"})
    header, meta, start = quant.read_safetensors_header(p)
    assert meta == {"k": "v"} and start % 8 == 0
    assert header["a"]["dtype"] == "F32" and header["a"]["shape"] == [3, 5]
    back = quant.load_safetensors(p)
    for k, v in t.items():
        assert back[k].dtype == v.dtype and np.array_equal(back[k], v)
    assert set(quant.load_safetensors(p, names={"c"})) == {"c"}


def test_safetensors_agrees_with_the_safetensors_package(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    from safetensors import safe_open
    t = {"w": RNG.standard_normal((6, 8)).astype(np.float16),
         "q": RNG.integers(0, 256, (6, 4)).astype(np.uint8),
         "i": RNG.integers(-5, 5, (3,)).astype(np.int32)}
    ours = str(tmp_path / "ours.safetensors")
    quant.save_safetensors(ours, t, {"clove.format": quant.INT4_FORMAT})
    theirs_read = st.load_file(ours)
    for k, v in t.items():
        assert np.array_equal(theirs_read[k], v) and theirs_read[k].dtype == v.dtype
    with safe_open(ours, framework="numpy") as f:
        assert f.metadata() == {"clove.format": quant.INT4_FORMAT}
    theirs = str(tmp_path / "theirs.safetensors")
    st.save_file(t, theirs, metadata={"m": "1"})
    back = quant.load_safetensors(theirs)
    for k, v in t.items():
        assert np.array_equal(back[k], v) and back[k].dtype == v.dtype
    assert quant.read_safetensors_header(theirs)[1] == {"m": "1"}


def test_int4_linear_file_round_trip(tmp_path):
    src = str(tmp_path / "fp16.safetensors")
    W1 = (RNG.standard_normal((32, 256)) * 0.05).astype(np.float16)
    W2 = (RNG.standard_normal((8, 384)) * 0.05).astype(np.float16)
    quant.save_safetensors(src, {"layers.0.mlp.gate_proj": W1, "layers.0.mlp.down_proj": W2,
                                 "norm": np.ones(256, np.float16)})
    dst = str(tmp_path / "int4.safetensors")
    names = quant.quantize_linear_file(src, dst)
    assert names == ["layers.0.mlp.down_proj", "layers.0.mlp.gate_proj"]  # 1-D "norm" skipped
    w = quant.load_int4_linear(dst)
    q, s, z = w["layers.0.mlp.gate_proj"]
    rq, rs, rz = quant.quantize_rows(W1.astype(np.float32))
    assert np.array_equal(q, rq) and np.array_equal(s, rs) and np.array_equal(z, rz)
    assert q.shape == (32, 128) and s.shape == (32, 2)
    with pytest.raises(ValueError):
        quant.load_int4_linear(src)  # no format metadata


def test_safetensors_rejects_bad_files(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    with open(p, "wb") as f:
        f.write(b"\x01\x02")
    with pytest.raises(ValueError):
        quant.read_safetensors_header(p)
    with pytest.raises(ValueError):
        quant.save_int4_linear(p, {"x": (np.zeros((4, 64), np.uint8), np.zeros((4, 2), np.float16),
                                         np.zeros((4, 1), np.float16))})
