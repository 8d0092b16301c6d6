"""The reference's model directory (model_config.json + model.flax.zst):
simple_llm_amd.checkpoint against the formats' specifications. CPU only.

The expected bytes below are assembled by hand from the msgpack
specification (fixmap 0x8N, fixstr 0xaN, fixarray 0x9N, bin8 0xc4, ext8 0xc7,
fixext16 0xd8, float64 0xcb) around flax's documented layout of an array
leaf: extension type 1 holding msgpack((shape, dtype name, C-order bytes)).
flax itself is absent from this image and the reference ships no checkpoint
file, so byte compatibility with real flax output is parity unpinned beyond
that layout.
"""
from __future__ import annotations

import json
import os
import struct

import msgpack
import numpy as np
import pytest

from simple_llm_amd import checkpoint as C
from simple_llm_amd import model as M


def _ext8(code: int, data: bytes) -> bytes:
    return bytes([0xC7, len(data), code]) + data


def test_array_leaf_bytes_follow_the_msgpack_spec():
    state = {"a": np.array([1, 2], np.int8)}
    inner = bytes([0x93, 0x91, 0x02, 0xA4]) + b"int8" + bytes([0xC4, 0x02, 0x01, 0x02])
    want = bytes([0x81, 0xA1]) + b"a" + _ext8(1, inner)
    assert C.msgpack_serialize(state) == want
    got = C.msgpack_restore(want)
    assert list(got) == ["a"] and got["a"].dtype == np.int8 and got["a"].tolist() == [1, 2]


def test_scalar_and_complex_leaves():
    # numpy scalar: extension 3 holding its 0-d array triple (16 bytes -> fixext16)
    inner = bytes([0x93, 0x90, 0xA7]) + b"float32" + bytes([0xC4, 0x04]) + struct.pack("<f", 1.5)
    want = bytes([0x81, 0xA1]) + b"s" + bytes([0xD8, 0x03]) + inner
    assert C.msgpack_serialize({"s": np.float32(1.5)}) == want
    s = C.msgpack_restore(want)["s"]
    assert isinstance(s, np.float32) and s == 1.5
    # Python complex: extension 2 holding msgpack((re, im))
    inner = bytes([0x92, 0xCB]) + struct.pack(">d", 1.0) + bytes([0xCB]) + struct.pack(">d", -2.0)
    want = bytes([0x81, 0xA1]) + b"c" + _ext8(2, inner)
    assert C.msgpack_serialize({"c": complex(1.0, -2.0)}) == want
    assert C.msgpack_restore(want)["c"] == complex(1.0, -2.0)


def test_bfloat16_leaves_widen_to_float32():
    bits = struct.pack("<3H", 0x3F80, 0xC000, 0x3F00)  # 1.0, -2.0, 0.5
    inner = bytes([0x93, 0x91, 0x03, 0xA8]) + b"bfloat16" + bytes([0xC4, 0x06]) + bits
    got = C.msgpack_restore(bytes([0x81, 0xA1]) + b"w" + _ext8(1, inner))["w"]
    assert got.dtype == np.float32 and got.tolist() == [1.0, -2.0, 0.5]


def test_large_leaves_are_chunked(monkeypatch):
    monkeypatch.setattr(C, "MAX_CHUNK_BYTES", 16)  # 4 float32 per chunk
    a = np.arange(10, dtype=np.float32).reshape(2, 5)
    data = C.msgpack_serialize({"x": a, "y": np.ones(4, np.float32)})
    raw = msgpack.unpackb(data, ext_hook=C._ext_unpack, raw=False)
    x = raw["x"]
    assert x["__msgpack_chunked_array__"] is True and x["shape"] == {"0": 2, "1": 5}
    assert [x["chunks"][k].tolist() for k in ("0", "1", "2")] == [[0, 1, 2, 3], [4, 5, 6, 7], [8, 9]]
    assert isinstance(raw["y"], np.ndarray)  # exactly 16 bytes: not chunked
    back = C.msgpack_restore(data)
    assert np.array_equal(back["x"], a) and np.array_equal(back["y"], np.ones(4))


def test_zstd_frames(tmp_path):
    p = str(tmp_path / "f.zst")
    C.write_zstd(p, b"hello " * 1000)
    raw = open(p, "rb").read()
    assert raw[:4] == bytes([0x28, 0xB5, 0x2F, 0xFD])  # zstd frame magic, little endian
    assert C.read_zstd(p) == b"hello " * 1000
    # two frames back to back (a streaming writer's output) read as one stream
    with open(p, "ab") as f:
        f.write(open(p, "rb").read())
    assert C.read_zstd(p) == b"hello " * 2000
    # a streamed frame, whose header does not declare its size
    import pyarrow as pa
    sink = pa.BufferOutputStream()
    with pa.CompressedOutputStream(sink, "zstd") as f:
        f.write(b"abc" * 5000)
    streamed = sink.getvalue().to_pybytes()
    assert C._zstd_content_size(streamed) == -1
    open(p, "wb").write(streamed)
    assert C.read_zstd(p) == b"abc" * 5000


@pytest.mark.parametrize("n", [0, 1, 255, 256, 65791, 65792, 1 << 20])
def test_zstd_declared_size(n):
    """Frame_Content_Size field widths: 1 byte (single segment), 2 bytes
    (value - 256, for 256..65791), 4 bytes, 8 bytes."""
    import pyarrow as pa
    data = (bytes(range(256)) * (n // 256 + 1))[:n]
    for level in (1, 3, 19):
        frame = pa.Codec("zstd", compression_level=level).compress(data, asbytes=True)
        assert C._zstd_content_size(frame) == n


def _small():
    tm = M.TransformerModelParams(vocab_size=61, embedding_dim=32, context_size=24, n_heads=4,
                                  n_layers=3, epochs=[2, 5])
    return tm, M.initialize_params(tm, seed=7, std=0.1)


def test_model_dir_round_trip_is_exact(tmp_path):
    tm, params = _small()
    d = str(tmp_path / "model")
    C.save_model_dir(d, tm, params)
    assert sorted(os.listdir(d)) == ["model.flax.zst", "model_config.json"]
    assert json.load(open(os.path.join(d, "model_config.json"))) == {
        "vocab_size": 61, "embedding_dim": 32, "context_size": 24, "n_heads": 4, "n_layers": 3,
        "epochs": [2, 5]}
    state = C.msgpack_restore(C.read_zstd(os.path.join(d, "model.flax.zst")))
    # ModelParams / LayerParams field order; the layer list keyed "0", "1", ...
    assert list(state) == ["embedding", "pos_encoding", "layers"]
    assert list(state["layers"]) == ["0", "1", "2"]
    assert tuple(state["layers"]["0"]) == M.LAYER_FIELDS
    tm2, p2 = C.load_model_dir(d)
    assert tm2 == tm
    for k in ("embedding", "pos_encoding"):
        assert p2[k].dtype == np.float32 and np.array_equal(p2[k], params[k])
    for i in range(3):
        for f in M.LAYER_FIELDS:
            assert np.array_equal(p2["layers"][i][f], params["layers"][i][f]), (i, f)
            assert p2["layers"][i][f].flags.writeable


def test_model_dir_errors(tmp_path):
    tm, params = _small()
    d = str(tmp_path / "m")
    C.save_model_dir(d, tm, params)
    cfg = json.load(open(os.path.join(d, "model_config.json")))
    cfg["n_layers"] = 2
    json.dump(cfg, open(os.path.join(d, "model_config.json"), "w"))
    with pytest.raises(ValueError, match="do not match"):
        C.load_model_dir(d)
    for drop in ("pos_encoding", "ff_b2"):
        broken = C.state_from_params(params)
        if drop == "pos_encoding":
            del broken["pos_encoding"]
        else:
            del broken["layers"]["1"]["ff_b2"]
        C.write_zstd(os.path.join(d, "model.flax.zst"), C.msgpack_serialize(broken))
        with pytest.raises(ValueError, match=f"missing '{drop}'"):
            C.load_model_dir(d)
