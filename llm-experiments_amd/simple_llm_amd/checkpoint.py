"""The reference's model directory on disk: load and save.

A model directory holds (simple-llm/src/common/util.py:32-37):
  model_config.json    TransformerModelParams fields (jax_backend.py:381-386)
  model.flax.zst       the ModelParams pytree (jax_backend.py:36-62), flax
                       msgpack serialisation, zstd-compressed (util.py:64-75)
  model_opt.flax.zst   optimizer state (training only; not read here)

Third-party formats, absent from this image and restated from their
published behaviour:
  * flax.serialization (flax >= 0.12.0, the reference's floor): to_bytes is
    msgpack (strict types) of the state dict -- a dataclass becomes a dict
    of its fields in field order, a list a dict keyed "0", "1", ... -- with
    numpy arrays as msgpack extension type 1 holding
    msgpack((shape, dtype name, C-order bytes)), numpy scalars as type 3
    holding the same triple for their 0-d array, Python complex as type 2
    holding msgpack((re, im)), and arrays above 2**30 bytes as
    {"__msgpack_chunked_array__": True, "shape": {"0": ..},
     "chunks": {"0": flat piece, ..}} with pieces of 2**30 bytes.
  * zstd frames (the reference uses the zstandard package) are read and
    written through pyarrow's zstd codec.
Byte-level compatibility with files written by real flax is not checked here
(flax is absent and the reference ships no checkpoint); round trips and the
format's documented structure are.
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Any, Dict

import msgpack
import numpy as np
import pyarrow as pa

CONFIG_FILE = "model_config.json"
PARAMS_FILE = "model.flax.zst"
_EXT_NDARRAY, _EXT_COMPLEX, _EXT_NPSCALAR = 1, 2, 3
_CHUNK_KEY = "__msgpack_chunked_array__"
MAX_CHUNK_BYTES = 2 ** 30
_LAYER_FIELDS = ("attn_wq", "attn_wk", "attn_wv", "attn_wo", "ff_w1", "ff_b1", "ff_w2", "ff_b2",
                 "ln_gamma1", "ln_beta1", "ln_gamma2", "ln_beta2")


# ---- zstd ------------------------------------------------------------------

def _zstd_content_size(raw: bytes) -> int:
    """Frame_Content_Size of the first zstd frame's header (RFC 8878 3.1.1.1),
    or -1 when the header does not declare it."""
    if len(raw) < 6 or raw[:4] != b"\x28\xb5\x2f\xfd":
        return -1
    fhd = raw[4]
    single = (fhd >> 5) & 1
    fcs_bytes = (0 if not single else 1, 2, 4, 8)[fhd >> 6]
    if fcs_bytes == 0:
        return -1
    at = 5 + (0 if single else 1) + (0, 1, 2, 4)[fhd & 3]
    if len(raw) < at + fcs_bytes:
        return -1
    size = int.from_bytes(raw[at:at + fcs_bytes], "little")
    return size + 256 if fcs_bytes == 2 else size


def read_zstd(path: str) -> bytes:
    """Every frame of a zstd file, concatenated: one frame from
    ZstdCompressor.compress (its header holds the decompressed size, so it is
    decompressed in one call into a buffer of that size), or a stream of
    frames from zstd.open (read through the stream decoder)."""
    with open(path, "rb") as f:
        raw = f.read()
    size = _zstd_content_size(raw)
    if size >= 0:
        try:
            return pa.decompress(raw, decompressed_size=size, codec="zstd", asbytes=True)
        except (pa.ArrowException, OSError):
            pass  # more than one frame: the declared size is the first frame's
    with pa.CompressedInputStream(pa.BufferReader(raw), "zstd") as f:
        return f.read()


def write_zstd(path: str, data: bytes, level: int = 3) -> None:
    """One zstd frame (level 3: zstandard.ZstdCompressor's default)."""
    with open(path, "wb") as f:
        f.write(pa.Codec("zstd", compression_level=level).compress(data, asbytes=True))


# ---- flax msgpack ------------------------------------------------------------

def _array_bytes(x: np.ndarray) -> bytes:
    if x.dtype.hasobject or x.dtype.isalignedstruct:
        raise ValueError("object and structured arrays cannot be serialised")
    return msgpack.packb((x.shape, x.dtype.name, np.ascontiguousarray(x).tobytes("C")),
                         use_bin_type=True)


def _array_of_bytes(data: bytes) -> np.ndarray:
    shape, name, buf = msgpack.unpackb(data, raw=True)
    name = name.decode()
    if name == "bfloat16":  # numpy has no bfloat16: widen the bit patterns to float32
        bits = np.frombuffer(buf, dtype=np.uint16).astype(np.uint32) << 16
        return bits.view(np.float32).reshape(shape, order="C")
    return np.frombuffer(buf, dtype=np.dtype(name)).reshape(shape, order="C")


def _ext_unpack(code: int, data: bytes):
    if code == _EXT_NDARRAY:
        return _array_of_bytes(data)
    if code == _EXT_NPSCALAR:
        return _array_of_bytes(data)[()]
    if code == _EXT_COMPLEX:
        re, im = msgpack.unpackb(data)
        return complex(re, im)
    return msgpack.ExtType(code, data)


def _ext_pack(x):
    if isinstance(x, np.ndarray):
        return msgpack.ExtType(_EXT_NDARRAY, _array_bytes(x))
    if isinstance(x, np.generic):
        return msgpack.ExtType(_EXT_NPSCALAR, _array_bytes(np.asarray(x)))
    if isinstance(x, complex):
        return msgpack.ExtType(_EXT_COMPLEX, msgpack.packb((x.real, x.imag)))
    raise TypeError(f"cannot serialise {type(x)}")


def _chunk_leaves(x):
    if isinstance(x, dict):
        return {k: _chunk_leaves(v) for k, v in x.items()}
    if isinstance(x, np.ndarray) and x.size * x.dtype.itemsize > MAX_CHUNK_BYTES:
        step = max(1, MAX_CHUNK_BYTES // x.dtype.itemsize)
        flat = np.ascontiguousarray(x).reshape(-1)
        return {_CHUNK_KEY: True, "shape": {str(i): n for i, n in enumerate(x.shape)},
                "chunks": {str(j): flat[i:i + step]
                           for j, i in enumerate(range(0, flat.size, step))}}
    return x


def _restore_chunks(x):
    if isinstance(x, dict):
        if _CHUNK_KEY in x:
            shape = tuple(x["shape"][str(i)] for i in range(len(x["shape"])))
            chunks = [x["chunks"][str(i)] for i in range(len(x["chunks"]))]
            return np.concatenate([np.asarray(c).reshape(-1) for c in chunks]).reshape(shape)
        return {k: _restore_chunks(v) for k, v in x.items()}
    return x


def msgpack_restore(data: bytes) -> Dict[str, Any]:
    """State dict of flax's msgpack bytes."""
    return _restore_chunks(msgpack.unpackb(data, ext_hook=_ext_unpack, raw=False))


def msgpack_serialize(state: Dict[str, Any]) -> bytes:
    """flax's msgpack bytes of a state dict (dicts, lists as "0".. dicts, arrays)."""
    return msgpack.packb(_chunk_leaves(state), default=_ext_pack, strict_types=True)


# ---- model params <-> state dict --------------------------------------------

def state_from_params(params: dict) -> Dict[str, Any]:
    """The state dict flax makes of ModelParams (jax_backend.py:57-62)."""
    return {"embedding": np.asarray(params["embedding"]),
            "pos_encoding": np.asarray(params["pos_encoding"]),
            "layers": {str(i): {f: np.asarray(lp[f]) for f in _LAYER_FIELDS}
                       for i, lp in enumerate(params["layers"])}}


def params_from_state(state: Dict[str, Any]) -> dict:
    """The build's params dict (float32, writable copies) of a ModelParams
    state dict."""
    try:
        layers = state["layers"]
        n = len(layers)
        out = {"embedding": np.array(state["embedding"], np.float32),
               "pos_encoding": np.array(state["pos_encoding"], np.float32),
               "layers": [{f: np.array(layers[str(i)][f], np.float32) for f in _LAYER_FIELDS}
                          for i in range(n)]}
    except KeyError as e:
        raise ValueError(f"checkpoint is missing {e} (expected ModelParams fields)") from None
    return out


# ---- directory ----------------------------------------------------------------

def load_model_dir(model_path: str):
    """(TransformerModelParams, params dict) of a reference model directory
    (jax_backend.py:396-410 without the optimizer state)."""
    from .model import TransformerModelParams

    with open(os.path.join(model_path, CONFIG_FILE)) as f:
        cfg = json.load(f)
    tm = TransformerModelParams(**cfg)
    params = params_from_state(msgpack_restore(read_zstd(os.path.join(model_path, PARAMS_FILE))))
    d = tm.embedding_dim
    if params["embedding"].shape != (tm.vocab_size, d) or len(params["layers"]) != tm.n_layers \
            or params["pos_encoding"].shape != (tm.context_size, d):
        raise ValueError("checkpoint shapes do not match model_config.json")
    return tm, params


def save_model_dir(model_path: str, tm, params: dict) -> None:
    """Writes model_config.json and model.flax.zst (jax_backend.py:389-394)."""
    os.makedirs(model_path, exist_ok=True)
    write_zstd(os.path.join(model_path, PARAMS_FILE), msgpack_serialize(state_from_params(params)))
    with open(os.path.join(model_path, CONFIG_FILE), "w") as f:
        json.dump(dataclasses.asdict(tm), f, indent=2)


def load_model(hp, total_steps, model_path: str, ctx=None, kv_dtype=None):
    """A device TransformerModel with a reference model directory's weights.

    Same arguments as the reference's load_model (jax_backend.py:389-410,
    called as generate.py:94 does); hp and total_steps only shape the
    optimizer the reference rebuilds for training, so they are accepted and
    not used here."""
    import torch

    from .gpu import gpu
    from .model import TransformerModel

    del hp, total_steps
    tm, params = load_model_dir(model_path)
    ctx = ctx if ctx is not None else gpu.context_create()
    return TransformerModel(ctx, tm, params, kv_dtype=kv_dtype or torch.float32)


def save_model(model, model_path: str) -> None:
    """The reference's save_model (jax_backend.py:381-386) for a
    TransformerModel: its config and host weights (no optimizer state)."""
    save_model_dir(model_path, model.tm_params, model.params)
