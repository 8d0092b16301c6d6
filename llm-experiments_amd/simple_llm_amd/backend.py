"""Module-level model functions with the reference backend's signatures.

The reference's generate loop (simple-llm/src/generate.py:29-64) calls two
free functions of its JAX backend, and this module gives them a drop-in:

  forward(params, inputs, n_layers, n_heads, head_dim)
      simple-llm/src/jax_backend.py:143-148: logits of every position of
      [B, T] token ids. Here one prefill of all T tokens through the device
      model (skv_embed, the tiled MFMA projections of skv_linear,
      skv_append_prefill_attn), on a cache kept per batch size.
  sample_token(key, logits, temperature, top_k, top_p, min_p,
               repetition_penalty, recent_tokens)
      simple-llm/src/jax_backend.py:413-515: one next token from a logits
      row, through skv_sample (penalty, temperature, min-p, top-k, top-p and
      the draw on the device; greedy is the first maximum).

plus LayerParams / ModelParams with the reference's field names
(jax_backend.py:36-62), so a caller can build params as it does there.

Device weights are made once per params object and reused while that object
(and the arrays it holds) stay the same: the cache is keyed by the object's
identity and the identities of its arrays, as the reference's params are
immutable (jax_backend.py:41). A params whose arrays are modified in place
needs forward_cache_clear().
"""
from __future__ import annotations

import collections
import dataclasses
from typing import Any, Optional

import numpy as np
import torch

from . import _lib
from .model import LAYER_FIELDS, TransformerModel, TransformerModelParams


@dataclasses.dataclass(frozen=True)
class LayerParams:
    """One layer's weights (reference: jax_backend.py:36-55), [in, out]
    matrices as the reference stores them."""

    attn_wq: Any
    attn_wk: Any
    attn_wv: Any
    attn_wo: Any
    ff_w1: Any
    ff_b1: Any
    ff_w2: Any
    ff_b2: Any
    ln_gamma1: Any
    ln_beta1: Any
    ln_gamma2: Any
    ln_beta2: Any


@dataclasses.dataclass(frozen=True)
class ModelParams:
    """The model's weights (reference: jax_backend.py:57-62)."""

    embedding: Any
    pos_encoding: Any
    layers: list


def _field(obj, name):
    if isinstance(obj, dict):
        return obj[name]
    return getattr(obj, name)


def _host(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        return a.detach().float().cpu().numpy()
    return np.asarray(a, np.float32)


def _as_dict(params, n_layers: int) -> dict:
    """The build's params dict (host float32) of a ModelParams-like object
    or dict, first n_layers layers."""
    try:
        layers = list(_field(params, "layers"))
        out = {"embedding": _host(_field(params, "embedding")),
               "pos_encoding": _host(_field(params, "pos_encoding")),
               "layers": [{f: _host(_field(lp, f)) for f in LAYER_FIELDS}
                          for lp in layers[:n_layers]]}
    except (KeyError, AttributeError) as e:
        raise ValueError(f"params is missing {e} (expected ModelParams / LayerParams fields)") \
            from None
    return out


def _leaves(params):
    """The layer objects and arrays params holds (the cache entry's
    fingerprint, compared by identity; the entry keeps them alive, so an
    array replaced since cannot come back under a reused id); None when a
    field is missing (_as_dict then says which)."""
    try:
        objs = [_field(params, "embedding"), _field(params, "pos_encoding")]
        for lp in _field(params, "layers"):
            objs.append(lp)
            objs.extend(_field(lp, f) for f in LAYER_FIELDS)
    except (KeyError, AttributeError, TypeError):
        return None
    return tuple(objs)


def _same(a, b) -> bool:
    return a is not None and b is not None and len(a) == len(b) and \
        all(x is y for x, y in zip(a, b))


_MAX_MODELS = 4
_models: "collections.OrderedDict[tuple, tuple]" = collections.OrderedDict()
_ctx = None


def _context():
    global _ctx
    if _ctx is None:
        from .gpu import gpu
        _ctx = gpu.context_create()
    return _ctx


def forward_cache_clear() -> None:
    """Drops the device weights made by forward() (after params were
    modified in place)."""
    _models.clear()


def device_model(params, n_layers: int, n_heads: int, head_dim: int,
                 ctx=None) -> TransformerModel:
    """The device model of params (made on first use, then reused)."""
    key = (id(params), int(n_layers), int(n_heads), int(head_dim))
    hit = _models.get(key)
    fp = _leaves(params)
    if hit is not None and hit[0] is params and _same(hit[1], fp):
        _models.move_to_end(key)
        return hit[2]
    p = _as_dict(params, n_layers)
    V, d = p["embedding"].shape
    if n_heads <= 0 or head_dim <= 0 or n_heads * head_dim != d:
        raise ValueError(f"n_heads * head_dim = {n_heads} * {head_dim} does not match the "
                         f"embedding dim {d}")
    if n_layers <= 0 or len(p["layers"]) < n_layers:
        raise ValueError(f"params hold {len(p['layers'])} layers, n_layers={n_layers}")
    tm = TransformerModelParams(vocab_size=int(V), embedding_dim=int(d),
                                context_size=int(p["pos_encoding"].shape[0]),
                                n_heads=int(n_heads), n_layers=int(n_layers))
    model = TransformerModel(ctx if ctx is not None else _context(), tm, p)
    # the entry keeps params alive, so its id is not reused while cached
    _models[key] = (params, fp, model)
    while len(_models) > _MAX_MODELS:
        _models.popitem(last=False)
    return model


def forward(params, inputs, n_layers: int, n_heads: int, head_dim: int) -> torch.Tensor:
    """Logits of every position, [B, T, V] float32 on the device
    (reference: jax_backend.py:143-148). inputs: [B, T] token ids (any int
    array or tensor), T <= the rows of params' pos_encoding; position t of
    every row uses pos_encoding[t]. The reference adds the whole
    pos_encoding table, so it takes T equal to its context_size; for that T
    the two agree (within fp32 rounding). Weights: the first n_layers layers,
    heads of head_dim."""
    model = device_model(params, n_layers, n_heads, head_dim)
    if isinstance(inputs, torch.Tensor):
        inputs = inputs.detach().cpu().numpy()
    tokens = np.asarray(inputs)
    if tokens.ndim != 2 or tokens.shape[0] <= 0 or tokens.shape[1] <= 0:
        raise ValueError(f"inputs must be [B, T] token ids, got shape {tokens.shape}")
    if not np.issubdtype(tokens.dtype, np.integer):
        raise ValueError("inputs must be integer token ids")
    B, T = tokens.shape
    tm = model.tm_params
    if T > tm.context_size:
        raise ValueError(f"inputs have {T} positions, pos_encoding only {tm.context_size}")
    key = ("fwd_cache", B)
    cache = model._bufs.get(key)
    if cache is None:
        cache = model._bufs[key] = model.new_cache(B)
    else:
        cache.current_len = 0
    return model.prefill(cache, tokens.astype(np.int64), all_logits=True)


def _seed_of(key) -> int:
    """A 64-bit draw seed of an int, or of an array of words (a PRNG key)."""
    if isinstance(key, (int, np.integer)):
        return int(key) & ((1 << 64) - 1)
    if isinstance(key, torch.Tensor):
        key = key.detach().cpu().numpy()
    words = np.asarray(key).reshape(-1).astype(np.uint64)
    s = 0
    for i, w in enumerate(words.tolist()):
        s ^= (int(w) & 0xFFFFFFFF) << (32 * (i % 2))
        if i % 2 == 1:
            s = (s * 0x9E3779B97F4A7C15 + i) & ((1 << 64) - 1)
    return s & ((1 << 64) - 1)


def sample_token(key, logits, temperature, top_k, top_p, min_p, repetition_penalty,
                 recent_tokens) -> int:
    """Next token id from one logits row (reference: jax_backend.py:413-515).

    The repetition penalty divides the logit of each distinct token of
    recent_tokens; temperature == 0 is greedy (the first maximum); otherwise
    softmax(logits / temperature) filtered by min_p, top_k and top_p
    (renormalised after each), then one draw, all on the device (skv_sample).
    key: an int seed or an array of words (a PRNG key); the draw's uniform is
    splitmix64 of (seed, 0, len(recent_tokens)), so the same key and inputs
    give the same token. The reference's jax.random stream is not
    reproduced: the token drawn for a given key differs from the reference's,
    the distribution it is drawn from is the same. logits: [V] (or [1, V])
    float tensor or array, on the device or the host."""
    lg = logits if isinstance(logits, torch.Tensor) else torch.from_numpy(
        np.ascontiguousarray(np.asarray(logits, np.float32)))
    lg = lg.reshape(-1)
    V = int(lg.numel())
    if V <= 0:
        raise ValueError("logits must hold at least one entry")
    if temperature < 0 or top_k < 0 or min_p < 0 or repetition_penalty <= 0:
        raise ValueError("bad sampling parameters")
    ctx = _context()
    dev = ctx.device
    lg = lg.to(device=dev, dtype=torch.float32).contiguous().reshape(1, V)
    if isinstance(recent_tokens, torch.Tensor):
        recent_tokens = recent_tokens.detach().cpu().numpy()
    recent = np.asarray(recent_tokens, np.int64).reshape(-1)
    n = int(recent.size)
    if n and (recent.min() < 0 or recent.max() >= V):
        raise ValueError("recent token out of the vocabulary")
    L = _lib.lib()
    s = _lib.stream_handle(dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    if temperature == 0.0 and (repetition_penalty == 1.0 or n == 0):
        wsb = L.skv_argmax_workspace_bytes(1, V)
        ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=dev)
        _lib.check(L.skv_argmax(out.data_ptr(), lg.data_ptr(), 1, V, ws.data_ptr(), wsb, s),
                   "skv_argmax")
        return int(out.item())
    if V > 65536:
        raise ValueError("device sampling supports vocab sizes up to 65536")
    seq = torch.from_numpy(np.ascontiguousarray(recent.astype(np.int32).reshape(1, -1)
                                                if n else np.zeros((1, 1), np.int32))).to(dev)
    lens = torch.full((1,), n, dtype=torch.int32, device=dev)
    wsb = L.skv_sample_workspace_bytes(1, V)
    ws = torch.empty(max(wsb, 8), dtype=torch.uint8, device=dev)
    _lib.check(L.skv_sample(out.data_ptr(), None, lg.data_ptr(), seq.data_ptr(),
                            max(n, 1), lens.data_ptr(), 1, V, float(temperature), int(top_k),
                            float(top_p), float(min_p), float(repetition_penalty), n,
                            _seed_of(key), ws.data_ptr(), wsb, s), "skv_sample")
    return int(out.item())


__all__ = ["LayerParams", "ModelParams", "forward", "sample_token", "device_model",
           "forward_cache_clear"]
