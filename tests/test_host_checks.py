"""Host-side argument checks of the drop-in API that need no GPU work: they
raise ValueError before any launch, as the reference's checks do
(simple-llm/src/gpu/gpu_kv_cache.py:55-64, 144-159, 247-264)."""
from __future__ import annotations

import numpy as np
import pytest


def test_max_len_below_a_fill_is_rejected():
    from simple_llm_amd.gpu.gpu_kv_cache import _check_max_len
    _check_max_len(300, np.array([0, 300, 17]))  # covers every fill
    with pytest.raises(ValueError, match="max_len=299 is below the longest fill 300"):
        _check_max_len(299, np.array([0, 300, 17]))


def test_paged_cache_without_a_table_is_rejected():
    from simple_llm_amd.gpu.gpu_kv_cache import _check_layer
    from simple_llm_amd.gpu.gpu_types import KVCache, KVCacheLayer

    layer = KVCacheLayer(None, None, lens=None, host_lens=np.zeros(2, np.int64))
    cache = KVCache.__new__(KVCache)  # no device tensors: only the fields the check reads
    cache.layers, cache.block_size, cache.block_table = [layer], 16, None
    with pytest.raises(ValueError, match="no block table yet"):
        _check_layer(cache, 0)
    with pytest.raises(ValueError, match="out of range"):
        _check_layer(cache, -1)
    cache.block_table = object()
    _check_layer(cache, 0)


def test_backend_forward_rejects_shapes_before_any_device_work():
    """forward() (jax_backend.py:143-148's drop-in) checks n_heads * head_dim
    against the embedding and n_layers against the params first."""
    from simple_llm_amd import backend
    from oracle import model_oracle as mo

    params = mo.init_params(50, 64, 2, 16, seed=0)
    toks = np.zeros((1, 4), np.int32)
    with pytest.raises(ValueError, match="does not match the embedding dim 64"):
        backend.forward(params, toks, 2, 3, 16)
    with pytest.raises(ValueError, match="params hold 2 layers, n_layers=3"):
        backend.forward(params, toks, 3, 4, 16)
    with pytest.raises(ValueError, match="missing"):
        backend.forward({"embedding": params["embedding"]}, toks, 2, 4, 16)
    assert not backend._models  # nothing was built


def test_backend_sample_token_rejects_bad_parameters():
    from simple_llm_amd import backend

    lg = np.zeros(10, np.float32)
    for args in ((-1.0, 0, 1.0, 0.0, 1.0), (1.0, -2, 1.0, 0.0, 1.0), (1.0, 0, 1.0, -0.1, 1.0),
                 (1.0, 0, 1.0, 0.0, 0.0)):
        with pytest.raises(ValueError, match="bad sampling parameters"):
            backend.sample_token(0, lg, *args, [])
    with pytest.raises(ValueError, match="at least one entry"):
        backend.sample_token(0, np.zeros(0, np.float32), 1.0, 0, 1.0, 0.0, 1.0, [])


def test_backend_seed_of_keys():
    """An int key is the seed; an array key (a PRNG key's words) folds to a
    64-bit seed that depends on every word."""
    from simple_llm_amd.backend import _seed_of

    assert _seed_of(42) == 42 and _seed_of(-1) == (1 << 64) - 1
    a = _seed_of(np.array([0, 42], np.uint32))
    assert a == _seed_of([0, 42]) and 0 <= a < (1 << 64)
    assert a != _seed_of(np.array([0, 43], np.uint32))
    assert a != _seed_of(np.array([1, 42], np.uint32))


def test_backend_weight_cache_fingerprint_is_by_identity():
    """The device weights of forward() are reused only while params holds the
    very same layer objects and arrays: a replaced array (even an equal one)
    is a different fingerprint; the entry keeps the old objects alive, so a
    new array cannot come back under a reused id."""
    from simple_llm_amd import backend
    from oracle import model_oracle as mo

    params = mo.init_params(50, 64, 2, 16, seed=0)
    fp = backend._leaves(params)
    assert backend._same(fp, backend._leaves(params))
    params["layers"][1]["ff_b2"] = params["layers"][1]["ff_b2"].copy()  # equal values, new array
    assert not backend._same(fp, backend._leaves(params))
    params["layers"].pop()
    assert not backend._same(fp, backend._leaves(params))
    assert backend._leaves({"embedding": params["embedding"]}) is None
    assert not backend._same(None, None)
