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
