"""KV-cache management and cached attention on gfx950.

Drop-in for simple-llm/src/gpu/gpu_kv_cache.py: same functions, arguments,
checks and error messages:
  kv_cache_create          gpu_kv_cache.py:26-87
  kv_cache_reset           gpu_kv_cache.py:90-105
  kv_cache_update          gpu_kv_cache.py:113-186
  attention_with_kv_cache  gpu_kv_cache.py:194-289
The work is done by hand-written HIP kernels behind the C ABI in
include/skv.h (append: skv_append; attention: skv_decode_attn). There is no
CPU path: without libskv.so every call raises.

Differences from the reference, all supersets of its behaviour:
  * lengths are per layer and per sequence, kept on the device and advanced
    by the append kernel (see KVCache in gpu_types.py for the position rule);
  * decode attention has no length cap (the reference raises above
    attention_workgroup_size = 256, gpu_kv_cache.py:250-257);
  * bf16 storage, grouped-query heads and a paged layout are options of
    KVCacheConfig; the defaults reproduce the reference's fp32 MHA cache.

Extensions beyond the reference's four functions:
  kv_cache_append           append with per-sequence positions (no
                            full-cache error: full sequences are skipped)
  kv_cache_set_block_table  install the page table of a paged cache
  kv_cache_prefill          append a chunk of tokens (prefill), optionally
                            followed by causal attention over prefix + chunk
"""
from __future__ import annotations

import ctypes
import math
import threading
from typing import List, Optional

import numpy as np
import torch

from .. import _lib
from .gpu_ops import batch_count, validate_buffer_shape_2d
from .gpu_types import (
    GPUBuffer2D,
    GPUContext,
    KVCache,
    KVCacheConfig,
    KVCacheLayer,
)

# ============================================================================
# KV-CACHE CREATION
# ============================================================================


def kv_cache_create(ctx: GPUContext, config: KVCacheConfig) -> KVCache:
    """Allocate zero-filled K/V storage for every layer; current_len = 0.

    Same validation as the reference (gpu_kv_cache.py:55-64). Contiguous
    caches are [batch_size * max_seq_len, n_kv_heads * head_dim] per tensor;
    paged caches are a pool [n_blocks * block_size, n_kv_heads * head_dim]
    whose page table starts as the identity mapping (sequence b owns pages
    b*max_blocks .. b*max_blocks + max_blocks - 1) when the pool is big
    enough; a smaller pool has no table until kv_cache_set_block_table
    installs one (appends and attention raise ValueError before that).
    """
    if config.batch_size <= 0:
        raise ValueError(f"batch_size must be > 0, got {config.batch_size}")
    if config.max_seq_len <= 0:
        raise ValueError(f"max_seq_len must be > 0, got {config.max_seq_len}")
    if config.n_layers <= 0:
        raise ValueError(f"n_layers must be > 0, got {config.n_layers}")
    if config.n_heads <= 0:
        raise ValueError(f"n_heads must be > 0, got {config.n_heads}")
    if config.head_dim <= 0:
        raise ValueError(f"head_dim must be > 0, got {config.head_dim}")
    n_kv = config.n_kv_heads or config.n_heads
    if n_kv <= 0 or config.n_heads % n_kv != 0:
        raise ValueError(f"n_heads ({config.n_heads}) must be a multiple of n_kv_heads ({n_kv})")
    if config.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"dtype must be torch.float32 or torch.bfloat16, got {config.dtype}")

    e_kv = n_kv * config.head_dim
    B = config.batch_size
    block_table = None
    n_blocks = 0
    if config.block_size > 0:
        bs = config.block_size
        if bs & (bs - 1):
            raise ValueError(f"block_size must be a power of two, got {bs}")
        max_blocks = -(-config.max_seq_len // bs)
        n_blocks = config.n_blocks or B * max_blocks
        rows = n_blocks * bs
        if n_blocks >= B * max_blocks:
            block_table = torch.arange(B * max_blocks, dtype=torch.int32).reshape(
                B, max_blocks).to(ctx.device)
    else:
        rows = B * config.max_seq_len

    layers: List[KVCacheLayer] = []
    for _ in range(config.n_layers):
        k = torch.zeros((rows, e_kv), dtype=config.dtype, device=ctx.device)
        v = torch.zeros((rows, e_kv), dtype=config.dtype, device=ctx.device)
        layers.append(KVCacheLayer(
            k_cache=GPUBuffer2D(buffer=k, shape=(rows, e_kv), size=rows * e_kv),
            v_cache=GPUBuffer2D(buffer=v, shape=(rows, e_kv), size=rows * e_kv),
            lens=torch.zeros(B, dtype=torch.int32, device=ctx.device),
            host_lens=np.zeros(B, dtype=np.int64)))

    return KVCache(layers=layers, batch_size=B, max_seq_len=config.max_seq_len, current_len=0,
                   n_heads=config.n_heads, head_dim=config.head_dim, n_kv_heads=n_kv,
                   dtype=config.dtype, block_size=config.block_size, n_blocks=n_blocks,
                   block_table=block_table)


def kv_cache_reset(cache: KVCache) -> None:
    """Empty the cache without touching its contents (reference :90-105)."""
    cache.current_len = 0


def kv_cache_set_block_table(cache: KVCache, block_table: torch.Tensor) -> None:
    """Install a page table [batch_size, ceil(max_seq_len / block_size)] of pool page ids."""
    if not cache.paged:
        raise ValueError("kv_cache_set_block_table: cache is not paged")
    max_blocks = -(-cache.max_seq_len // cache.block_size)
    if tuple(block_table.shape) != (cache.batch_size, max_blocks):
        raise ValueError(f"block_table shape mismatch: got {tuple(block_table.shape)}, "
                         f"expected {(cache.batch_size, max_blocks)}")
    host = block_table.detach().to("cpu")
    if host.numel() and (int(host.min()) < 0 or int(host.max()) >= cache.n_blocks):
        raise ValueError(f"block_table entries must lie in [0, {cache.n_blocks})")
    cache.block_table = block_table.to(device=cache.layers[0].lens.device,
                                       dtype=torch.int32).contiguous()


# ============================================================================
# KV-CACHE UPDATE
# ============================================================================


def _check_layer(cache: KVCache, layer_idx: int) -> None:
    if layer_idx < 0 or layer_idx >= len(cache.layers):
        raise ValueError(f"layer_idx {layer_idx} out of range [0, {len(cache.layers)})")
    if cache.paged and cache.block_table is None:
        raise ValueError("the paged cache has no block table yet: its pool is smaller than "
                         "batch_size * ceil(max_seq_len / block_size) pages, so install one "
                         "with kv_cache_set_block_table first")


def _check_max_len(max_len: int, fills: np.ndarray) -> None:
    # the split-K grid covers batch_size * max_len tokens of the flat token
    # stream; a fill beyond it would come back as NaN rows
    top = int(fills.max()) if fills.size else 0
    if max_len < top:
        raise ValueError(f"max_len={max_len} is below the longest fill {top}: the attention "
                         f"plan would not cover every filled position")


def _check_tensor(t: torch.Tensor, name: str, device: torch.device) -> None:
    # Kernels dereference these pointers on the GPU: host tensors never reach them.
    # Fast path first (get_device() is an int; t.device builds an object).
    if (device.type == "cuda" and t.is_cuda and t.get_device() == (device.index or 0)
            and t.is_contiguous() and t.data_ptr() % 16 == 0):
        return
    if device.type != "cuda" or not t.is_cuda:
        raise ValueError(f"{name}: the KV cache and its operands must live on the ROCm "
                         f"device (cache on {device}, {name} on {t.device})")
    if t.device.index != (device.index or 0):
        raise ValueError(f"{name} must live on {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def _launch_append(ctx: GPUContext, cache: KVCache, layer: KVCacheLayer, k: torch.Tensor,
                   v: torch.Tensor) -> None:
    dev = layer.lens.device
    for t, n in ((k, "new_k"), (v, "new_v")):
        _check_tensor(t, n, dev)
    if k.dtype != v.dtype:
        raise ValueError("new_k and new_v must share a dtype")
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    cdt, idt = _lib.dtype_code(cache.dtype), _lib.dtype_code(k.dtype)
    if cache.paged:
        max_blocks = cache.block_table.shape[1]
        rc = L.skv_append_paged(layer.k_cache.buffer.data_ptr(), layer.v_cache.buffer.data_ptr(),
                                k.data_ptr(), v.data_ptr(), layer.lens.data_ptr(),
                                cache.block_table.data_ptr(), max_blocks, cache.block_size,
                                cache.batch_size, cache.n_kv_heads, cache.head_dim, cdt, idt,
                                stream)
    else:
        rc = L.skv_append(layer.k_cache.buffer.data_ptr(), layer.v_cache.buffer.data_ptr(),
                          k.data_ptr(), v.data_ptr(), layer.lens.data_ptr(), cache.batch_size,
                          cache.n_kv_heads, cache.head_dim, cache.max_seq_len, cdt, idt, stream)
    _lib.check(rc, "skv_append")
    # mirror the kernel's rule: write and advance where pos < capacity
    cap = cache.block_table.shape[1] * cache.block_size if cache.paged else cache.max_seq_len
    layer.host_lens = np.where(layer.host_lens < cap, layer.host_lens + 1, layer.host_lens)


def kv_cache_update(ctx: GPUContext, cache: KVCache, layer_idx: int, new_k: GPUBuffer2D,
                    new_v: GPUBuffer2D) -> None:
    """Append one token per sequence to one layer (reference :113-186).

    new_k, new_v: [batch_size, n_kv_heads * head_dim]. Raises ValueError on a
    bad layer index, a full cache or a shape mismatch, before any GPU work.
    The layer's fill advances by one.
    """
    _check_layer(cache, layer_idx)
    layer = cache.layers[layer_idx]
    cur = int(layer.host_lens.max())
    if cur >= cache.max_seq_len:
        raise ValueError(
            f"Cache is full: current_len={cur}, max_seq_len={cache.max_seq_len}")
    e_kv = cache.n_kv_heads * cache.head_dim
    expected_rows = cache.batch_size * 1
    validate_buffer_shape_2d(new_k, (expected_rows, e_kv), "new_k")
    validate_buffer_shape_2d(new_v, (expected_rows, e_kv), "new_v")
    batch_count(ctx)
    _launch_append(ctx, cache, layer, new_k.buffer, new_v.buffer)


def kv_cache_append(ctx: GPUContext, cache: KVCache, layer_idx: int, new_k: torch.Tensor,
                    new_v: torch.Tensor) -> np.ndarray:
    """Per-sequence append (extension): sequence b writes at its own fill.

    new_k, new_v: tensors of [batch_size, n_kv_heads, head_dim] (or
    [batch_size, n_kv_heads * head_dim]). Sequences that are already full are
    skipped (retired). Returns the host mirror of the new fills.
    """
    _check_layer(cache, layer_idx)
    e_kv = cache.n_kv_heads * cache.head_dim
    for t, n in ((new_k, "new_k"), (new_v, "new_v")):
        if t.numel() != cache.batch_size * e_kv:
            raise ValueError(f"{n} must hold batch_size*n_kv_heads*head_dim = "
                             f"{cache.batch_size * e_kv} elements, got {t.numel()}")
    batch_count(ctx)
    layer = cache.layers[layer_idx]
    _launch_append(ctx, cache, layer, new_k, new_v)
    return layer.host_lens.copy()


# ============================================================================
# ATTENTION WITH KV-CACHE
# ============================================================================


def _workspace(ctx: GPUContext, nbytes: int) -> torch.Tensor:
    ws = ctx.decode_workspace
    if ws is None or ws.numel() < nbytes or ws.device != ctx.device:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=ctx.device)
        ctx.decode_workspace = ws
    return ws


_WS_BYTES: dict = {}
_PLAN_OUT = threading.local()


def _decode_ws_bytes(B: int, h_q: int, d: int, n_chunks: int) -> int:
    # skv_decode_workspace_bytes, memoised: a decode loop asks for the same few
    # sizes every call and the ctypes round trip costs more than the lookup
    key = (B, h_q, d, n_chunks)
    need = _WS_BYTES.get(key)
    if need is None:
        if len(_WS_BYTES) > 4096:
            _WS_BYTES.clear()
        need = _WS_BYTES[key] = int(_lib.lib().skv_decode_workspace_bytes(B, h_q, d, n_chunks))
    return need


def _fills_after_append(fills: np.ndarray, cap: int) -> tuple[np.ndarray, int, int]:
    """(fills after one append, their maximum, their sum); full sequences stay put.

    Small batches go through Python ints: three numpy calls on an 8-entry
    array cost about 4 us of host time per decode call, the list about 1 us."""
    if fills.size <= 64:
        after = [f + 1 if f < cap else cap for f in fills.tolist()]
        top = max(after) if after else 0
        return np.array(after, dtype=np.int64), top, sum(after)
    after = np.minimum(fills + 1, cap)
    return after, int(after.max()), int(after.sum())


def decode_plan(ctx: GPUContext, batch_size: int, n_heads: int, n_kv_heads: int, max_len: int,
                total_len: int = 0, *, head_dim: int, dtype: torch.dtype) -> tuple[int, int]:
    """(chunk_tokens, n_chunks_max) of the split-K decode for these sizes.

    total_len: filled tokens over the batch (0: batch_size * max_len);
    head_dim and the cache dtype select the kernel the plan is tuned for."""
    out = getattr(_PLAN_OUT, "refs", None)
    if out is None:  # per thread: the call releases the GIL while it fills them
        c, n = ctypes.c_int(), ctypes.c_int()
        out = _PLAN_OUT.refs = (c, n, ctypes.byref(c), ctypes.byref(n))
    rc = _lib.lib().skv_decode_plan(batch_size, n_heads, n_kv_heads, int(head_dim),
                                    _lib.dtype_code(dtype), max(int(max_len), 1), int(total_len),
                                    int(ctx.config.decode_chunk_tokens), out[2], out[3])
    if rc:
        _lib.check(rc, "skv_decode_plan")
    return out[0].value, out[1].value


# Plans by (sizes, max_len, chunk hint): the plan of a total fill in [lo, hi] is (chunk, n).
_PLAN_SPANS: dict = {}


def _decode_plan_span(ctx: GPUContext, batch_size: int, n_heads: int, n_kv_heads: int,
                      max_len: int, total_len: int, head_dim: int,
                      dtype: torch.dtype) -> tuple[int, int]:
    """decode_plan for a decode loop: the plan changes rarely as the fills grow, and
    skv_decode_plan's chunk never decreases as total_len grows (n_chunks_max follows the
    chunk; tests/test_abi.py checks both). So a miss also finds, by doubling and bisection,
    the largest total with the same plan, and the calls up to it skip the ctypes query (~2
    us of host time each)."""
    hint = int(ctx.config.decode_chunk_tokens)
    key = (batch_size, n_heads, n_kv_heads, head_dim, dtype, max_len, hint)
    span = _PLAN_SPANS.get(key)
    if span is not None and span[0] <= total_len <= span[1]:
        return span[2], span[3]
    plan = decode_plan(ctx, batch_size, n_heads, n_kv_heads, max_len, total_len,
                       head_dim=head_dim, dtype=dtype)

    def same(t: int) -> bool:
        return decode_plan(ctx, batch_size, n_heads, n_kv_heads, max_len, t,
                           head_dim=head_dim, dtype=dtype) == plan

    # largest total with this plan, up to every sequence at max_len
    top = max(batch_size * max(int(max_len), 1), total_len)
    lo, step = total_len, 1
    while lo + step <= top and same(lo + step):
        lo += step
        step *= 2
    hi = min(lo + step, top + 1)  # plan(lo) == plan, plan(hi) != plan or hi past top
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if same(mid):
            lo = mid
        else:
            hi = mid
    if len(_PLAN_SPANS) > 1024:
        _PLAN_SPANS.clear()
    _PLAN_SPANS[key] = (total_len, lo, plan[0], plan[1])
    return plan


def decode_attention(ctx: GPUContext, cache: KVCache, layer_idx: int, q: torch.Tensor,
                     out: torch.Tensor, scale: Optional[float] = None,
                     max_len: Optional[int] = None) -> None:
    """Single-query attention of every sequence over its filled prefix.

    q, out: contiguous device tensors of [batch_size, n_heads, head_dim]
    elements (float32 or bfloat16). max_len: an upper bound of the fills
    (default: the host mirror's maximum), used to size the split-K grid; the
    chunk size follows the batch's total fill (host mirror).
    """
    _check_layer(cache, layer_idx)
    layer = cache.layers[layer_idx]
    dev = layer.lens.device
    _check_tensor(q, "q_new", dev)
    _check_tensor(out, "output", dev)
    e_q = cache.n_heads * cache.head_dim
    if q.numel() != cache.batch_size * e_q or out.numel() != cache.batch_size * e_q:
        raise ValueError(f"q_new/output must hold batch_size*n_heads*head_dim = "
                         f"{cache.batch_size * e_q} elements")
    if max_len is None:
        max_len = int(layer.host_lens.max())
    _check_max_len(max_len, layer.host_lens)
    total = int(np.minimum(layer.host_lens, max_len).sum())
    chunk, nchunks = _decode_plan_span(ctx, cache.batch_size, cache.n_heads, cache.n_kv_heads,
                                       max_len, total, cache.head_dim, cache.dtype)
    L = _lib.lib()
    need = _decode_ws_bytes(cache.batch_size, cache.n_heads, cache.head_dim, nchunks)
    ws = _workspace(ctx, need)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(cache.head_dim)
    stream = _lib.stream_handle(dev)
    cdt, qdt, odt = (_lib.dtype_code(cache.dtype), _lib.dtype_code(q.dtype),
                     _lib.dtype_code(out.dtype))
    if cache.paged:
        rc = L.skv_decode_attn_paged(out.data_ptr(), q.data_ptr(), layer.k_cache.buffer.data_ptr(),
                                     layer.v_cache.buffer.data_ptr(), layer.lens.data_ptr(),
                                     cache.block_table.data_ptr(), cache.block_table.shape[1],
                                     cache.block_size, cache.batch_size, cache.n_heads,
                                     cache.n_kv_heads, cache.head_dim, sc, chunk, nchunks,
                                     ws.data_ptr(), ws.numel(), cdt, qdt, odt, stream)
    else:
        rc = L.skv_decode_attn(out.data_ptr(), q.data_ptr(), layer.k_cache.buffer.data_ptr(),
                               layer.v_cache.buffer.data_ptr(), layer.lens.data_ptr(),
                               cache.batch_size, cache.n_heads, cache.n_kv_heads, cache.head_dim,
                               cache.max_seq_len, sc, chunk, nchunks, ws.data_ptr(), ws.numel(),
                               cdt, qdt, odt, stream)
    _lib.check(rc, "skv_decode_attn")


def kv_cache_append_attend(ctx: GPUContext, cache: KVCache, layer_idx: int, new_k: torch.Tensor,
                           new_v: torch.Tensor, q: torch.Tensor, out: torch.Tensor,
                           scale: Optional[float] = None,
                           max_len: Optional[int] = None) -> np.ndarray:
    """kv_cache_append followed by decode_attention in one call (extension).

    Appends new_k/new_v ([batch_size, n_kv_heads, head_dim], or flat) at each
    sequence's fill (full sequences are skipped), then attends q
    ([batch_size, n_heads, head_dim]) over the fills including the new token,
    writing out. The same results as the two calls, without the separate
    append launch (skv_append_decode_attn). max_len bounds the fills after
    the append (default: the host mirror's). Returns the new fills.
    """
    _check_layer(cache, layer_idx)
    layer = cache.layers[layer_idx]
    dev = layer.lens.device
    e_kv = cache.n_kv_heads * cache.head_dim
    for t, n in ((new_k, "new_k"), (new_v, "new_v")):
        _check_tensor(t, n, dev)
        if t.numel() != cache.batch_size * e_kv:
            raise ValueError(f"{n} must hold batch_size*n_kv_heads*head_dim = "
                             f"{cache.batch_size * e_kv} elements, got {t.numel()}")
    if new_k.dtype != new_v.dtype:
        raise ValueError("new_k and new_v must share a dtype")
    _check_tensor(q, "q_new", dev)
    _check_tensor(out, "output", dev)
    e_q = cache.n_heads * cache.head_dim
    if q.numel() != cache.batch_size * e_q or out.numel() != cache.batch_size * e_q:
        raise ValueError(f"q_new/output must hold batch_size*n_heads*head_dim = "
                         f"{cache.batch_size * e_q} elements")
    batch_count(ctx)
    cap = cache.block_table.shape[1] * cache.block_size if cache.paged else cache.max_seq_len
    after, top, total = _fills_after_append(layer.host_lens, cap)
    if max_len is None:
        max_len = top
    elif max_len < top:
        _check_max_len(max_len, after)  # raises
    # every fill is <= max_len here, so the total needs no clamp
    chunk, nchunks = _decode_plan_span(ctx, cache.batch_size, cache.n_heads, cache.n_kv_heads,
                                       max_len, total, cache.head_dim, cache.dtype)
    L = _lib.lib()
    need = _decode_ws_bytes(cache.batch_size, cache.n_heads, cache.head_dim, nchunks)
    ws = _workspace(ctx, need)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(cache.head_dim)
    stream = _lib.stream_handle(dev)
    cdt, idt = _lib.dtype_code(cache.dtype), _lib.dtype_code(new_k.dtype)
    qdt, odt = _lib.dtype_code(q.dtype), _lib.dtype_code(out.dtype)
    kc, vc = layer.k_cache.buffer.data_ptr(), layer.v_cache.buffer.data_ptr()
    if cache.paged:
        rc = L.skv_append_decode_attn_paged(
            out.data_ptr(), q.data_ptr(), kc, vc, new_k.data_ptr(), new_v.data_ptr(),
            layer.lens.data_ptr(), cache.block_table.data_ptr(), cache.block_table.shape[1],
            cache.block_size, cache.batch_size, cache.n_heads, cache.n_kv_heads, cache.head_dim,
            sc, chunk, nchunks, ws.data_ptr(), ws.numel(), cdt, idt, qdt, odt, stream)
    else:
        rc = L.skv_append_decode_attn(
            out.data_ptr(), q.data_ptr(), kc, vc, new_k.data_ptr(), new_v.data_ptr(),
            layer.lens.data_ptr(), cache.batch_size, cache.n_heads, cache.n_kv_heads,
            cache.head_dim, cache.max_seq_len, sc, chunk, nchunks, ws.data_ptr(), ws.numel(), cdt,
            idt, qdt, odt, stream)
    _lib.check(rc, "skv_append_decode_attn")
    layer.host_lens = after
    return after.copy()


def attention_with_kv_cache(ctx: GPUContext, cache: KVCache, layer_idx: int, q_new: GPUBuffer2D,
                            output: GPUBuffer2D) -> None:
    """Attention of the newest query over the cached K/V (reference :194-289).

    q_new, output: [batch_size, n_heads * head_dim]. Sequence b attends
    positions [0, fill_b) of layer layer_idx, which include the token the
    last update appended. Raises ValueError on a bad layer index, an empty
    layer or a shape mismatch. No length cap.
    """
    _check_layer(cache, layer_idx)
    layer = cache.layers[layer_idx]
    if int(layer.host_lens.max()) == 0:
        raise ValueError("Cache is empty: current_len=0")
    e_q = cache.n_heads * cache.head_dim
    expected_q_rows = cache.batch_size * 1
    validate_buffer_shape_2d(q_new, (expected_q_rows, e_q), "q_new")
    validate_buffer_shape_2d(output, (expected_q_rows, e_q), "output")
    batch_count(ctx)
    decode_attention(ctx, cache, layer_idx, q_new.buffer, output.buffer)


# ============================================================================
# CHUNKED PREFILL (extension; the reference appends one token per call)
# ============================================================================


def _prefill_workspace(ctx: GPUContext, nbytes: int) -> Optional[torch.Tensor]:
    if nbytes == 0:
        return None
    ws = ctx.prefill_workspace
    if ws is None or ws.numel() < nbytes or ws.device != ctx.device:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=ctx.device)
        ctx.prefill_workspace = ws
    return ws


def kv_cache_prefill(ctx: GPUContext, cache: KVCache, layer_idx: int, new_k: torch.Tensor,
                     new_v: torch.Tensor, q: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, n_new=None,
                     scale: Optional[float] = None, n_splits: int = 0) -> np.ndarray:
    """Append a chunk of up to C tokens per sequence to one layer and, if q is
    given, attend the chunk's queries causally over prefix + chunk.

    new_k, new_v: [batch_size, C, n_kv_heads, head_dim] device tensors (float32
    or bfloat16). q, out: [batch_size, C, n_heads, head_dim]. n_new: optional
    per-sequence token counts (<= C) for a ragged chunk; rows i >= n_new[b] of
    out are zeros. Query row i of sequence b sits at position fill_b + i and
    attends positions [0, fill_b + i] (the causal mask of the reference's
    flash_attention, gpu/gpu_kernels.py:695-701, shifted by the cached
    prefix). The layer's fills advance by n_new. Returns the new fills.

    A bfloat16 cache runs the bf16 MFMA prefill; a float32 cache runs every
    product in fp32 (float32 q and out).

    Raises ValueError (before any GPU work) on a bad layer, shapes, a chunk
    that would overflow a sequence ("Cache is full"), a paged cache, or a
    float32 cache with non-float32 q/output.
    """
    _check_layer(cache, layer_idx)
    if cache.paged:
        raise ValueError("kv_cache_prefill: paged caches take single-token appends only")
    layer = cache.layers[layer_idx]
    dev = layer.lens.device
    B, Hq, Hkv, D, T = (cache.batch_size, cache.n_heads, cache.n_kv_heads, cache.head_dim,
                        cache.max_seq_len)
    for t, nm in ((new_k, "new_k"), (new_v, "new_v")):
        _check_tensor(t, nm, dev)
        if t.dim() != 4 or t.shape[0] != B or t.shape[2] != Hkv or t.shape[3] != D:
            raise ValueError(f"{nm} must be [batch_size, C, n_kv_heads, head_dim] = "
                             f"[{B}, C, {Hkv}, {D}], got {tuple(t.shape)}")
    if new_k.shape != new_v.shape or new_k.dtype != new_v.dtype:
        raise ValueError("new_k and new_v must share shape and dtype")
    C = int(new_k.shape[1])
    if C <= 0:
        raise ValueError("the chunk must hold at least one token")
    n_host = (np.full(B, C, np.int64) if n_new is None
              else np.asarray(n_new, dtype=np.int64).reshape(B))
    if (n_host < 0).any() or (n_host > C).any():
        raise ValueError(f"n_new entries must lie in [0, {C}]")
    start = layer.host_lens.copy()
    if int((start + n_host).max()) > T:
        raise ValueError(f"Cache is full: chunk of {int(n_host.max())} tokens after "
                         f"current_len={int(start.max())}, max_seq_len={T}")
    want_attn = q is not None
    if want_attn:
        if out is None:
            raise ValueError("kv_cache_prefill: out is required with q")
        for t, nm in ((q, "q"), (out, "output")):
            _check_tensor(t, nm, dev)
            if tuple(t.shape) != (B, C, Hq, D):
                raise ValueError(f"{nm} must be [{B}, {C}, {Hq}, {D}], got {tuple(t.shape)}")
        if cache.dtype == torch.float32 and (q.dtype != torch.float32 or
                                             out.dtype != torch.float32):
            raise ValueError("kv_cache_prefill: attention over a float32 cache takes float32 "
                             "q and output")
    batch_count(ctx)
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    cdt, idt = _lib.dtype_code(cache.dtype), _lib.dtype_code(new_k.dtype)
    n_dev = (None if n_new is None else
             torch.from_numpy(n_host.astype(np.int32)).to(dev, non_blocking=False))
    n_ptr = n_dev.data_ptr() if n_dev is not None else None
    kc, vc = layer.k_cache.buffer, layer.v_cache.buffer
    if want_attn:
        ns = ctypes.c_int()
        if n_splits > 0:
            ns.value = int(n_splits)
        else:
            _lib.check(L.skv_prefill_plan(B, C, Hq, Hkv, int((start + n_host).max()),
                                          ctypes.byref(ns)), "skv_prefill_plan")
        need = L.skv_prefill_workspace_bytes(B, C, Hq, D, ns.value)
        ws = _prefill_workspace(ctx, need)
        sc = float(scale) if scale is not None else 1.0 / float(np.sqrt(D))
        # chunk append + attention + fill advance in one call
        rc = L.skv_append_prefill_attn(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                       new_k.data_ptr(), new_v.data_ptr(), layer.lens.data_ptr(),
                                       n_ptr, B, C, Hq, Hkv, D, T, sc, ns.value,
                                       ws.data_ptr() if ws is not None else None,
                                       ws.numel() if ws is not None else 0, cdt, idt,
                                       _lib.dtype_code(q.dtype), _lib.dtype_code(out.dtype),
                                       stream)
        _lib.check(rc, "skv_append_prefill_attn")
    else:
        rc = L.skv_append_chunk(kc.data_ptr(), vc.data_ptr(), new_k.data_ptr(),
                                new_v.data_ptr(), layer.lens.data_ptr(), n_ptr, B, C, Hkv, D, T,
                                cdt, idt, stream)
        _lib.check(rc, "skv_append_chunk")
        rc = L.skv_advance(layer.lens.data_ptr(), n_ptr, C, B, T, stream)
        _lib.check(rc, "skv_advance")
    layer.host_lens = np.minimum(start + n_host, T)
    return layer.host_lens.copy()
