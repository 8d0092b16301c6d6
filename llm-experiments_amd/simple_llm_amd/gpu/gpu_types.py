"""Types of the GPU layer, mirroring the reference's gpu_types.py.

Reference: simple-llm/src/gpu/gpu_types.py (GPUConfig 19-201, GPUBuffer1D/2D
212-235, BatchState 250-261, GPUContext 264-270, KVCacheLayer 403-421,
KVCache 424-445, KVCacheConfig 448-467).

Memory is owned by torch tensors on the ROCm device instead of wgpu buffers;
`GPUBuffer2D.buffer` is a contiguous 2-D tensor of the stated shape.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple, Union

import numpy as np
import torch


@dataclass
class GPUConfig:
    """Tunables that exist on this backend (reference: gpu_types.py:19-201).

    The reference's tile/workgroup presets select WGSL variants at runtime.
    Here kernels are compiled ahead of time for gfx950; what remains tunable
    is the decode split size and the batching limit. `attention_workgroup_size`
    is kept for API compatibility only: decode attention has no length cap.
    """

    max_batch_operations: int = 1000
    max_workgroups_per_dim: int = 2**31 - 1
    attention_workgroup_size: int = 256
    flash_attn_max_head_dim: int = 128
    flash_attn_br: int = 32
    flash_attn_bc: int = 32
    decode_chunk_tokens: int = 0  # 0: choose per call (skv_decode_plan)


@dataclass
class GPUBuffer1D:
    buffer: torch.Tensor
    shape: Tuple[int]
    size: int


@dataclass
class GPUBuffer2D:
    buffer: torch.Tensor
    shape: Tuple[int, int]
    size: int


GPUBufferAny = Union[GPUBuffer1D, GPUBuffer2D]


@dataclass
class PipelineCache:
    """Kept for API compatibility: kernels live precompiled in libskv.so."""

    pipelines: dict = field(default_factory=dict)
    bind_groups: dict = field(default_factory=dict)


@dataclass
class BatchState:
    """An open command batch (reference: gpu_types.py:250-261).

    HIP launches are stream ordered, so a batch records nothing; it enforces
    the reference's per-batch operation limit and begin/commit pairing.
    """

    encoder: Optional[object]
    retained_buffers: List[object] = field(default_factory=list)
    enable_profiling: bool = False
    operation_count: int = 0


@dataclass
class GPUContext:
    device: torch.device
    config: GPUConfig
    batch_state: Optional[BatchState]
    pipeline_cache: PipelineCache
    reduction_workspace: Optional[GPUBuffer1D] = None
    # split-K workspaces of decode and prefill attention, grown on demand
    decode_workspace: Optional[torch.Tensor] = None
    prefill_workspace: Optional[torch.Tensor] = None


class KVCacheLayer:
    """K/V storage of one transformer layer (reference: gpu_types.py:403-421).

    k_cache, v_cache: GPUBuffer2D of shape [batch_size * max_seq_len, E_kv]
    (contiguous layout) or [n_blocks * block_size, E_kv] (paged pool), where
    E_kv = n_kv_heads * head_dim.

    lens: int32 device tensor [batch_size], filled positions per sequence,
    advanced on the device by every append. host_lens mirrors it exactly on
    the host (every change the kernels make is deterministic), so validation
    never has to read the device.
    """

    def __init__(self, k_cache: GPUBuffer2D, v_cache: GPUBuffer2D,
                 lens: Optional[torch.Tensor] = None,
                 host_lens: Optional[np.ndarray] = None):
        self.k_cache = k_cache
        self.v_cache = v_cache
        self.lens = lens
        self.host_lens = host_lens

    def __repr__(self) -> str:
        return f"KVCacheLayer(k_cache={self.k_cache.shape}, v_cache={self.v_cache.shape})"


class KVCache:
    """KV cache for all layers (reference: gpu_types.py:424-445).

    Fields of the reference: layers, batch_size, max_seq_len, current_len,
    n_heads, head_dim. Extensions (defaults reproduce the reference):
    n_kv_heads (grouped-query attention), dtype (float32 or bfloat16
    storage), block_size / n_blocks / block_table (paged layout).

    current_len is the number of filled positions. Each layer tracks its own
    fill, so updating layers 0..L-1 once per token writes every layer at the
    same position (the reference increments one shared counter per layer
    call, gpu_kv_cache.py:186, which its own docstring at :138-141 says the
    caller should do once per token). Reading current_len returns the
    longest fill over layers and sequences; on a cache updated one layer at a
    time, as in the reference's test (gpu_test.py:2275-2301), that is the
    number of updates, as there. Assigning current_len sets every layer and
    sequence to that fill.
    """

    def __init__(self, layers: List[KVCacheLayer], batch_size: int, max_seq_len: int,
                 current_len: int, n_heads: int, head_dim: int,
                 n_kv_heads: Optional[int] = None, dtype: torch.dtype = torch.float32,
                 block_size: int = 0, n_blocks: int = 0,
                 block_table: Optional[torch.Tensor] = None):
        self.layers = layers
        self.batch_size = batch_size
        self.max_seq_len = max_seq_len
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.n_kv_heads = n_kv_heads or n_heads
        self.dtype = dtype
        self.block_size = block_size
        self.n_blocks = n_blocks
        self.block_table = block_table
        self.current_len = current_len

    @property
    def paged(self) -> bool:
        return self.block_size > 0

    @property
    def current_len(self) -> int:
        return int(max(int(layer.host_lens.max()) for layer in self.layers))

    @current_len.setter
    def current_len(self, value: int) -> None:
        value = int(value)
        for layer in self.layers:
            layer.host_lens[:] = value
            layer.lens.fill_(value)

    def seq_lens(self, layer_idx: int = 0) -> np.ndarray:
        """Filled positions per sequence of one layer (host mirror)."""
        return self.layers[layer_idx].host_lens.copy()

    def __repr__(self) -> str:
        return (f"KVCache(layers={len(self.layers)}, batch_size={self.batch_size}, "
                f"max_seq_len={self.max_seq_len}, current_len={self.current_len}, "
                f"n_heads={self.n_heads}, n_kv_heads={self.n_kv_heads}, "
                f"head_dim={self.head_dim}, dtype={self.dtype}, block_size={self.block_size})")


@dataclass
class KVCacheConfig:
    """KV cache allocation request (reference: gpu_types.py:448-467).

    The first five fields are the reference's. Extensions:
      n_kv_heads  kv heads for grouped-query attention (None: n_heads)
      dtype       storage dtype, torch.float32 or torch.bfloat16
      block_size  > 0 selects the paged layout with pages of this many tokens
                  (a power of two); max_seq_len is then the per-sequence limit
      n_blocks    pages in the pool (0: batch_size * ceil(max_seq_len/block_size))
    """

    batch_size: int
    max_seq_len: int
    n_layers: int
    n_heads: int
    head_dim: int
    n_kv_heads: Optional[int] = None
    dtype: torch.dtype = torch.float32
    block_size: int = 0
    n_blocks: int = 0
