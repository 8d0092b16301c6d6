"""Facade of the GPU layer (reference: simple-llm/src/gpu/gpu.py:30-35, 152-155).

Re-exports the names the reference's hot path and its tests use:
`gpu.kv_cache_create`, `gpu.KVCacheConfig`, `gpu.batch_begin`, ...
"""
from .gpu_buffer import (
    gpu_buffer_1d_create,
    gpu_buffer_1d_read,
    gpu_buffer_1d_write,
    gpu_buffer_2d_create,
    gpu_buffer_2d_read,
    gpu_buffer_2d_write,
    gpu_buffer_from_tensor,
    gpu_buffer_zerofy,
)
from .gpu_device import context_create, device_config_create, device_create, pipeline_cache_create
from .gpu_kv_cache import (
    attention_with_kv_cache,
    decode_attention,
    decode_plan,
    kv_cache_append,
    kv_cache_append_attend,
    kv_cache_create,
    kv_cache_prefill,
    kv_cache_reset,
    kv_cache_set_block_table,
    kv_cache_update,
)
from .gpu_pass_backward import flash_attention_backward
from .gpu_pass_forward import flash_attention
from .gpu_ops import batch_begin, batch_commit, validate_buffer_shape_1d, validate_buffer_shape_2d
from .gpu_types import (
    BatchState,
    GPUBuffer1D,
    GPUBuffer2D,
    GPUConfig,
    GPUContext,
    KVCache,
    KVCacheConfig,
    KVCacheLayer,
    PipelineCache,
)

__all__ = [
    # Types
    "GPUBuffer1D",
    "GPUBuffer2D",
    "GPUConfig",
    "GPUContext",
    "BatchState",
    "PipelineCache",
    "KVCache",
    "KVCacheConfig",
    "KVCacheLayer",
    # Device
    "device_create",
    "device_config_create",
    "pipeline_cache_create",
    "context_create",
    # Buffers
    "gpu_buffer_1d_create",
    "gpu_buffer_2d_create",
    "gpu_buffer_1d_write",
    "gpu_buffer_2d_write",
    "gpu_buffer_1d_read",
    "gpu_buffer_2d_read",
    "gpu_buffer_zerofy",
    "gpu_buffer_from_tensor",
    # Ops
    "batch_begin",
    "batch_commit",
    "validate_buffer_shape_1d",
    "validate_buffer_shape_2d",
    # KV-cache
    "kv_cache_create",
    "kv_cache_reset",
    "kv_cache_update",
    "attention_with_kv_cache",
    "kv_cache_append",
    "kv_cache_append_attend",
    "kv_cache_prefill",
    "kv_cache_set_block_table",
    "decode_attention",
    "decode_plan",
    # Training-side attention
    "flash_attention",
    "flash_attention_backward",
]
