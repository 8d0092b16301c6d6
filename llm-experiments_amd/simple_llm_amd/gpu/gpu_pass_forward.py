"""Training-side attention forward: causal FlashAttention with its row
statistics, fp32, on gfx950.

Drop-in for flash_attention of simple-llm/src/gpu/gpu_pass_forward.py:497-588:
same arguments, checks and error messages. The reference's WGSL kernel
(gpu/gpu_kernels.py:499-770) runs one workgroup per (query block, head,
sequence) with an online softmax over key blocks; skv_flash_fwd runs the same
computation on fp32 MFMA tiles and writes O, L (softmax sums) and M (row
maxima of the scaled scores), which flash_attention_backward consumes.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from .gpu_ops import batch_count, validate_buffer_shape_1d, validate_buffer_shape_2d
from .gpu_types import GPUBuffer1D, GPUBuffer2D, GPUContext


def _f32(buf, name: str) -> torch.Tensor:
    t = buf.buffer
    if t.dtype != torch.float32 or not t.is_contiguous() or t.device.type != "cuda":
        raise ValueError(f"{name} must be a contiguous float32 device buffer")
    return t


def flash_attention(
    ctx: GPUContext,
    Q: GPUBuffer2D,
    K: GPUBuffer2D,
    V: GPUBuffer2D,
    O: GPUBuffer2D,
    L: GPUBuffer1D,
    M: GPUBuffer1D,
    batch_size: int,
    seq_len: int,
    n_heads: int,
    head_dim: int,
) -> None:
    """Causal attention forward (reference: gpu_pass_forward.py:497-588).

    Q, K, V, O: [batch_size*seq_len, n_heads*head_dim]; L, M:
    [batch_size*seq_len*n_heads], indexed (b*seq_len + t)*n_heads + h.
    Raises ValueError on a bad shape or dimension, as the reference does.
    """
    if head_dim > ctx.config.flash_attn_max_head_dim:
        raise ValueError(
            f"head_dim {head_dim} exceeds maximum supported by config: "
            f"{ctx.config.flash_attn_max_head_dim}. "
            f"Increase flash_attn_max_head_dim in GPUConfig or use smaller head_dim.")
    if batch_size <= 0 or seq_len <= 0 or n_heads <= 0 or head_dim <= 0:
        raise ValueError(
            f"Invalid dimensions: batch_size={batch_size}, seq_len={seq_len}, "
            f"n_heads={n_heads}, head_dim={head_dim}")
    embedding_dim = n_heads * head_dim
    total_tokens = batch_size * seq_len
    validate_buffer_shape_2d(Q, (total_tokens, embedding_dim), "Q")
    validate_buffer_shape_2d(K, (total_tokens, embedding_dim), "K")
    validate_buffer_shape_2d(V, (total_tokens, embedding_dim), "V")
    validate_buffer_shape_2d(O, (total_tokens, embedding_dim), "O")
    stats_size = batch_size * seq_len * n_heads
    validate_buffer_shape_1d(L, stats_size, "L")
    validate_buffer_shape_1d(M, stats_size, "M")
    q, k, v, o, lt, mt = (_f32(b, n) for b, n in zip((Q, K, V, O, L, M),
                                                     ("Q", "K", "V", "O", "L", "M")))
    lib = _lib.lib()
    batch_count(ctx)
    rc = lib.skv_flash_fwd(o.data_ptr(), lt.data_ptr(), mt.data_ptr(), q.data_ptr(),
                           k.data_ptr(), v.data_ptr(), batch_size, seq_len, n_heads, head_dim,
                           float(1.0 / np.sqrt(head_dim)), _lib.stream_handle(q.device))
    _lib.check(rc, "skv_flash_fwd")


__all__ = ["flash_attention"]
