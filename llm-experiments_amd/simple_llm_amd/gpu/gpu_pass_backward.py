"""Training-side attention: causal FlashAttention backward on gfx950.

Drop-in for flash_attention_backward of simple-llm/src/gpu/gpu_pass_backward.py:445-580:
same arguments, checks and error messages. The reference runs one stage-1
pass per Q block, each writing partial dK/dV into grad_K_workspace and
grad_V_workspace, then a reduce pass (gpu/gpu_kernels.py:2038-2455). Here
skv_flash_bwd computes dQ and then dK/dV in two MFMA kernels with no
partials; the caller's workspaces are still required and shape-checked as in
the reference, and the row deltas (batch_size * seq_len * n_heads floats)
are kept in the first bytes of grad_K_workspace.
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


def flash_attention_backward(
    ctx: GPUContext,
    Q: GPUBuffer2D,
    K: GPUBuffer2D,
    V: GPUBuffer2D,
    O: GPUBuffer2D,
    L: GPUBuffer1D,
    M: GPUBuffer1D,
    grad_O: GPUBuffer2D,
    grad_Q: GPUBuffer2D,
    grad_K_workspace: GPUBuffer2D,
    grad_V_workspace: GPUBuffer2D,
    grad_K: GPUBuffer2D,
    grad_V: GPUBuffer2D,
    batch_size: int,
    seq_len: int,
    n_heads: int,
    head_dim: int,
) -> None:
    """Gradients of causal attention (reference: gpu_pass_backward.py:445-580).

    Q, K, V, O, grad_O, grad_Q, grad_K, grad_V: [batch_size*seq_len, n_heads*head_dim];
    L, M: [batch_size*seq_len*n_heads], the forward's softmax sums and row maxima;
    grad_K_workspace, grad_V_workspace: [num_q_blocks*batch_size*seq_len, n_heads*head_dim],
    num_q_blocks = ceil(seq_len / ctx.config.flash_attn_br).
    Raises ValueError on a bad shape or dimension, as the reference does.
    """
    config = ctx.config
    if head_dim > config.flash_attn_max_head_dim:
        raise ValueError(
            f"head_dim {head_dim} exceeds maximum supported by config: "
            f"{config.flash_attn_max_head_dim}")
    if batch_size <= 0 or seq_len <= 0 or n_heads <= 0 or head_dim <= 0:
        raise ValueError(
            f"Invalid dimensions: batch_size={batch_size}, seq_len={seq_len}, "
            f"n_heads={n_heads}, head_dim={head_dim}")

    embedding_dim = n_heads * head_dim
    total_tokens = batch_size * seq_len
    stats_size = batch_size * seq_len * n_heads
    validate_buffer_shape_2d(Q, (total_tokens, embedding_dim), "Q")
    validate_buffer_shape_2d(K, (total_tokens, embedding_dim), "K")
    validate_buffer_shape_2d(V, (total_tokens, embedding_dim), "V")
    validate_buffer_shape_2d(O, (total_tokens, embedding_dim), "O")
    validate_buffer_shape_1d(L, stats_size, "L")
    validate_buffer_shape_1d(M, stats_size, "M")
    validate_buffer_shape_2d(grad_O, (total_tokens, embedding_dim), "grad_O")
    validate_buffer_shape_2d(grad_Q, (total_tokens, embedding_dim), "grad_Q")
    validate_buffer_shape_2d(grad_K, (total_tokens, embedding_dim), "grad_K")
    validate_buffer_shape_2d(grad_V, (total_tokens, embedding_dim), "grad_V")
    num_q_blocks = (seq_len + config.flash_attn_br - 1) // config.flash_attn_br
    workspace_tokens = num_q_blocks * total_tokens
    validate_buffer_shape_2d(grad_K_workspace, (workspace_tokens, embedding_dim),
                             "grad_K_workspace")
    validate_buffer_shape_2d(grad_V_workspace, (workspace_tokens, embedding_dim),
                             "grad_V_workspace")

    names = ("Q", "K", "V", "O", "L", "M", "grad_O", "grad_Q", "grad_K_workspace", "grad_K",
             "grad_V")
    bufs = (Q, K, V, O, L, M, grad_O, grad_Q, grad_K_workspace, grad_K, grad_V)
    q, k, v, o, lt, mt, go, gq, ws, gk, gv = (_f32(b, n) for b, n in zip(bufs, names))
    lib = _lib.lib()
    batch_count(ctx)
    rc = lib.skv_flash_bwd(gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), q.data_ptr(),
                           k.data_ptr(), v.data_ptr(), o.data_ptr(), lt.data_ptr(), mt.data_ptr(),
                           go.data_ptr(), batch_size, seq_len, n_heads, head_dim,
                           float(1.0 / np.sqrt(head_dim)), ws.data_ptr(),
                           ws.numel() * ws.element_size(), _lib.stream_handle(q.device))
    _lib.check(rc, "skv_flash_bwd")


__all__ = ["flash_attention_backward"]
