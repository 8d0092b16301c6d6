"""Command batching and shape validation (reference: simple-llm/src/gpu/gpu_ops.py).

On HIP every launch is enqueued on torch's current stream in program order,
so batch_begin/batch_commit do not defer work; they keep the reference's
contract: a per-batch operation limit (RuntimeError, gpu_ops.py:277-283),
and commit without an open batch is an error (:352-353). Ops may also be
issued outside a batch.
"""
from __future__ import annotations

from typing import Tuple

from .gpu_types import BatchState, GPUBuffer1D, GPUBuffer2D, GPUContext


def validate_buffer_shape_1d(buffer: GPUBuffer1D, expected_size: int, name: str) -> None:
    """Reference: gpu_ops.py:23-42."""
    if expected_size <= 0:
        raise ValueError(f"Invalid expected size for {name}: {expected_size}")
    if buffer.shape != (expected_size,):
        raise ValueError(
            f"{name} shape mismatch: got {buffer.shape}, expected ({expected_size},)")


def validate_buffer_shape_2d(buffer: GPUBuffer2D, expected_shape: Tuple[int, int],
                             name: str) -> None:
    """Reference: gpu_ops.py:45-64 (same checks and messages)."""
    if expected_shape[0] <= 0 or expected_shape[1] <= 0:
        raise ValueError(f"Invalid expected shape for {name}: {expected_shape}")
    if tuple(buffer.shape) != tuple(expected_shape):
        raise ValueError(
            f"{name} shape mismatch: got {buffer.shape}, expected {expected_shape}")


def batch_begin(ctx: GPUContext, enable_profiling: bool = False) -> None:
    ctx.batch_state = BatchState(encoder=object(), retained_buffers=[],
                                 enable_profiling=enable_profiling, operation_count=0)


def batch_count(ctx: GPUContext) -> None:
    """Count one operation against the open batch's limit (if a batch is open)."""
    st = ctx.batch_state
    if st is None or st.encoder is None:
        return
    max_ops = ctx.config.max_batch_operations
    if st.operation_count >= max_ops:
        raise RuntimeError(
            f"Batch operation limit ({max_ops}) exceeded. Call batch_commit() to flush operations.")
    st.operation_count += 1


def batch_commit(ctx: GPUContext) -> None:
    st = ctx.batch_state
    if st is None or st.encoder is None:
        raise RuntimeError("Batch already submitted or not initialized")
    st.encoder = None
    st.retained_buffers.clear()
