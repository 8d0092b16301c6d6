"""Device buffers on torch tensors (reference: simple-llm/src/gpu/gpu_buffer.py).

The reference creates wgpu storage buffers (fp32/int32/uint32 only,
gpu_buffer.py:31-39), zero-fills with queue.write_buffer (:121-129) and reads
back through a mapped staging buffer (:151-182). Here a buffer is a
contiguous device tensor; new buffers are zero-filled as WebGPU buffers are.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from .gpu_types import GPUBuffer1D, GPUBuffer2D, GPUBufferAny, GPUContext

_NP_TO_TORCH = {np.dtype(np.float32): torch.float32, np.dtype(np.int32): torch.int32,
                np.dtype(np.uint32): torch.int32}


def _tensor(ctx: GPUContext, shape, data: Optional[np.ndarray],
            dtype: Optional[torch.dtype]) -> torch.Tensor:
    if data is not None:
        if np.dtype(data.dtype) not in _NP_TO_TORCH:
            raise ValueError(f"Unsupported dtype: {data.dtype}. Supported: float32, int32, uint32")
        host = np.ascontiguousarray(data)
        if host.dtype == np.uint32:
            host = host.view(np.int32)
        t = torch.from_numpy(host.reshape(shape)).to(ctx.device)
        return t if dtype is None or dtype == t.dtype else t.to(dtype)
    return torch.zeros(shape, dtype=dtype or torch.float32, device=ctx.device)


def gpu_buffer_1d_create(ctx: GPUContext, size: int, data: Optional[np.ndarray] = None,
                         dtype: Optional[torch.dtype] = None) -> GPUBuffer1D:
    if size <= 0:
        raise ValueError(f"Buffer size must be positive, got {size}")
    if data is not None and data.shape != (size,):
        raise ValueError(f"Data shape {data.shape} doesn't match buffer size ({size},)")
    return GPUBuffer1D(buffer=_tensor(ctx, (size,), data, dtype), shape=(size,), size=size)


def gpu_buffer_2d_create(ctx: GPUContext, rows: int, cols: int,
                         data: Optional[np.ndarray] = None,
                         dtype: Optional[torch.dtype] = None) -> GPUBuffer2D:
    """2-D buffer; `dtype` (extension) selects e.g. torch.bfloat16 storage."""
    if rows <= 0 or cols <= 0:
        raise ValueError(f"Buffer dimensions must be positive, got ({rows}, {cols})")
    if data is not None and data.shape != (rows, cols):
        raise ValueError(f"Data shape {data.shape} doesn't match buffer shape ({rows}, {cols})")
    return GPUBuffer2D(buffer=_tensor(ctx, (rows, cols), data, dtype), shape=(rows, cols),
                       size=rows * cols)


def gpu_buffer_from_tensor(t: torch.Tensor) -> GPUBufferAny:
    """Wrap an existing contiguous 1-D or 2-D device tensor (no copy)."""
    if not t.is_contiguous():
        raise ValueError("buffer tensors must be contiguous")
    if t.dim() == 1:
        return GPUBuffer1D(buffer=t, shape=(t.shape[0],), size=t.numel())
    if t.dim() == 2:
        return GPUBuffer2D(buffer=t, shape=(t.shape[0], t.shape[1]), size=t.numel())
    raise ValueError(f"expected a 1-D or 2-D tensor, got {t.dim()}-D")


def gpu_buffer_zerofy(ctx: GPUContext, gpu_buffer: GPUBufferAny) -> None:
    gpu_buffer.buffer.zero_()


def _write(in_data: np.ndarray, buffer: GPUBufferAny) -> None:
    src = torch.from_numpy(np.ascontiguousarray(in_data, dtype=np.float32))
    buffer.buffer.copy_(src.reshape(buffer.buffer.shape).to(buffer.buffer.dtype))


def gpu_buffer_1d_write(ctx: GPUContext, in_data: np.ndarray, buffer: GPUBuffer1D) -> None:
    _write(in_data, buffer)


def gpu_buffer_2d_write(ctx: GPUContext, in_data: np.ndarray, buffer: GPUBuffer2D) -> None:
    _write(in_data, buffer)


def _read(buffer: GPUBufferAny, out_data: np.ndarray) -> None:
    """Synchronous read into a preallocated array (reference :151-182)."""
    host = buffer.buffer.detach().to("cpu")
    if host.dtype == torch.bfloat16:
        host = host.float()
    np.copyto(out_data, host.numpy().reshape(out_data.shape).astype(out_data.dtype, copy=False))


def gpu_buffer_1d_read(ctx: GPUContext, buffer: GPUBuffer1D, out_data: np.ndarray) -> None:
    _read(buffer, out_data)


def gpu_buffer_2d_read(ctx: GPUContext, buffer: GPUBuffer2D, out_data: np.ndarray) -> None:
    _read(buffer, out_data)
