"""Device and context creation (reference: simple-llm/src/gpu/gpu_device.py).

The reference requests a WebGPU adapter (gpu_device.py:23-49) and builds a
GPUConfig from per-vendor presets (:343-431). Here the device is the ROCm GPU
torch sees; kernels are compiled ahead of time for gfx950, so there is no
pipeline compilation and no vendor table.
"""
from __future__ import annotations

import torch

from .gpu_types import BatchState, GPUConfig, GPUContext, PipelineCache


def device_create(index: int = 0) -> torch.device:
    """The ROCm device; RuntimeError if there is none (reference :40-49)."""
    if not torch.cuda.is_available():
        raise RuntimeError("No GPU adapter found: torch reports no ROCm device")
    if torch.version.hip is None:
        raise RuntimeError("torch was not built for ROCm; this backend targets gfx950 only")
    dev = torch.device("cuda", index)
    arch = torch.cuda.get_device_properties(dev).gcnArchName
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"device {index} is {arch}; libskv.so is built for gfx950 only")
    return dev


def device_config_create(device: torch.device) -> GPUConfig:
    return GPUConfig()


def pipeline_cache_create(device: torch.device) -> PipelineCache:
    return PipelineCache()


def context_create(device: torch.device | None = None,
                   config: GPUConfig | None = None) -> GPUContext:
    """Convenience: device + config + empty batch state in one call."""
    dev = device if device is not None else device_create()
    return GPUContext(device=dev, config=config or device_config_create(dev),
                      batch_state=None, pipeline_cache=pipeline_cache_create(dev))


__all__ = ["device_create", "device_config_create", "pipeline_cache_create", "context_create",
           "BatchState"]
