"""Where the paged KV cache lives.

Same interface as the reference's app/memory/strategies.py:35-70 and the
same 5-D layout (num_layers, total_blocks, block_size, num_kv_heads,
head_dim).  The difference is the ROCm branch: the reference's
HipZeroCopyStrategy (strategies.py:132-155) keeps the cache in pinned HOST
memory; here a ROCm device gets :class:`DeviceKVCacheStrategy`, which places
both caches in HBM where the HIP kernels read them.
"""

from __future__ import annotations

import os
from abc import ABC, abstractmethod
from typing import Tuple, Union

import torch


def resolve_device(device: Union[str, torch.device, None] = None) -> torch.device:
    """strategies.py:7-11: "auto" -> cuda when available, else cpu."""
    requested = device or os.getenv("LLM_DEVICE", "auto")
    if requested == "auto":
        requested = "cuda" if torch.cuda.is_available() else "cpu"
    return torch.device(requested)


def resolve_dtype(dtype: Union[str, torch.dtype, None] = None) -> torch.dtype:
    """strategies.py:14-32: "auto" -> bf16 on a GPU, else fp32."""
    requested = dtype or os.getenv("LLM_DTYPE", "auto")
    if isinstance(requested, torch.dtype):
        return requested
    requested = requested.lower()
    if requested == "auto":
        return torch.bfloat16 if torch.cuda.is_available() else torch.float32
    aliases = {
        "fp16": torch.float16,
        "float16": torch.float16,
        "bf16": torch.bfloat16,
        "bfloat16": torch.bfloat16,
        "fp32": torch.float32,
        "float32": torch.float32,
    }
    try:
        return aliases[requested]
    except KeyError as exc:
        raise ValueError(f"Unsupported dtype: {requested}") from exc


class KVCacheMemoryStrategy(ABC):
    @abstractmethod
    def allocate_cache(self, total_blocks: int, block_size: int, num_layers: int, num_heads: int,
                       head_dim: int, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        ...

    @abstractmethod
    def copy_blocks(self, src_cache: torch.Tensor, dst_cache: torch.Tensor, physical_blocks: list) -> None:
        ...

    @abstractmethod
    def sync(self) -> None:
        ...

    @property
    @abstractmethod
    def device(self) -> torch.device:
        ...

    @property
    @abstractmethod
    def requires_copy_on_swap(self) -> bool:
        ...


def _cache_shape(total_blocks, block_size, num_layers, num_heads, head_dim):
    return (num_layers, total_blocks, block_size, num_heads, head_dim)


class CpuKVCacheStrategy(KVCacheMemoryStrategy):
    """Host cache (strategies.py:73-97)."""

    def __init__(self) -> None:
        self._device = torch.device("cpu")

    @property
    def device(self) -> torch.device:
        return self._device

    def allocate_cache(self, total_blocks, block_size, num_layers, num_heads, head_dim, dtype):
        shape = _cache_shape(total_blocks, block_size, num_layers, num_heads, head_dim)
        return torch.empty(shape, dtype=dtype), torch.empty(shape, dtype=dtype)

    def copy_blocks(self, src_cache, dst_cache, physical_blocks):
        for bid in physical_blocks:
            dst_cache[:, bid].copy_(src_cache[:, bid])

    def sync(self) -> None:
        pass

    @property
    def requires_copy_on_swap(self) -> bool:
        return False


class DeviceKVCacheStrategy(KVCacheMemoryStrategy):
    """Both caches in HBM of one ROCm device.

    Allocated once, zero-filled, through torch's caching allocator on the
    device's current stream; the HIP kernels address them directly.  At
    288 GB of HBM per MI355X the pool is sized by the caller's budget, not
    by host RAM.
    """

    def __init__(self, device_id: int = 0) -> None:
        self._device = torch.device("cuda", device_id)

    @property
    def device(self) -> torch.device:
        return self._device

    def allocate_cache(self, total_blocks, block_size, num_layers, num_heads, head_dim, dtype):
        shape = _cache_shape(total_blocks, block_size, num_layers, num_heads, head_dim)
        key_cache = torch.zeros(shape, dtype=dtype, device=self._device)
        value_cache = torch.zeros(shape, dtype=dtype, device=self._device)
        return key_cache, value_cache

    def copy_blocks(self, src_cache, dst_cache, physical_blocks):
        """Copy the named physical blocks (every layer) from src_cache into
        dst_cache with the HIP block-copy kernel, on the current stream."""
        if not physical_blocks:
            return
        from .. import paged_ops

        ids = [int(b) for b in physical_blocks]
        paged_ops.copy_blocks(src_cache, dst_cache, [(b, b) for b in ids])

    def sync(self) -> None:
        torch.cuda.current_stream(self._device).synchronize()

    @property
    def requires_copy_on_swap(self) -> bool:
        return True


def strategy_from_device(device: Union[str, torch.device]) -> KVCacheMemoryStrategy:
    """strategies.py:162-168, with the ROCm device mapped to HBM."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return CpuKVCacheStrategy()
    return DeviceKVCacheStrategy(device_id=dev.index or 0)


def detect_strategy() -> KVCacheMemoryStrategy:
    if not torch.cuda.is_available():
        return CpuKVCacheStrategy()
    return strategy_from_device("cuda")
