"""Where the paged KV cache lives.

The interface is the reference's (app/memory/strategies.py:35-70): a
strategy allocates the two caches in the fixed 5-D layout (num_layers,
total_blocks, block_size, num_kv_heads, head_dim) and copies blocks.  The
difference is the ROCm branch: the reference's HipZeroCopyStrategy
(strategies.py:132-155) keeps the cache in pinned HOST memory; here a ROCm
device gets :class:`DeviceKVCacheStrategy`, which places both caches in HBM
where the HIP kernels read them, and pinned host memory is only the swap
space that preempted sequences' blocks move to (:meth:`allocate_host_pool`).
"""

from __future__ import annotations

import os
from abc import ABC, abstractmethod
from typing import Tuple, Union

import torch

# Names accepted for LLM_DTYPE / a dtype argument (strategies.py:14-32).
_DTYPE_NAMES = {
    torch.float16: ("fp16", "float16"),
    torch.bfloat16: ("bf16", "bfloat16"),
    torch.float32: ("fp32", "float32"),
}
_DTYPE_BY_NAME = {name: dtype for dtype, names in _DTYPE_NAMES.items() for name in names}


def resolve_device(device: Union[str, torch.device, None] = None) -> torch.device:
    """The store's device: the argument, else $LLM_DEVICE, where "auto" (the
    default) is the GPU when one is visible (strategies.py:7-11)."""
    name = device if device is not None and device != "" else os.getenv("LLM_DEVICE", "auto")
    if name == "auto":
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    return torch.device(name)


def resolve_dtype(dtype: Union[str, torch.dtype, None] = None) -> torch.dtype:
    """The cache dtype: a torch dtype as is, else a name from the argument or
    $LLM_DTYPE; "auto" (the default) is bf16 with a GPU and fp32 without
    (strategies.py:14-32).  An unknown name is a ValueError."""
    if isinstance(dtype, torch.dtype):
        return dtype
    name = (dtype or os.getenv("LLM_DTYPE", "auto")).lower()
    if name == "auto":
        return torch.bfloat16 if torch.cuda.is_available() else torch.float32
    if name not in _DTYPE_BY_NAME:
        raise ValueError(f"Unsupported dtype: {name}")
    return _DTYPE_BY_NAME[name]


def cache_shape(total_blocks: int, block_size: int, num_layers: int, num_heads: int, head_dim: int):
    """(num_layers, total_blocks, block_size, num_kv_heads, head_dim)."""
    return (int(num_layers), int(total_blocks), int(block_size), int(num_heads), int(head_dim))


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

    def allocate_host_pool(self, total_cpu_blocks: int, block_size: int, num_layers: int, num_heads: int,
                           head_dim: int, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """Swap space for preempted sequences' blocks, same block shape as the
        caches.  Only a store whose caches are not host memory has one."""
        raise RuntimeError(f"{type(self).__name__} has no host swap pool")


class CpuKVCacheStrategy(KVCacheMemoryStrategy):
    """Both caches in host memory (strategies.py:73-97): the reference's CPU
    path, kept for CPU runs of the operator API."""

    @property
    def device(self) -> torch.device:
        return torch.device("cpu")

    def allocate_cache(self, total_blocks, block_size, num_layers, num_heads, head_dim, dtype):
        shape = cache_shape(total_blocks, block_size, num_layers, num_heads, head_dim)
        return torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)

    def copy_blocks(self, src_cache, dst_cache, physical_blocks):
        """The named physical blocks of every layer, src -> dst."""
        if len(physical_blocks):
            ids = torch.as_tensor(list(physical_blocks), dtype=torch.long)
            dst_cache.index_copy_(1, ids, src_cache.index_select(1, ids))

    def sync(self) -> None:
        return None

    @property
    def requires_copy_on_swap(self) -> bool:
        return False


class DeviceKVCacheStrategy(KVCacheMemoryStrategy):
    """Both caches in HBM of one ROCm device.

    Allocated once, zero-filled, through torch's caching allocator; the HIP
    kernels address them directly.  At 288 GB of HBM per MI355X the pool is
    sized by the caller's budget, not by host RAM.  Preempted sequences swap
    to a pinned host pool (:meth:`allocate_host_pool`) through the HIP swap
    kernel (pa_swap_blocks).
    """

    def __init__(self, device_id: int = 0) -> None:
        self._device = torch.device("cuda", device_id)

    @property
    def device(self) -> torch.device:
        return self._device

    def allocate_cache(self, total_blocks, block_size, num_layers, num_heads, head_dim, dtype):
        shape = cache_shape(total_blocks, block_size, num_layers, num_heads, head_dim)
        return (torch.zeros(shape, dtype=dtype, device=self._device),
                torch.zeros(shape, dtype=dtype, device=self._device))

    def allocate_host_pool(self, total_cpu_blocks, block_size, num_layers, num_heads, head_dim, dtype):
        """Pinned (hipHostMalloc'd) host tensors the swap kernel maps into the
        device's address space."""
        shape = cache_shape(total_cpu_blocks, block_size, num_layers, num_heads, head_dim)
        return (torch.zeros(shape, dtype=dtype, pin_memory=True),
                torch.zeros(shape, dtype=dtype, pin_memory=True))

    def copy_blocks(self, src_cache, dst_cache, physical_blocks):
        """Copy the named physical blocks (every layer) from src_cache into
        dst_cache with the HIP block-copy kernel, on the current stream."""
        if not len(physical_blocks):
            return
        from .. import paged_ops

        paged_ops.copy_blocks(src_cache, dst_cache, [(int(b), int(b)) for b in physical_blocks])

    def sync(self) -> None:
        torch.cuda.current_stream(self._device).synchronize()

    @property
    def requires_copy_on_swap(self) -> bool:
        return True


def strategy_from_device(device: Union[str, torch.device]) -> KVCacheMemoryStrategy:
    """CPU -> host caches; a ROCm device -> HBM caches on that device
    (strategies.py:162-168 maps ROCm to pinned host memory instead)."""
    dev = torch.device(device)
    if dev.type == "cuda":
        return DeviceKVCacheStrategy(device_id=dev.index if dev.index is not None else 0)
    return CpuKVCacheStrategy()


def detect_strategy() -> KVCacheMemoryStrategy:
    return strategy_from_device("cuda" if torch.cuda.is_available() else "cpu")
