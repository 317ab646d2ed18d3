"""Paged KV pool layout and the block bookkeeping the decode runner needs.

This module sits at the reference's path, engine/memory/block_allocator.py, and
exports the names the reference's kernel integration imports from it
(engine/kernels/paged_attention_integration.py:24, and compute_num_blocks at
:252): PhysicalBlockPool, BlockTable, BlockAllocator, compute_num_blocks. So
this package's engine/kernels/ files run unchanged on top of either this
module or the reference's own.

PhysicalBlockPool keeps the reference's layout contract
(block_allocator.py:69-101): per layer one K and one V tensor of shape
[num_blocks, block_size, num_kv_heads, head_dim], allocated with torch.empty
(uninitialised). BlockTable keeps the reference's fields and helpers
(block_allocator.py:292-319): physical ids in logical order and the token
count that is the single source of KV occupancy.

BlockAllocator here is a plain LIFO free list with reference counts: the
surface the runner, the tests and the benchmark use (allocate, free, fork,
can_allocate, ref_counts; reference block_allocator.py:143-270). The
reference's prefix cache and LRU pool of cached free blocks sit above the
kernel boundary and are not rebuilt; the runner reads only allocate() and
ref_counts, which the reference's allocator has too.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

import torch


def _kv_dims(model_config: Any) -> tuple:
    """(layers, kv heads, head_dim) of a transformers-style config."""
    layers = getattr(model_config, "num_hidden_layers", None)
    heads = getattr(model_config, "num_attention_heads", None)
    kv_heads = getattr(model_config, "num_key_value_heads", None) or heads
    head_dim = getattr(model_config, "head_dim", None)
    if not head_dim and heads:
        head_dim = getattr(model_config, "hidden_size", 0) // heads
    if not (layers and kv_heads and head_dim):
        raise ValueError(f"cannot infer the KV shape from {type(model_config).__name__}: "
                         f"layers={layers}, kv_heads={kv_heads}, head_dim={head_dim}")
    return int(layers), int(kv_heads), int(head_dim)


def compute_num_blocks(model_config: Any, block_size: int, gpu_memory_utilization: float = 0.9,
                       device: Optional[torch.device | str] = None,
                       dtype: torch.dtype = torch.float16) -> int:
    """Blocks that fit `gpu_memory_utilization` of the device's free memory.

    A block costs K and V rows of every layer: 2 * layers * block_size *
    kv_heads * head_dim * element bytes (reference block_allocator.py:20-64).
    """
    dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
    if dev.type != "cuda":
        raise ValueError(f"compute_num_blocks needs a GPU device, got {dev}")
    layers, kv_heads, head_dim = _kv_dims(model_config)
    per_block = (2 * layers * block_size * kv_heads * head_dim
                 * torch.tensor([], dtype=dtype).element_size())
    free, _total = torch.cuda.mem_get_info(dev)
    return int(free * gpu_memory_utilization) // per_block


@dataclass
class PhysicalBlockPool:
    num_blocks: int
    block_size: int
    num_layers: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype = torch.float16
    device: Optional[torch.device | str] = None
    k_cache: list = field(init=False)
    v_cache: list = field(init=False)

    def __post_init__(self):
        self.device = torch.device(self.device or ("cuda" if torch.cuda.is_available() else "cpu"))
        shape = (self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim)
        self.k_cache = [torch.empty(shape, dtype=self.dtype, device=self.device)
                        for _ in range(self.num_layers)]
        self.v_cache = [torch.empty(shape, dtype=self.dtype, device=self.device)
                        for _ in range(self.num_layers)]

    @property
    def total_vram_bytes(self) -> int:
        elem = torch.tensor([], dtype=self.dtype).element_size()
        return (2 * self.num_layers * self.num_blocks * self.block_size * self.num_kv_heads
                * self.head_dim * elem)

    @classmethod
    def from_model_config(cls, model_config: Any, block_size: int = 16,
                          gpu_memory_utilization: float = 0.9,
                          device: Optional[torch.device | str] = None,
                          dtype: torch.dtype = torch.float16) -> "PhysicalBlockPool":
        layers, kv_heads, head_dim = _kv_dims(model_config)
        n = compute_num_blocks(model_config, block_size, gpu_memory_utilization, device, dtype)
        return cls(num_blocks=n, block_size=block_size, num_layers=layers,
                   num_kv_heads=kv_heads, head_dim=head_dim, dtype=dtype, device=device)


@dataclass
class BlockTable:
    seq_id: int
    block_size: int
    physical_block_ids: list = field(default_factory=list)
    num_tokens: int = 0

    def num_blocks_needed_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def last_block_has_space(self) -> bool:
        if not self.physical_block_ids:
            return False
        return self.num_tokens % self.block_size != 0

    def free(self, allocator) -> None:
        for b in self.physical_block_ids:
            allocator.free(b)
        self.physical_block_ids.clear()


class BlockAllocator:
    """LIFO free list of block ids with reference counts (shared blocks count > 1).

    `enable_prefix_cache` is accepted for the reference's constructor
    signature; this allocator keeps no cache, so it must be False.
    """

    def __init__(self, num_blocks: int, enable_prefix_cache: bool = False):
        if enable_prefix_cache:
            raise NotImplementedError("the prefix cache lives in the serving engine's allocator")
        self.num_blocks = num_blocks
        self.enable_prefix_cache = False
        self._free = list(range(num_blocks - 1, -1, -1))
        self.ref_counts: dict[int, int] = {}

    def num_available(self) -> int:
        return len(self._free)

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    def get_free_block_count(self) -> int:
        return len(self._free)

    def can_allocate(self, n: int) -> bool:
        return len(self._free) >= n

    def allocate(self) -> int:
        if not self._free:
            raise MemoryError("no free KV blocks")
        b = self._free.pop()
        self.ref_counts[b] = 1
        return b

    def fork(self, block_id: int) -> int:
        if block_id not in self.ref_counts:
            raise ValueError(f"block {block_id} is not allocated")
        self.ref_counts[block_id] += 1
        return block_id

    def free(self, block_id: int) -> None:
        if block_id not in self.ref_counts:
            raise ValueError(f"double free of block {block_id}")
        self.ref_counts[block_id] -= 1
        if self.ref_counts[block_id] == 0:
            del self.ref_counts[block_id]
            self._free.append(block_id)

    release = free
