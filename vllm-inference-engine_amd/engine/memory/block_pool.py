"""Paged KV pool layout and minimal block bookkeeping for the decode runner.

PhysicalBlockPool keeps the reference's layout contract
(engine/memory/block_allocator.py:81-109): per layer one K and one V tensor of
shape [num_blocks, block_size, num_kv_heads, head_dim], allocated with
torch.empty (uninitialised). BlockTable keeps the reference's fields and
helpers (block_allocator.py:304-332): physical ids in logical order and the
token count that is the single source of KV occupancy.

FreeListAllocator is only what the runner, the tests and the benchmark need
to hand out block ids: a LIFO free list with reference counts. The
reference's allocator (prefix cache, LRU cached-free pool) and its scheduler
sit above the kernel boundary and are not part of this package; the runner
accepts any allocator with allocate() and ref_counts, as the reference's does.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


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


class FreeListAllocator:
    """LIFO free list of block ids with reference counts (shared blocks count > 1)."""

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self._free = list(range(num_blocks - 1, -1, -1))
        self.ref_counts: dict[int, int] = {}

    @property
    def num_free(self) -> int:
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
