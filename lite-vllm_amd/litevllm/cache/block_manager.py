"""Paged-KV block bookkeeping (host side).

Same interface and allocation order as the reference
(cache/block_manager.py:13-144): a free list handed out from its end (so the
first block given out is num_blocks - 1 and freed blocks are reused first),
reference counts for copy-on-write forks, per-sequence block tables.  The
block ids it hands out are what the packing kernel turns into slot_mapping
and block tables.  Addition: an optional evictor (the prefix cache) that is
asked to release cached-but-unused blocks when the free list runs dry.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Optional


@dataclass
class PhysicalBlock:
    block_id: int
    ref_count: int = 0
    is_cached: bool = False
    hash_value: Optional[int] = None


class BlockAllocator:
    """Free-list allocator; ``reserved_blocks`` leading ids are never handed out."""

    def __init__(self, num_blocks: int, device: str = "gpu", reserved_blocks: int = 0) -> None:
        self.device = device
        self.num_blocks = num_blocks
        self.reserved_blocks = reserved_blocks
        self.blocks = [PhysicalBlock(block_id=i) for i in range(num_blocks)]
        self.free_list: list[int] = list(range(reserved_blocks, num_blocks))

    @property
    def num_free_blocks(self) -> int:
        return len(self.free_list)

    def allocate(self) -> PhysicalBlock:
        if not self.free_list:
            raise RuntimeError(f"No free blocks on {self.device}")
        block = self.blocks[self.free_list.pop()]
        block.ref_count = 1
        return block

    def free(self, block: PhysicalBlock) -> None:
        block.ref_count -= 1
        if block.ref_count <= 0:
            block.ref_count = 0
            block.is_cached = False
            block.hash_value = None
            self.free_list.append(block.block_id)

    def ref(self, block: PhysicalBlock) -> None:
        block.ref_count += 1


@dataclass
class BlockTable:
    """Logical block index -> physical block of one sequence.  ``ids`` mirrors
    the block ids so packing reads them without walking the block objects."""
    blocks: list[PhysicalBlock] = field(default_factory=list)
    ids: list[int] = field(default_factory=list)

    def append(self, block: PhysicalBlock) -> None:
        self.blocks.append(block)
        self.ids.append(block.block_id)

    @property
    def physical_block_ids(self) -> list[int]:
        return list(self.ids)

    def __len__(self) -> int:
        return len(self.blocks)


class BlockManager:
    def __init__(self, block_size: int, num_gpu_blocks: int, num_cpu_blocks: int = 0,
                 reserved_blocks: int = 0) -> None:
        self.block_size = block_size
        self.gpu_allocator = BlockAllocator(num_gpu_blocks, "gpu", reserved_blocks)
        self.cpu_allocator = BlockAllocator(num_cpu_blocks, "cpu") if num_cpu_blocks > 0 else None
        self.block_tables: dict[int, BlockTable] = {}
        # Called with the number of blocks still missing; returns how many it
        # released.  Installed by the prefix cache when it is enabled.
        self.evictor: Optional[Callable[[int], int]] = None
        # tables created by fork() (they share blocks with their source)
        self.num_forks = 0

    @property
    def num_free_gpu_blocks(self) -> int:
        return self.gpu_allocator.num_free_blocks

    def _ensure_free(self, n: int) -> None:
        short = n - self.gpu_allocator.num_free_blocks
        if short > 0 and self.evictor is not None:
            self.evictor(short)

    def can_allocate(self, num_required_blocks: int) -> bool:
        self._ensure_free(num_required_blocks)
        return self.gpu_allocator.num_free_blocks >= num_required_blocks

    def allocate(self, seq_id: int, num_blocks: int,
                 prefix: Optional[list[PhysicalBlock]] = None) -> BlockTable:
        """New table for seq_id: the shared `prefix` blocks (ref-counted),
        then `num_blocks` fresh ones."""
        table = BlockTable()
        for block in prefix or ():
            self.gpu_allocator.ref(block)
            table.append(block)
        self._ensure_free(num_blocks)
        for _ in range(num_blocks):
            table.append(self.gpu_allocator.allocate())
        self.block_tables[seq_id] = table
        return table

    def append_slot(self, seq_id: int) -> Optional[PhysicalBlock]:
        self._ensure_free(1)
        block = self.gpu_allocator.allocate()
        self.block_tables[seq_id].append(block)
        return block

    def free(self, seq_id: int) -> None:
        table = self.block_tables.pop(seq_id, None)
        if table is None:
            return
        for block in table.blocks:
            self.gpu_allocator.free(block)

    def get_block_table(self, seq_id: int) -> BlockTable:
        return self.block_tables[seq_id]

    def fork(self, src_seq_id: int, dst_seq_id: int) -> BlockTable:
        """Copy-on-write: the destination shares every source block."""
        dst = BlockTable()
        for block in self.block_tables[src_seq_id].blocks:
            self.gpu_allocator.ref(block)
            dst.append(block)
        self.block_tables[dst_seq_id] = dst
        self.num_forks += 1
        return dst
