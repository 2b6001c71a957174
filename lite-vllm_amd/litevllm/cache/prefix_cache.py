"""Prefix cache: reuse the KV blocks of identical prompt prefixes.

Interface of the reference's PrefixCache (cache/prefix_cache.py:18-75:
lookup / insert / evict over full blocks), wired into scheduling here (the
reference instantiates it but never consults it, llm_engine.py:71-72).  One
deliberate difference: a block's key chains the key of the block before it,
so a block is only reused after the same *prefix*; the reference hashes each
block's 16 tokens alone, which would hand out KV computed under a different
prefix whenever a block's tokens repeat.  Cached blocks hold one reference of
their own and are released (oldest first) when the allocator runs dry.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Optional

from .block_manager import BlockManager, BlockTable, PhysicalBlock


def _chain_hash(parent: Optional[int], tokens: tuple[int, ...]) -> int:
    return hash((parent, tokens))


class PrefixCache:
    def __init__(self, block_size: int, block_manager: Optional[BlockManager] = None) -> None:
        self.block_size = block_size
        self.cache: "OrderedDict[int, PhysicalBlock]" = OrderedDict()
        self.block_manager = block_manager
        self.hit_tokens = 0               # prompt tokens served from the cache
        if block_manager is not None:
            block_manager.evictor = self.evict_unused

    def _keys(self, token_ids: list[int], n_blocks: int):
        parent = None
        bs = self.block_size
        for i in range(n_blocks):
            parent = _chain_hash(parent, tuple(token_ids[i * bs:(i + 1) * bs]))
            yield parent

    def lookup(self, token_ids: list[int],
               block_manager: Optional[BlockManager] = None) -> tuple[list[PhysicalBlock], int]:
        """Longest cached run of full leading blocks: (blocks, num_cached_tokens)."""
        matched: list[PhysicalBlock] = []
        for h in self._keys(token_ids, len(token_ids) // self.block_size):
            block = self.cache.get(h)
            if block is None:
                break
            self.cache.move_to_end(h)
            matched.append(block)
        return matched, len(matched) * self.block_size

    def insert(self, token_ids: list[int], block_table: BlockTable) -> None:
        """Register the full blocks of token_ids (their KV must be computed)."""
        n = min(len(token_ids) // self.block_size, len(block_table))
        for i, h in enumerate(self._keys(token_ids, n)):
            if h in self.cache:
                continue
            block = block_table.blocks[i]
            if block.is_cached:
                continue
            block.is_cached = True
            block.hash_value = h
            block.ref_count += 1          # the cache's own reference
            self.cache[h] = block

    def evict(self, block: PhysicalBlock) -> None:
        if block.hash_value is not None and self.cache.get(block.hash_value) is block:
            del self.cache[block.hash_value]
            block.is_cached = False
            block.hash_value = None

    def evict_unused(self, needed: int) -> int:
        """Release up to `needed` cached blocks no sequence uses (oldest first)."""
        if self.block_manager is None:
            return 0
        released = 0
        for h in list(self.cache.keys()):
            if released >= needed:
                break
            block = self.cache[h]
            if block.ref_count == 1:
                del self.cache[h]
                block.is_cached = False
                block.hash_value = None
                self.block_manager.gpu_allocator.free(block)
                released += 1
        return released
