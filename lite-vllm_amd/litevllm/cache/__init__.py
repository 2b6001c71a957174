from .block_manager import BlockAllocator, BlockManager, BlockTable, PhysicalBlock
from .kv_cache import KVCache
from .prefix_cache import PrefixCache

__all__ = ["BlockAllocator", "BlockManager", "BlockTable", "PhysicalBlock", "KVCache",
           "PrefixCache"]
