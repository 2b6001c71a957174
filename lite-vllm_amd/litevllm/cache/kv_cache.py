"""Physical KV tensors: per layer K and V of shape
(num_blocks, block_size, num_kv_heads, head_dim), the reference layout
(cache/kv_cache.py:41-50) that the HIP kernels read and write in place.
All layers live in one allocation [num_layers, 2, num_blocks, ...]."""

from __future__ import annotations

import torch


class KVCache:
    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.float16, device: str = "cuda") -> None:
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.storage = torch.zeros((num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim),
                                   dtype=dtype, device=device)
        self.key_caches = [self.storage[i, 0] for i in range(num_layers)]
        self.value_caches = [self.storage[i, 1] for i in range(num_layers)]

    def get_kv(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.key_caches[layer_idx], self.value_caches[layer_idx]

    @property
    def total_bytes(self) -> int:
        return self.storage.numel() * self.storage.element_size()

    @classmethod
    def profile_num_blocks(cls, available_memory_bytes: int, num_layers: int, block_size: int,
                           num_kv_heads: int, head_dim: int,
                           dtype: torch.dtype = torch.float16) -> int:
        elem = torch.tensor([], dtype=dtype).element_size()
        per_block = 2 * block_size * num_kv_heads * head_dim * elem * num_layers
        return max(1, int(available_memory_bytes // per_block))
