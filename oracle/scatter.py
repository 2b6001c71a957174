"""CPU restatement of the KV scatter (test oracle).

Restates the inline scatter of Attention.forward (reference
litevllm/layers/attention.py:79-84) and PagedAttention.write_to_cache
(attention.py:17-33): key_cache[slot // bs, slot % bs] = key[t].
Negative slots are skipped (the build's padding convention).
"""

from __future__ import annotations

import numpy as np


def kv_scatter(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray,
               value_cache: np.ndarray, slot_mapping: np.ndarray) -> None:
    bs = key_cache.shape[1]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = slots >= 0
    b_idx = slots[keep] // bs
    b_off = slots[keep] % bs
    key_cache[b_idx, b_off] = key[keep]
    value_cache[b_idx, b_off] = value[keep]
