"""Rotary position embedding (NeoX half-split) with the reference's
interface (layers/rotary_emb.py:12-117): a cos/sin cache over
max_position_embeddings, linear / dynamic / YaRN frequency scaling."""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_position_embeddings: int = 4096, base: float = 10000.0,
                 rope_scaling: Optional[dict] = None, device: Optional[str] = None) -> None:
        super().__init__()
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        self.rope_scaling = rope_scaling
        inv_freq = self._inv_freq()
        t = torch.arange(max_position_embeddings, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        self.register_buffer("cos_cached", freqs.cos().to(device or "cpu"), persistent=False)
        self.register_buffer("sin_cached", freqs.sin().to(device or "cpu"), persistent=False)

    def _inv_freq(self) -> torch.Tensor:
        d = self.head_dim
        exps = torch.arange(0, d, 2, dtype=torch.float32) / d
        inv = 1.0 / (self.base ** exps)
        if self.rope_scaling:
            kind = self.rope_scaling.get("type", "linear")
            factor = float(self.rope_scaling.get("factor", 1.0))
            if kind == "linear":
                inv = inv / factor
            elif kind == "dynamic":
                # The reference's dynamic rule (rotary_emb.py:41-47) evaluates
                # its stretched base at the trained length itself, where the
                # stretch factor is 1: the frequencies stay unscaled.
                pass
            elif kind == "yarn":
                inv = self._yarn(inv, factor)
        return inv

    def _yarn(self, inv: torch.Tensor, factor: float) -> torch.Tensor:
        d = self.head_dim
        low = max(math.floor(d * math.log(1 / (32.0 * 2 * math.pi)) / (2 * math.log(self.base))), 0)
        high = min(math.ceil(d * math.log(1 / (1.0 * 2 * math.pi)) / (2 * math.log(self.base))),
                   d // 2 - 1)
        ramp = ((torch.arange(d // 2, dtype=torch.float32) - low) / max(high - low, 1)).clamp(0, 1)
        return (1 - ramp) * (inv / factor) + ramp * inv

    def forward(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return self.cos_cached[positions], self.sin_cached[positions]


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
