"""Model interface and registry (reference models/base.py:18-74)."""

from __future__ import annotations

import abc
from typing import Optional

import torch
import torch.nn as nn

from litevllm.config import ModelConfig


class BaseModelForCausalLM(nn.Module, abc.ABC):
    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.config = config

    @abc.abstractmethod
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor,
                kv_caches: Optional[list[tuple[torch.Tensor, torch.Tensor]]] = None,
                slot_mapping: Optional[torch.Tensor] = None,
                block_tables: Optional[torch.Tensor] = None,
                context_lens: Optional[torch.Tensor] = None, is_prefill: bool = True,
                attn_metadata=None, logits_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Logits for every token, or only for the rows in logits_indices."""

    @abc.abstractmethod
    def load_weights(self, weights: dict[str, torch.Tensor]) -> None:
        ...

    @torch.no_grad()
    def init_dummy_weights(self, seed: int = 0, std: float = 0.02) -> None:
        """Seeded random weights (CPU generator, so every device sees the same
        bits): N(0, std) for projections and embeddings, ones for norms."""
        g = torch.Generator().manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float32) * std)

    @classmethod
    def get_model_cls(cls, model_type: str) -> type["BaseModelForCausalLM"]:
        from .llama import LlamaForCausalLM
        from .qwen3 import Qwen3ForCausalLM
        registry = {"llama": LlamaForCausalLM, "qwen2": Qwen3ForCausalLM,
                    "qwen3": Qwen3ForCausalLM}
        model_cls = registry.get(model_type)
        if model_cls is None:
            raise ValueError(f"Unsupported model type: {model_type}. Supported: {list(registry)}")
        return model_cls
