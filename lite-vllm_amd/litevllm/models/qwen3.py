"""Qwen3 (reference models/qwen3.py:24-230): the Llama stack with per-head
q/k RMSNorm before RoPE, explicit head_dim, no attention bias by default."""

from __future__ import annotations

from litevllm.config import ModelConfig
from litevllm.models.llama import LlamaForCausalLM


class Qwen3ForCausalLM(LlamaForCausalLM):
    @staticmethod
    def _qk_norm(config: ModelConfig) -> bool:
        return config.use_qk_norm
