"""Engine configuration dataclasses.

Field names and defaults follow the reference's config/config.py:15-178
(ModelConfig, CacheConfig, SchedulerConfig, EngineConfig, SamplingParams) so
user code carries over.  Additions: ``SamplingParams.ignore_eos`` (the
reference has none; its EOS falls back to token 0, tokenizer.py:48-51),
``ModelConfig.load_format="dummy"`` (seeded random weights, no checkpoint)
and ``ModelConfig.from_hf_dict`` for architectures given as a plain dict.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

import torch

_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


@dataclass
class ModelConfig:
    model: str
    dtype: str = "auto"
    trust_remote_code: bool = True
    revision: Optional[str] = None
    max_model_len: Optional[int] = None
    load_format: str = "auto"          # "auto" (safetensors/bin) or "dummy" (seeded random)
    hf_overrides: Optional[dict] = None  # architecture fields used instead of a config.json

    vocab_size: int = 0
    hidden_size: int = 0
    num_hidden_layers: int = 0
    num_attention_heads: int = 0
    num_key_value_heads: int = 0
    head_dim: int = 0
    intermediate_size: int = 0
    rope_theta: float = 10000.0
    rope_scaling: Optional[dict] = None
    max_position_embeddings: int = 4096
    model_type: str = ""
    attention_bias: bool = False
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = False
    use_qk_norm: bool = False

    def resolve(self) -> None:
        """Populate the architecture fields from hf_overrides or config.json."""
        if self.hf_overrides is not None:
            cfg: dict[str, Any] = dict(self.hf_overrides)
        else:
            from transformers import AutoConfig
            cfg = AutoConfig.from_pretrained(self.model, trust_remote_code=self.trust_remote_code,
                                             revision=self.revision).to_dict()
        self._apply(cfg)

    def _apply(self, cfg: dict[str, Any]) -> None:
        self.vocab_size = cfg["vocab_size"]
        self.hidden_size = cfg["hidden_size"]
        self.num_hidden_layers = cfg["num_hidden_layers"]
        self.num_attention_heads = cfg["num_attention_heads"]
        self.num_key_value_heads = cfg.get("num_key_value_heads") or self.num_attention_heads
        self.head_dim = cfg.get("head_dim") or self.hidden_size // self.num_attention_heads
        self.intermediate_size = cfg.get("intermediate_size", 0)
        rs = cfg.get("rope_scaling")
        self.rope_theta = cfg.get("rope_theta") or (rs or {}).get("rope_theta") or 10000.0
        if isinstance(rs, dict) and rs.get("type", rs.get("rope_type")) not in (None, "default"):
            self.rope_scaling = {"type": rs.get("type", rs.get("rope_type")),
                                 "factor": float(rs.get("factor") or 1.0)}
        else:
            self.rope_scaling = None
        self.max_position_embeddings = cfg.get("max_position_embeddings", 4096)
        self.model_type = cfg.get("model_type", "")
        self.attention_bias = bool(cfg.get("attention_bias", self.model_type == "qwen2"))
        self.rms_norm_eps = cfg.get("rms_norm_eps", 1e-6)
        self.tie_word_embeddings = bool(cfg.get("tie_word_embeddings", False))
        self.use_qk_norm = bool(cfg.get("use_qk_norm", cfg.get("qk_norm", self.model_type == "qwen3")))
        if self.max_model_len is None:
            self.max_model_len = self.max_position_embeddings

    @property
    def torch_dtype(self) -> torch.dtype:
        """"auto" is bf16 on a ROCm GPU (MI355X computes bf16 natively) and fp32 on CPU."""
        if self.dtype == "auto":
            return torch.bfloat16 if torch.cuda.is_available() else torch.float32
        return _DTYPES.get(self.dtype, torch.float16)


@dataclass
class CacheConfig:
    block_size: int = 16
    num_gpu_blocks: Optional[int] = None
    num_cpu_blocks: int = 0
    gpu_memory_utilization: float = 0.85
    enable_prefix_caching: bool = False
    # decode rows whose block tables start with the same blocks read that
    # shared prefix once per group in attention
    shared_prefix_attention: bool = True


@dataclass
class SchedulerConfig:
    max_num_seqs: int = 256
    max_num_batched_tokens: int = 8192
    chunked_prefill: bool = True
    chunk_size: int = 512


@dataclass
class EngineConfig:
    model_config: ModelConfig
    cache_config: CacheConfig = field(default_factory=CacheConfig)
    scheduler_config: SchedulerConfig = field(default_factory=SchedulerConfig)
    device: str = "auto"
    seed: int = 0
    skip_tokenizer_init: bool = False
    # False: decode-only steps replay HIP graphs captured per padded batch size
    enforce_eager: bool = False
    max_graph_batch: int = 256

    def resolve(self) -> None:
        if self.device == "auto":
            self.device = "cuda" if torch.cuda.is_available() else "cpu"
        self.model_config.resolve()


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = -1
    max_tokens: int = 256
    min_tokens: int = 0
    repetition_penalty: float = 1.0
    stop: list[str] = field(default_factory=list)
    stop_token_ids: list[int] = field(default_factory=list)
    skip_special_tokens: bool = True
    seed: Optional[int] = None
    ignore_eos: bool = False

    def __post_init__(self) -> None:
        # Same validation as the reference (config.py:172-178).
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if not 0.0 < self.top_p <= 1.0:
            raise ValueError("top_p must be in (0, 1]")
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
