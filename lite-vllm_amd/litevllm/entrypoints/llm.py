"""LLM — offline synchronous generation (reference entrypoints/llm.py:28-123).

Same constructor knobs and generate() contract (outputs in completion
order, greedy max_tokens=256 by default); additions: prompt_token_ids for
tokenizer-free use, load_format="dummy" / hf_overrides for seeded random
weights of a given architecture, skip_tokenizer_init.
"""

from __future__ import annotations

import argparse
from typing import Optional, Union

from litevllm.config import CacheConfig, EngineConfig, ModelConfig, SamplingParams, SchedulerConfig
from litevllm.engine.llm_engine import LLMEngine
from litevllm.engine.sequence import SequenceGroupOutput


class LLM:
    def __init__(self, model: str, dtype: str = "auto", max_model_len: Optional[int] = None,
                 gpu_memory_utilization: float = 0.85, block_size: int = 16,
                 max_num_seqs: int = 256, max_num_batched_tokens: int = 8192,
                 enable_prefix_caching: bool = False, chunked_prefill: bool = True,
                 chunk_size: int = 512, trust_remote_code: bool = True, seed: int = 0,
                 load_format: str = "auto", hf_overrides: Optional[dict] = None,
                 skip_tokenizer_init: bool = False, num_gpu_blocks: Optional[int] = None,
                 device: str = "auto", enforce_eager: bool = False) -> None:
        cfg = EngineConfig(
            model_config=ModelConfig(model=model, dtype=dtype, max_model_len=max_model_len,
                                     trust_remote_code=trust_remote_code,
                                     load_format=load_format, hf_overrides=hf_overrides),
            cache_config=CacheConfig(block_size=block_size, num_gpu_blocks=num_gpu_blocks,
                                     gpu_memory_utilization=gpu_memory_utilization,
                                     enable_prefix_caching=enable_prefix_caching),
            scheduler_config=SchedulerConfig(max_num_seqs=max_num_seqs,
                                             max_num_batched_tokens=max_num_batched_tokens,
                                             chunked_prefill=chunked_prefill,
                                             chunk_size=chunk_size),
            device=device, seed=seed, skip_tokenizer_init=skip_tokenizer_init,
            enforce_eager=enforce_eager)
        self.engine = LLMEngine(cfg)
        self.engine.initialize()

    def generate(self, prompts: Union[str, list[str], None] = None,
                 sampling_params: Optional[SamplingParams] = None,
                 prompt_token_ids: Optional[list[list[int]]] = None) -> list[SequenceGroupOutput]:
        if sampling_params is None:
            sampling_params = SamplingParams(temperature=0.0, max_tokens=256)
        if prompt_token_ids is not None:
            for ids in prompt_token_ids:
                self.engine.add_request(None, sampling_params, prompt_token_ids=list(ids))
        else:
            if isinstance(prompts, str):
                prompts = [prompts]
            for p in prompts or []:
                self.engine.add_request(p, sampling_params)
        return self.engine.run_to_completion()

    def __repr__(self) -> str:
        return f"LLM(model={self.engine.config.model_config.model!r})"


def main() -> None:
    """python -m litevllm --model DIR --prompt ... (reference llm.py:99-123)."""
    parser = argparse.ArgumentParser(description="litevllm offline inference")
    parser.add_argument("--model", type=str, required=True)
    parser.add_argument("--prompt", type=str, default="Hello!")
    parser.add_argument("--max-tokens", type=int, default=128)
    parser.add_argument("--temperature", type=float, default=0.0)
    parser.add_argument("--top-p", type=float, default=1.0)
    parser.add_argument("--top-k", type=int, default=-1)
    parser.add_argument("--dtype", type=str, default="auto")
    parser.add_argument("--seed", type=int, default=0)
    args = parser.parse_args()
    params = SamplingParams(temperature=args.temperature, top_p=args.top_p, top_k=args.top_k,
                            max_tokens=args.max_tokens)
    llm = LLM(model=args.model, dtype=args.dtype, seed=args.seed)
    for out in llm.generate([args.prompt], params):
        print(f"\nPrompt: {out.prompt_text}\nOutput: {out.output_text}\n"
              f"Tokens: {out.num_prompt_tokens} prompt + {out.num_output_tokens} generated")
