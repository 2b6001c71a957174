"""litevllm (MI355X build): lite-vllm's continuous-batching hot path on
hand-written gfx950 HIP kernels behind a C ABI (include/litevllm_hip.h).

Public API as the reference (litevllm/__init__.py): LLM, SamplingParams,
AsyncLLM.  The per-step tensor work (packing, KV scatter, paged attention,
sampling) runs in liblitevllm_hip.so, loaded on first use.
"""

from litevllm.config import SamplingParams
from litevllm.entrypoints.async_llm import AsyncLLM
from litevllm.entrypoints.llm import LLM

__version__ = "0.1.0+mi355x"

__all__ = ["LLM", "SamplingParams", "AsyncLLM"]
