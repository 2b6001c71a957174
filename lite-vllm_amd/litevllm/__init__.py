"""litevllm (MI355X build): lite-vllm's continuous-batching hot path on
hand-written gfx950 HIP kernels behind a C ABI (include/litevllm_hip.h).

The public engine API (LLM, AsyncLLM, SamplingParams) mirrors lite-vllm
0.1.0 (reference litevllm/__init__.py); the per-step tensor work (packing,
KV scatter, paged attention, sampling) runs in liblitevllm_hip.so.
"""

__version__ = "0.1.0+mi355x"
