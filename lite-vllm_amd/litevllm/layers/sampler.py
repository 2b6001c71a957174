"""Sampler with the reference's interface (layers/sampler.py:147-225).

Greedy and plain temperature sampling run in one fused HIP kernel
(lv_sample): greedy = first index of the fp32 max; temperature = inverse-CDF
draw of softmax(x/T) at a uniform u (drawn with torch.rand when the caller
does not supply one, which matches torch.multinomial in distribution).
Top-k / top-p and the repetition penalty keep the reference's torch
implementation (sampler.py:190-225) on the GPU tensors; they are not part of
the accelerated path.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import ops
from ..config import SamplingParams


class Sampler:
    @staticmethod
    def sample(logits: torch.Tensor, sampling_params: SamplingParams,
               past_token_ids: Optional[torch.Tensor] = None,
               uniform: Optional[torch.Tensor] = None,
               generator: Optional[torch.Generator] = None) -> torch.Tensor:
        if logits.dim() == 1:
            logits = logits.unsqueeze(0)
        if past_token_ids is not None and sampling_params.repetition_penalty != 1.0:
            logits = _apply_repetition_penalty(logits.clone(), past_token_ids,
                                               sampling_params.repetition_penalty)
        B = logits.shape[0]
        dev = logits.device
        T = float(sampling_params.temperature)
        if T == 0.0:
            return ops.sample(logits, torch.zeros(B, dtype=torch.float32, device=dev))
        if sampling_params.top_k > 0 or sampling_params.top_p < 1.0:
            probs = F.softmax(logits.float() / T, dim=-1)
            probs = _apply_top_k_top_p(probs, sampling_params.top_k, sampling_params.top_p)
            return torch.multinomial(probs, num_samples=1, generator=generator).squeeze(-1)
        if uniform is None:
            uniform = torch.rand(B, dtype=torch.float32, device=dev, generator=generator)
        return ops.sample(logits, torch.full((B,), T, dtype=torch.float32, device=dev), uniform)

    @staticmethod
    def sample_batched(logits: torch.Tensor, temperatures: torch.Tensor,
                       uniforms: torch.Tensor) -> torch.Tensor:
        """Row r greedy if temperatures[r] == 0, else sampled at uniforms[r]."""
        return ops.sample(logits, temperatures, uniforms)


def _apply_repetition_penalty(logits: torch.Tensor, past_token_ids: torch.Tensor,
                              penalty: float) -> torch.Tensor:
    for i in range(logits.shape[0]):
        ids = past_token_ids[i].unique()
        score = logits[i, ids]
        logits[i, ids] = torch.where(score > 0, score / penalty, score * penalty)
    return logits


def _apply_top_k_top_p(probs: torch.Tensor, top_k: int, top_p: float) -> torch.Tensor:
    if top_k > 0:
        k = min(top_k, probs.size(-1))
        threshold = torch.topk(probs, k, dim=-1).values[..., -1, None]
        probs = torch.where(probs < threshold, torch.zeros_like(probs), probs)
    if top_p < 1.0:
        sorted_probs, sorted_idx = torch.sort(probs, descending=True, dim=-1)
        cum = torch.cumsum(sorted_probs, dim=-1)
        sorted_probs = torch.where(cum - sorted_probs > top_p, torch.zeros_like(sorted_probs),
                                   sorted_probs)
        probs = torch.zeros_like(probs).scatter_(-1, sorted_idx, sorted_probs)
    return probs / probs.sum(dim=-1, keepdim=True).clamp_min(1e-9)
