#!/usr/bin/env python3
"""Write tests/golden/reference_model_streams.npz from the reference itself.

BUILD CONTAINER ONLY: imports the reference package from /root/reference
(lite-vllm 0.1.0, pure Python/torch), which does not exist on the GPU host.
The committed .npz is data (token ids, logits, margins); nothing here is
needed at test time.

For each case the script writes a local model directory (config.json +
model.safetensors holding ``model_weights.make_weights(cfg, seed)``), builds
the reference's LLMEngine on the CPU in fp32 (engine/llm_engine.py:29-86:
ModelRunner.load_model reading the safetensors, KVCache, BlockManager,
Scheduler), enqueues the prompts as token ids (SequenceGroup.create +
Scheduler.add_request, bypassing tokenization as the reference's own
engine does after encode, llm_engine.py:88-106), and runs
run_to_completion with greedy SamplingParams.  The tokenizer is replaced by
a stub whose EOS id matches no token (the reference has no ignore_eos; its
EOS would otherwise fall back to id 0, tokenizer.py:48-51) and whose decode
returns "" -- text plays no part in the streams.

Captured per sequence and per step: the logits row the reference's
LLMEngine._process_outputs hands to Sampler.sample (llm_engine.py:172-197;
the last prompt token's row after the prefill forward, then one row per
decode forward through the paged cache, attention.py:91-139), and the token
it drew.  Small models keep the whole logits rows; config 1 (vocab 32000)
keeps the tokens and each step's top-1 minus top-2 margin.

Usage: python tests/golden/make_model_fixtures.py
"""

from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")
OUT = HERE / "reference_model_streams.npz"

sys.path.insert(0, str(HERE))
import model_weights as mw  # noqa: E402


def _import_reference():
    if not (REFERENCE / "litevllm").is_dir():
        raise SystemExit(f"{REFERENCE} not found: this script runs in the build container only")
    sys.path.insert(0, str(REFERENCE))
    import litevllm  # noqa: F401
    if not Path(litevllm.__file__).resolve().is_relative_to(REFERENCE.resolve()):
        raise SystemExit(f"imported {litevllm.__file__}, not the reference")
    from litevllm.config import CacheConfig, EngineConfig, ModelConfig, SamplingParams
    from litevllm.engine import llm_engine
    from litevllm.engine.sequence import SequenceGroup
    return CacheConfig, EngineConfig, ModelConfig, SamplingParams, llm_engine, SequenceGroup


class _NoTextTokenizer:
    eos_token_id = -1

    def decode(self, token_ids, skip_special_tokens=True):
        return ""


def run_reference(cfg: dict, seed: int, prompts: list[list[int]], max_tokens: int):
    """Greedy streams and the per-step logits rows of the reference engine."""
    from safetensors.torch import save_file
    CacheConfig, EngineConfig, ModelConfig, SamplingParams, llm_engine, SequenceGroup = \
        _import_reference()
    weights = mw.make_weights(cfg, seed)
    with tempfile.TemporaryDirectory() as d:
        (Path(d) / "config.json").write_text(json.dumps(dict(cfg, torch_dtype="float32")))
        save_file({k: v.contiguous() for k, v in weights.items()}, str(Path(d) / "model.safetensors"))
        llm_engine.get_tokenizer = lambda *a, **k: _NoTextTokenizer()
        eng = llm_engine.LLMEngine(EngineConfig(ModelConfig(d, dtype="float32"),
                                                CacheConfig(block_size=16, num_gpu_blocks=256),
                                                device="cpu", seed=0))
        eng.initialize()
        rows: dict[int, list[torch.Tensor]] = {}
        order: list[int] = []
        orig_process = eng._process_outputs
        orig_sample = eng.sampler.sample

        def process(logits, seq_groups):
            order.extend(s.seq_id for sg in seq_groups for s in sg.get_unfinished_seqs())
            return orig_process(logits, seq_groups)

        def sample(logits, params, *a, **k):
            rows.setdefault(order.pop(0), []).append(logits.reshape(-1).detach().clone())
            return orig_sample(logits, params, *a, **k)

        eng._process_outputs = process
        eng.sampler.sample = sample
        groups = []
        for i, p in enumerate(prompts):
            sg = SequenceGroup.create(f"req{i}", p, SamplingParams(temperature=0.0,
                                                                   max_tokens=max_tokens))
            eng.scheduler.add_request(sg)
            groups.append(sg)
        eng.run_to_completion()
    streams = [list(sg.seqs[0].data.output_token_ids) for sg in groups]
    logits = [torch.stack(rows[sg.seqs[0].seq_id]) for sg in groups]
    for s, lg in zip(streams, logits):
        assert len(s) == max_tokens and lg.shape[0] == max_tokens
        assert s == lg.argmax(-1).tolist()
    return streams, logits


def _flat(prompts):
    lens = np.array([len(p) for p in prompts], dtype=np.int64)
    return np.concatenate([np.asarray(p, dtype=np.int64) for p in prompts]), lens


def main() -> None:
    out = {}
    g = torch.Generator().manual_seed(7)
    tiny_prompts = [torch.randint(0, 512, (n,), generator=g).tolist() for n in (5, 23, 40)]
    for name, cfg in (("qwen3_tiny", mw.QWEN3_TINY), ("llama_tiny", mw.LLAMA_TINY)):
        streams, logits = run_reference(cfg, seed=1, prompts=tiny_prompts, max_tokens=12)
        flat, lens = _flat(tiny_prompts)
        out[f"{name}/prompt_ids"] = flat
        out[f"{name}/prompt_lens"] = lens
        out[f"{name}/tokens"] = np.asarray(streams, dtype=np.int64)
        out[f"{name}/logits"] = torch.stack(logits).numpy().astype(np.float32)
        print(f"{name}: streams {streams}", flush=True)
    prompts = mw.config1_prompts()
    streams, logits = run_reference(mw.CONFIG1_LLAMA, seed=0, prompts=prompts, max_tokens=32)
    flat, lens = _flat(prompts)
    top2 = torch.stack([torch.topk(lg, 2, dim=-1).values for lg in logits])
    out["config1/prompt_ids"] = flat
    out["config1/prompt_lens"] = lens
    out["config1/tokens"] = np.asarray(streams, dtype=np.int64)
    out["config1/margins"] = (top2[..., 0] - top2[..., 1]).numpy().astype(np.float32)
    print(f"config1: first tokens {[s[:4] for s in streams]}", flush=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
