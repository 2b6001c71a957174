"""End-to-end engine on the GPU: the reference-API layers on the HIP kernels,
config 1 (tiny Llama, fp32) against the CPU oracle model, a Qwen3-shaped
bf16 run with chunked prefill and prefix caching."""

from __future__ import annotations

import asyncio
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from litevllm import LLM, AsyncLLM, SamplingParams
from litevllm.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
from litevllm.layers.attention import Attention, PagedAttention
from litevllm.layers.sampler import Sampler
from oracle.attention import decode_attention
from oracle.model import OracleDecoder

pytestmark = pytest.mark.gpu

TINY_LLAMA = dict(model_type="llama", vocab_size=32000, hidden_size=256, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                  intermediate_size=688, rope_theta=10000.0, rms_norm_eps=1e-6,
                  max_position_embeddings=4096)


def _say(msg):
    print(f"[case] {msg}", flush=True)


def test_reference_sampler_kats_on_gpu(device):
    _say("sampler KATs")
    logits = torch.tensor([[1.0, 5.0, 3.0, 0.5], [4.0, 0.0, 2.0, 1.0]], device=device)
    assert Sampler.sample(logits, SamplingParams(temperature=0.0, max_tokens=8)).tolist() == [1, 0]
    torch.manual_seed(0)
    out = Sampler.sample(torch.randn(4, 32, device=device), SamplingParams(temperature=1.0))
    assert out.shape == (4,) and bool(((out >= 0) & (out < 32)).all())
    planted = torch.zeros(1, 8, device=device)
    planted[0, 3] = 100.0
    assert Sampler.sample(planted, SamplingParams(temperature=1.0, top_k=1)).tolist() == [3]
    assert Sampler.sample(planted, SamplingParams(temperature=1.0)).tolist() == [3]
    tp = torch.tensor([[10.0, 9.5, -100.0, -100.0]], device=device)
    assert Sampler.sample(tp, SamplingParams(temperature=1.0, top_p=0.9)).tolist()[0] in (0, 1)


def test_attention_reference_signature_paths(device):
    """Attention.forward without metadata: prefill = causal over the
    forward's own tokens (reference _prefill), decode = paged over tables."""
    _say("Attention.forward reference paths")
    g = torch.Generator().manual_seed(0)
    H, Hkv, D, bs, T = 8, 4, 64, 16, 37
    attn = Attention(H, D, Hkv)
    q = torch.randn(T, H, D, generator=g)
    k = torch.randn(T, Hkv, D, generator=g)
    v = torch.randn(T, Hkv, D, generator=g)
    kc = torch.zeros(8, bs, Hkv, D, device=device)
    vc = torch.zeros_like(kc)
    slots = torch.arange(3 * bs, 3 * bs + T, dtype=torch.int64, device=device)
    out = attn(q.to(device), k.to(device), v.to(device), kc, vc, None, slots, None,
               is_prefill=True).cpu()
    ref = F.scaled_dot_product_attention(
        q.permute(1, 0, 2).unsqueeze(0), k.repeat_interleave(2, 1).permute(1, 0, 2).unsqueeze(0),
        v.repeat_interleave(2, 1).permute(1, 0, 2).unsqueeze(0), is_causal=True)[0].permute(1, 0, 2)
    assert (out - ref).abs().max() < 1e-4
    # the scatter wrote the new K/V where slot_mapping said
    assert torch.equal(kc.view(-1, Hkv, D)[slots].cpu(), k)
    # decode over the same cache through the reference signature
    table = torch.tensor([[3, 4, 5]], dtype=torch.int32, device=device)
    ctx = torch.tensor([T], dtype=torch.int32, device=device)
    qd = torch.randn(1, H, D, generator=g)
    got = attn(qd.to(device), None, None, kc, vc, table, None, ctx, is_prefill=False).cpu()
    want = decode_attention(qd, kc.cpu(), vc.cpu(), table.cpu(), ctx.cpu(), attn.scale)
    assert (got - want).abs().max() < 1e-4
    PagedAttention.write_to_cache(k[:2].to(device), v[:2].to(device), kc, vc,
                                  torch.tensor([0, 1], device=device))
    assert torch.equal(kc[0, :2].cpu(), k[:2])


@pytest.mark.parametrize("eager", [True, False])
def test_config1_tiny_llama_matches_cpu_oracle(device, eager):
    """Config 1: 8 prompts (lengths U[16,64], ids U[0,32000)), greedy, 32
    tokens, ignore EOS, bs 16, chunk 512, fp32.  Every token equals the CPU
    oracle's until the oracle's top-2 logit margin falls below 1e-4; with
    and without the decode HIP graphs."""
    _say(f"config1 tiny llama eager={eager}")
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(16, 65, (8,), generator=g).tolist()
    prompts = [torch.randint(0, 32000, (n,), generator=g).tolist() for n in lens]
    llm = LLM("tiny-llama", dtype="float32", load_format="dummy", hf_overrides=TINY_LLAMA,
              skip_tokenizer_init=True, num_gpu_blocks=256, block_size=16, chunk_size=512,
              enforce_eager=eager)
    assert (llm.engine.model_runner.graphs is None) == eager
    outs = llm.generate(prompt_token_ids=prompts,
                        sampling_params=SamplingParams(temperature=0.0, max_tokens=32,
                                                       ignore_eos=True))
    assert len(outs) == 8
    by_prompt = {tuple(o.prompt_token_ids): o.output_token_ids for o in outs}
    state = llm.engine.model_runner.model.state_dict()
    oracle = OracleDecoder(state, llm.engine.config.model_config, use_qk_norm=False)
    compared = 0
    for p in prompts:
        got = by_prompt[tuple(p)]
        assert len(got) == 32
        want, margins = oracle.greedy(p, 32)
        for t, (a, b, m) in enumerate(zip(got, want, margins)):
            if m < 1e-4:
                break
            assert a == b, f"prompt len {len(p)}: token {t} differs ({a} vs {b}, margin {m:.2e})"
            compared += 1
    assert compared >= 8 * 16


QWEN3_SMALL = dict(model_type="qwen3", vocab_size=5000, hidden_size=256, num_hidden_layers=2,
                   num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                   intermediate_size=512, rope_theta=1e6, max_position_embeddings=4096)


def _qwen3_prompts():
    g = torch.Generator().manual_seed(1)
    shared = torch.randint(0, 5000, (96,), generator=g).tolist()
    return [shared + torch.randint(0, 5000, (int(n),), generator=g).tolist()
            for n in torch.randint(5, 120, (12,), generator=g)]


def _compare_with_oracle(llm, prompts, outs, n, min_margin, use_qk_norm):
    by_prompt = {tuple(o.prompt_token_ids): o.output_token_ids for o in outs}
    oracle = OracleDecoder(llm.engine.model_runner.model.state_dict(),
                           llm.engine.config.model_config, use_qk_norm=use_qk_norm)
    compared = 0
    for p in prompts:
        got = by_prompt[tuple(p)]
        assert len(got) == n
        want, margins = oracle.greedy(p, n)
        for t, (a, b, m) in enumerate(zip(got, want, margins)):
            if m < min_margin:
                break
            assert a == b, f"prompt len {len(p)}: token {t} differs ({a} vs {b}, margin {m:.2e})"
            compared += 1
    return compared


@pytest.mark.parametrize("dtype,min_margin,min_compared", [("float32", 1e-4, 60),
                                                           ("bfloat16", 0.08, 6)])
def test_qwen3_chunked_prefix_cached_matches_cpu_oracle(device, dtype, min_margin, min_compared):
    """Qwen3-shaped model (qk-norm, GQA 16/8, D=128): prompts of 101-215
    tokens sharing a 96-token prefix, prefill in chunks of 64 under a
    256-token step budget (so decodes and chunks share steps), prefix caching
    on.  Greedy tokens equal the CPU oracle's (fed the same weights) until
    the oracle's top-2 margin drops below a bound that covers the dtype's
    rounding (fp32: 1e-4; bf16, whose prefill goes through the MFMA chunk
    kernel: 0.08 on logits of scale ~0.3)."""
    _say(f"qwen3 small {dtype} chunked + prefix cache")
    prompts = _qwen3_prompts()
    llm = LLM("tiny-qwen3", dtype=dtype, load_format="dummy", hf_overrides=QWEN3_SMALL,
              skip_tokenizer_init=True, num_gpu_blocks=512, chunk_size=64,
              max_num_batched_tokens=256, enable_prefix_caching=True)
    sp = SamplingParams(temperature=0.0, max_tokens=20, ignore_eos=True)
    outs = llm.generate(prompt_token_ids=prompts, sampling_params=sp)
    assert len(outs) == len(prompts) and all(o.num_output_tokens == 20 for o in outs)
    assert llm.engine.prefix_cache.hit_tokens >= 96
    compared = _compare_with_oracle(llm, prompts, outs, 20, min_margin, use_qk_norm=True)
    assert compared >= min_compared


def test_shared_prefix_attention_in_the_engine(device, monkeypatch):
    """The prefix-cached Qwen3 run above with the shared-prefix attention
    pass forced on (its threshold lowered to one saved block): decode rows
    of prompts sharing the cached 96-token prefix read it once per group,
    in decode-graph replays and in mixed steps alike, and the greedy tokens
    still equal the CPU oracle's to the same margin."""
    _say("qwen3 small bf16 shared-prefix attention in the engine")
    from litevllm.engine import model_runner as mr
    monkeypatch.setattr(mr, "PREFIX_MIN_SAVED_BLOCKS", 1)
    used = {"graph": 0, "eager": 0}
    orig_find = mr.find_shared_prefixes
    graph_prepare = mr.DecodeGraphs.prepare

    def spy(*a, **k):
        groups = orig_find(*a, **k)
        if groups:
            used["graph" if spy.in_graph else "eager"] += 1
        return groups
    spy.in_graph = False

    def prepare(self, *a, **k):
        spy.in_graph = True
        try:
            return graph_prepare(self, *a, **k)
        finally:
            spy.in_graph = False
    monkeypatch.setattr(mr, "find_shared_prefixes", spy)
    monkeypatch.setattr(mr.DecodeGraphs, "prepare", prepare)
    prompts = _qwen3_prompts()
    llm = LLM("tiny-qwen3", dtype="bfloat16", load_format="dummy", hf_overrides=QWEN3_SMALL,
              skip_tokenizer_init=True, num_gpu_blocks=512, chunk_size=64,
              max_num_batched_tokens=256, enable_prefix_caching=True)
    assert llm.engine.model_runner.graphs.use_prefix
    sp = SamplingParams(temperature=0.0, max_tokens=20, ignore_eos=True)
    outs = llm.generate(prompt_token_ids=prompts, sampling_params=sp)
    assert all(o.num_output_tokens == 20 for o in outs)
    assert used["graph"] > 0 and used["eager"] > 0, used
    assert _compare_with_oracle(llm, prompts, outs, 20, 0.08, use_qk_norm=True) >= 6


def test_decode_graph_replays_with_changing_prefix_plans(device, monkeypatch):
    """Decode-graph replays while the shared-prefix plan changes from step to
    step (sharers finish at different lengths, so groups shrink and the plan
    empties): every replay equals the eager forward of the same static
    buffers, plan included, and the plan was active in some replays and
    empty in later ones."""
    _say("decode graph replays with changing shared-prefix plans")
    from litevllm.engine import model_runner as mr
    monkeypatch.setattr(mr, "PREFIX_MIN_SAVED_BLOCKS", 1)
    llm = LLM("tiny-qwen3", dtype="bfloat16", load_format="dummy", hf_overrides=QWEN3_SMALL,
              skip_tokenizer_init=True, num_gpu_blocks=512, chunk_size=64,
              enable_prefix_caching=True)
    eng = llm.engine
    runner = eng.model_runner
    assert runner.graphs is not None and runner.graphs.use_prefix
    orig = runner.execute_model
    seen = []

    def checked(meta):
        logits = orig(meta)
        if meta.graph_batch is not None:
            b = meta.graph_batch
            replayed = runner.graphs.logits[b].clone()
            with torch.inference_mode():
                eager = runner.graphs._forward(b)
            torch.cuda.synchronize()
            assert torch.equal(replayed, eager), f"replay {len(seen)}: batch {meta.num_decodes}"
            seen.append(runner.graphs._pfx_active)
        return logits

    runner.execute_model = checked
    g = torch.Generator().manual_seed(8)
    shared = torch.randint(0, 5000, (96,), generator=g).tolist()
    prompts = [shared + torch.randint(0, 5000, (5 + 7 * i,), generator=g).tolist()
               for i in range(6)]
    prompts += [torch.randint(0, 5000, (50,), generator=g).tolist() for _ in range(2)]
    # the first prompt runs alone so its blocks are cached before the others
    llm.generate(prompt_token_ids=prompts[:1],
                 sampling_params=SamplingParams(temperature=0.0, max_tokens=2, ignore_eos=True))
    for i, p in enumerate(prompts):
        eng.add_request(None, SamplingParams(temperature=0.0, max_tokens=4 + 3 * i,
                                             ignore_eos=True), prompt_token_ids=p)
    outs = eng.run_to_completion()
    assert sorted(o.num_output_tokens for o in outs) == [4 + 3 * i for i in range(len(prompts))]
    assert eng.prefix_cache.hit_tokens >= 96
    assert True in seen and False in seen[seen.index(True):], seen


def test_sampling_with_temperature_is_seeded(device):
    _say("seeded temperature sampling")
    cfg = dict(TINY_LLAMA, vocab_size=1000)
    runs = []
    for _ in range(2):
        llm = LLM("tiny", dtype="float32", load_format="dummy", hf_overrides=cfg,
                  skip_tokenizer_init=True, num_gpu_blocks=64, seed=3)
        outs = llm.generate(prompt_token_ids=[[1, 2, 3, 4, 5], [9, 8, 7]],
                            sampling_params=SamplingParams(temperature=0.8, max_tokens=10,
                                                           ignore_eos=True))
        runs.append(sorted(o.output_token_ids for o in outs))
    assert runs[0] == runs[1]


def test_async_llm_streams_and_finishes(device):
    _say("AsyncLLM")
    cfg = EngineConfig(model_config=ModelConfig("tiny", dtype="float32", load_format="dummy",
                                                hf_overrides=dict(TINY_LLAMA, vocab_size=1000)),
                       cache_config=CacheConfig(num_gpu_blocks=64), skip_tokenizer_init=True)

    async def run():
        eng = AsyncLLM(cfg)
        await eng.initialize()
        chunks = [c async for c in eng.stream(None, SamplingParams(max_tokens=5, ignore_eos=True),
                                              prompt_token_ids=[1, 2, 3])]
        return eng, chunks

    eng, chunks = asyncio.run(run())
    assert chunks == [] and not eng.has_unfinished   # no tokenizer: no text deltas


def test_decode_graph_replays_match_eager_forward(device):
    """Every replay of a captured decode graph equals the eager forward of
    the same padded batch, with the engine's own eager work (prefill chunks,
    sampling, host syncs) between the replays."""
    _say("decode graph replays vs eager")
    llm = LLM("tiny-qwen3", dtype="bfloat16", load_format="dummy", hf_overrides=QWEN3_SMALL,
              skip_tokenizer_init=True, num_gpu_blocks=256, chunk_size=64)
    eng = llm.engine
    runner = eng.model_runner
    assert runner.graphs is not None and eng.block_manager.gpu_allocator.reserved_blocks == 1
    orig = runner.execute_model
    seen = []

    def checked(meta):
        logits = orig(meta)
        if meta.graph_batch is not None:
            b = meta.graph_batch
            replayed = runner.graphs.logits[b].clone()
            with torch.inference_mode():
                eager = runner.graphs._forward(b)
            torch.cuda.synchronize()
            assert torch.equal(replayed, eager), f"replay {len(seen)}: batch {meta.num_decodes} -> {b}"
            seen.append((meta.num_decodes, b))
        return logits

    runner.execute_model = checked
    g = torch.Generator().manual_seed(5)
    prompts = [torch.randint(0, 5000, (40 + 13 * i,), generator=g).tolist() for i in range(5)]
    outs = llm.generate(prompt_token_ids=prompts,
                        sampling_params=SamplingParams(temperature=0.0, max_tokens=12,
                                                       ignore_eos=True))
    assert all(o.num_output_tokens == 12 for o in outs)
    assert len(seen) >= 5 and any(B < b for B, b in seen)   # padded replays included


def _reference_fixture():
    import sys
    from pathlib import Path
    golden = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(golden))
    import model_weights as mw
    return mw, np.load(golden / "reference_model_streams.npz")


@pytest.mark.parametrize("name", ["config1", "qwen3_tiny", "llama_tiny"])
def test_engine_reproduces_reference_engine_streams(device, name):
    """The reference's own LLMEngine (run on the CPU in fp32 by
    tests/golden/make_model_fixtures.py) produced these greedy streams for
    weights rebuilt here from tests/golden/model_weights.py; this engine on
    the HIP path, in fp32 with decode graphs on, produces the same tokens
    until the reference's own top-2 margin falls below 1e-4."""
    _say(f"engine vs reference engine streams: {name}")
    mw, fix = _reference_fixture()
    cfg = {"config1": mw.CONFIG1_LLAMA, "qwen3_tiny": mw.QWEN3_TINY,
           "llama_tiny": mw.LLAMA_TINY}[name]
    seed = 0 if name == "config1" else 1
    flat, lens = fix[f"{name}/prompt_ids"], fix[f"{name}/prompt_lens"]
    offs = np.concatenate([[0], np.cumsum(lens)])
    prompts = [flat[offs[i]:offs[i + 1]].tolist() for i in range(len(lens))]
    tokens = fix[f"{name}/tokens"]
    if name == "config1":
        margins = fix["config1/margins"]
    else:
        top2 = torch.topk(torch.from_numpy(fix[f"{name}/logits"]), 2, dim=-1).values
        margins = (top2[..., 0] - top2[..., 1]).numpy()
    llm = LLM(name, dtype="float32", load_format="dummy", hf_overrides=cfg,
              skip_tokenizer_init=True, num_gpu_blocks=256, block_size=16, chunk_size=512)
    assert llm.engine.model_runner.graphs is not None
    llm.engine.model_runner.model.load_weights(
        {k: v.to(device) for k, v in mw.make_weights(cfg, seed).items()})
    n = tokens.shape[1]
    outs = llm.generate(prompt_token_ids=prompts,
                        sampling_params=SamplingParams(temperature=0.0, max_tokens=n,
                                                       ignore_eos=True))
    by_prompt = {tuple(o.prompt_token_ids): o.output_token_ids for o in outs}
    compared = 0
    for i, p in enumerate(prompts):
        got = by_prompt[tuple(p)]
        for t in range(n):
            if margins[i, t] < 1e-4:
                break
            assert got[t] == tokens[i, t], f"{name} prompt {i} token {t}: {got[t]} vs {tokens[i, t]}"
            compared += 1
    assert compared >= tokens.size // 2
