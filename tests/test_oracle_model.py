"""Pins of the oracle decoder (CPU): incremental decoding equals a full
prefill, RMSNorm equals torch's rms_norm, attention equals SDPA."""

from __future__ import annotations

import sys
from pathlib import Path

import torch
import torch.nn.functional as F

from litevllm.config import ModelConfig
from litevllm.models.qwen3 import Qwen3ForCausalLM
from oracle.model import OracleDecoder

CFG = dict(model_type="qwen3", vocab_size=300, hidden_size=64, num_hidden_layers=2,
           num_attention_heads=4, num_key_value_heads=2, head_dim=16, intermediate_size=96,
           rope_theta=1e4, max_position_embeddings=256)


def _oracle(use_qk_norm=True):
    mc = ModelConfig("x", load_format="dummy", hf_overrides=CFG)
    mc.resolve()
    m = Qwen3ForCausalLM(mc)
    m.init_dummy_weights(0, std=0.2)
    return OracleDecoder(m.state_dict(), mc, use_qk_norm=use_qk_norm)


def test_incremental_decode_equals_full_prefill():
    o = _oracle()
    ids = [5, 17, 250, 3, 99, 42, 7]
    full = o.forward(ids, 0, [])
    kv: list = []
    o.forward(ids[:4], 0, kv)
    o.forward(ids[4:6], 4, kv)
    inc = o.forward(ids[6:], 6, kv)
    assert torch.allclose(full, inc, atol=1e-5)


def test_rms_matches_torch_and_position_matters():
    o = _oracle()
    x = torch.randn(3, 64)
    w = torch.rand(64)
    assert torch.allclose(o._rms(x, w), F.rms_norm(x, (64,), w, eps=1e-6), atol=1e-6)
    a = o.forward([1, 2, 3], 0, [])
    b = o.forward([1, 2, 3], 5, [])        # shifted positions change the output (RoPE)
    assert not torch.allclose(a, b)


def test_batched_decode_equals_per_sequence_forward():
    o = _oracle()
    prompts = [[5, 17, 250], [3, 99, 42, 7, 8], [11]]
    kvs = []
    for p in prompts:
        kv: list = []
        o.forward(p, 0, kv)
        kvs.append(kv)
    ref = []
    for p in prompts:
        kv: list = []
        o.forward(p, 0, kv)
        ref.append(o.forward([123], len(p), kv))
    got = o.decode_batch([123] * 3, [len(p) for p in prompts], kvs)
    assert torch.allclose(got, torch.stack(ref), atol=1e-5)
    assert all(kv[0][0].shape[0] == len(p) + 1 for kv, p in zip(kvs, prompts))


# ---------------------------------------------------------------------------
# Pins against the reference itself: tests/golden/reference_model_streams.npz
# holds the greedy streams and per-step logits rows of the reference's own
# LLMEngine on the CPU in fp32 (tests/golden/make_model_fixtures.py), for
# weights rebuilt here from tests/golden/model_weights.py.
# ---------------------------------------------------------------------------

import numpy as np  # noqa: E402
import pytest  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import model_weights as mw  # noqa: E402

FIX = np.load(GOLDEN / "reference_model_streams.npz")


def _fixture_prompts(name):
    flat, lens = FIX[f"{name}/prompt_ids"], FIX[f"{name}/prompt_lens"]
    offs = np.concatenate([[0], np.cumsum(lens)])
    return [flat[offs[i]:offs[i + 1]].tolist() for i in range(len(lens))]


def _fixture_oracle(cfg, seed, decoder_cls=OracleDecoder):
    mc = ModelConfig("x", load_format="dummy", hf_overrides=cfg)
    mc.resolve()
    state = mw.fused_state(cfg, mw.make_weights(cfg, seed))
    return decoder_cls(state, mc, use_qk_norm=mc.use_qk_norm)


def _teacher_forced_logits(o, prompt, tokens):
    """Oracle logits at each step when fed the reference's tokens."""
    kv: list = []
    out = [o.forward(prompt, 0, kv)]
    for t, tok in enumerate(tokens[:-1]):
        out.append(o.forward([tok], len(prompt) + t, kv))
    return torch.stack(out)


@pytest.mark.parametrize("name,cfg", [("qwen3_tiny", mw.QWEN3_TINY),
                                      ("llama_tiny", mw.LLAMA_TINY)])
def test_oracle_decoder_matches_reference_engine_logits(name, cfg):
    """Every step's logits row equals the reference engine's (prefill then
    paged decode, fp32) to 1e-5 relative to the logits' scale, and the greedy
    streams are identical."""
    o = _fixture_oracle(cfg, seed=1)
    ref_logits = torch.from_numpy(FIX[f"{name}/logits"])
    ref_tokens = FIX[f"{name}/tokens"]
    for i, p in enumerate(_fixture_prompts(name)):
        got = _teacher_forced_logits(o, p, ref_tokens[i].tolist())
        scale = ref_logits[i].abs().max()
        assert scale > 1.0
        assert (got - ref_logits[i]).abs().max() <= 1e-5 * scale, name
        assert o.greedy(p, len(ref_tokens[i]))[0] == ref_tokens[i].tolist()


@pytest.mark.parametrize("mistake", ["qk_norm_after_rope", "gate_up_swapped",
                                     "final_norm_weight_dropped", "no_norm_weight",
                                     "rope_interleaved"])
def test_reference_fixture_catches_structural_mistakes(mistake):
    """A copy of the oracle with one plausible structural mistake planted
    no longer matches the reference's logits (so the check above pins
    each of these)."""
    import math

    class Planted(OracleDecoder):
        def _rope(self, x, pos):
            if mistake != "rope_interleaved":
                return super()._rope(x, pos)
            c = self.cos[pos].unsqueeze(1)
            s = self.sin[pos].unsqueeze(1)
            x1, x2 = x[..., 0::2], x[..., 1::2]
            return torch.stack([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).flatten(-2)

        def _rms(self, x, w):
            if mistake == "no_norm_weight":
                w = torch.ones_like(w)
            return super()._rms(x, w)

    o = _fixture_oracle(mw.QWEN3_TINY, seed=1, decoder_cls=Planted)
    w = o.w
    if mistake == "gate_up_swapped":
        for k in [k for k in w if k.endswith("gate_up_proj.weight")]:
            g, u = w[k].chunk(2)
            w[k] = torch.cat([u, g])
    if mistake == "final_norm_weight_dropped":
        w["model.norm.weight"] = torch.ones_like(w["model.norm.weight"])
    if mistake == "qk_norm_after_rope":
        base_rope = o._rope
        qn = [w[f"model.layers.{i}.self_attn.q_norm.weight"] for i in range(2)]
        kn = [w[f"model.layers.{i}.self_attn.k_norm.weight"] for i in range(2)]
        # swap the two steps: RoPE on the raw heads, then the per-head norm
        o.use_qk_norm = False
        calls = {"n": 0}

        def rope_then_norm(x, pos):
            layer, which = divmod(calls["n"], 2)
            calls["n"] = (calls["n"] + 1) % 4
            weight = (qn if which == 0 else kn)[layer]
            return o._rms(base_rope(x, pos), weight)
        o._rope = rope_then_norm
    p = _fixture_prompts("qwen3_tiny")[1]
    ref = torch.from_numpy(FIX["qwen3_tiny/logits"][1])
    got = _teacher_forced_logits(o, p, FIX["qwen3_tiny/tokens"][1].tolist())
    assert not math.isclose(0.0, float((got - ref).abs().max()), abs_tol=1e-3), mistake


def test_oracle_decoder_reproduces_reference_config1_streams():
    """Config 1 (tiny Llama, vocab 32000, 8 prompts, 32 greedy tokens): the
    oracle's greedy tokens are the reference engine's until the reference's
    own top-2 margin falls below 1e-4 (fp32 rounding may swap a closer pair)."""
    o = _fixture_oracle(mw.CONFIG1_LLAMA, seed=0)
    prompts = _fixture_prompts("config1")
    assert prompts == mw.config1_prompts()
    tokens, margins = FIX["config1/tokens"], FIX["config1/margins"]
    compared = 0
    for i, p in enumerate(prompts):
        got, _ = o.greedy(p, tokens.shape[1])
        for t in range(tokens.shape[1]):
            if margins[i, t] < 1e-4:
                break
            assert got[t] == tokens[i, t], (i, t)
            compared += 1
    assert compared >= 8 * 16
