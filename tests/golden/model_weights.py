"""Deterministic checkpoint recipe shared by the reference-model fixtures.

``make_weights(cfg, seed)`` returns a state dict under the Hugging Face
parameter names that both the reference's ``load_weights`` and this build's
``LlamaForCausalLM.load_weights`` accept (separate q/k/v and gate/up
projections).  Every tensor comes from its own CPU generator seeded with
(seed, index in a fixed name order), so a test can rebuild the exact
weights the fixture script fed to the reference without shipping them.

Scales are chosen so every part of the network matters to the logits:
embeddings N(0, 1); projections N(0, 0.1^2), which gives attention scores of
order 1 (the softmax is far from uniform); norm weights 1 + 0.2 N(0, 1), so
a dropped or misplaced norm weight changes the result.
"""

from __future__ import annotations

import torch

# architecture dicts (the config.json fields both builds read)
QWEN3_TINY = dict(model_type="qwen3", vocab_size=512, hidden_size=128, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                  intermediate_size=256, rope_theta=1e6, rms_norm_eps=1e-6,
                  max_position_embeddings=1024, tie_word_embeddings=False)
# head_dim = hidden / heads = 64 (the attention kernels take head_dim 64 or 128)
LLAMA_TINY = dict(model_type="llama", vocab_size=512, hidden_size=256, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, intermediate_size=320,
                  rope_theta=10000.0, rms_norm_eps=1e-5, max_position_embeddings=1024,
                  tie_word_embeddings=False)
# config 1 (SURVEY config table): tiny Llama, vocab 32000
CONFIG1_LLAMA = dict(model_type="llama", vocab_size=32000, hidden_size=256, num_hidden_layers=2,
                     num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                     intermediate_size=688, rope_theta=10000.0, rms_norm_eps=1e-6,
                     max_position_embeddings=4096, tie_word_embeddings=False)


def param_shapes(cfg: dict) -> dict[str, tuple[int, ...]]:
    hidden = cfg["hidden_size"]
    heads = cfg["num_attention_heads"]
    kv = cfg.get("num_key_value_heads", heads)
    d = cfg.get("head_dim") or hidden // heads
    inter = cfg["intermediate_size"]
    qk_norm = cfg["model_type"] == "qwen3"
    shapes = {"model.embed_tokens.weight": (cfg["vocab_size"], hidden)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        shapes[p + "input_layernorm.weight"] = (hidden,)
        shapes[p + "self_attn.q_proj.weight"] = (heads * d, hidden)
        shapes[p + "self_attn.k_proj.weight"] = (kv * d, hidden)
        shapes[p + "self_attn.v_proj.weight"] = (kv * d, hidden)
        shapes[p + "self_attn.o_proj.weight"] = (hidden, heads * d)
        if qk_norm:
            shapes[p + "self_attn.q_norm.weight"] = (d,)
            shapes[p + "self_attn.k_norm.weight"] = (d,)
        shapes[p + "post_attention_layernorm.weight"] = (hidden,)
        shapes[p + "mlp.gate_proj.weight"] = (inter, hidden)
        shapes[p + "mlp.up_proj.weight"] = (inter, hidden)
        shapes[p + "mlp.down_proj.weight"] = (hidden, inter)
    shapes["model.norm.weight"] = (hidden,)
    if not cfg.get("tie_word_embeddings", False):
        shapes["lm_head.weight"] = (cfg["vocab_size"], hidden)
    return shapes


def make_weights(cfg: dict, seed: int) -> dict[str, torch.Tensor]:
    out = {}
    for i, (name, shape) in enumerate(sorted(param_shapes(cfg).items())):
        g = torch.Generator().manual_seed(seed * 100003 + i)
        x = torch.randn(shape, generator=g, dtype=torch.float32)
        if name.endswith("norm.weight"):
            x = 1.0 + 0.2 * x
        elif not name.endswith("embed_tokens.weight"):
            x = 0.1 * x
        out[name] = x
    return out


def fused_state(cfg: dict, weights: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The same weights in this build's fused layout (qkv_proj = [q; k; v],
    gate_up_proj = [gate; up]) -- what oracle.model.OracleDecoder reads."""
    out = {}
    for name, w in weights.items():
        if ".q_proj." in name:
            base = name.replace("q_proj", "qkv_proj")
            out[base] = torch.cat([w, weights[name.replace("q_proj", "k_proj")],
                                   weights[name.replace("q_proj", "v_proj")]])
        elif ".gate_proj." in name:
            out[name.replace("gate_proj", "gate_up_proj")] = torch.cat(
                [w, weights[name.replace("gate_proj", "up_proj")]])
        elif any(k in name for k in (".k_proj.", ".v_proj.", ".up_proj.")):
            continue
        else:
            out[name] = w
    return out


def config1_prompts() -> list[list[int]]:
    """Config 1's prompts: 8 prompts, lengths U[16, 64], ids U[0, 32000)."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(16, 65, (8,), generator=g).tolist()
    return [torch.randint(0, 32000, (n,), generator=g).tolist() for n in lens]
