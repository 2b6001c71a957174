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
