"""CPU fp32 restatement of the reference decoder models and greedy decoding
(test oracle for the end-to-end engine).

Restates LlamaForCausalLM / Qwen3ForCausalLM (reference models/llama.py:
18-198, models/qwen3.py:24-195, layers/rotary_emb.py:79-117) one sequence
at a time with a plain growing K/V list instead of a paged cache: prefill is
causal attention over the prompt (attention.py:141-151), each decode step
attends the whole history (attention.py:91-139).  Weights come from a model
state dict in this build's fused layout (qkv_proj, gate_up_proj), split back
into the reference's separate projections.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


class OracleDecoder:
    def __init__(self, state: dict[str, torch.Tensor], cfg, use_qk_norm: bool) -> None:
        self.cfg = cfg
        self.use_qk_norm = use_qk_norm
        self.w = {k: v.detach().to("cpu", torch.float32) for k, v in state.items()}
        d = cfg.head_dim
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        t = torch.arange(cfg.max_position_embeddings, dtype=torch.float32)
        freqs = torch.outer(t, inv)
        self.cos, self.sin = freqs.cos(), freqs.sin()

    def _rms(self, x, w):
        var = x.pow(2).mean(-1, keepdim=True)
        return w * (x * torch.rsqrt(var + self.cfg.rms_norm_eps))

    def _rope(self, x, pos):
        c = self.cos[pos].unsqueeze(1)
        s = self.sin[pos].unsqueeze(1)
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)

    def forward(self, ids: list[int], pos0: int, kv: list) -> torch.Tensor:
        """Feed tokens at positions pos0.., append their K/V to kv (one
        (K, V) pair per layer), return the logits of the last token."""
        c, w = self.cfg, self.w
        H, Hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        T = len(ids)
        pos = torch.arange(pos0, pos0 + T)
        x = w["model.embed_tokens.weight"][torch.tensor(ids)]
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}."
            h = self._rms(x, w[p + "input_layernorm.weight"])
            qkv = h @ w[p + "self_attn.qkv_proj.weight"].t()
            q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
            q, k, v = q.view(T, H, D), k.view(T, Hkv, D), v.view(T, Hkv, D)
            if self.use_qk_norm:
                q = self._rms(q, w[p + "self_attn.q_norm.weight"])
                k = self._rms(k, w[p + "self_attn.k_norm.weight"])
            q, k = self._rope(q, pos), self._rope(k, pos)
            if len(kv) <= i:
                kv.append((k, v))
            else:
                kv[i] = (torch.cat([kv[i][0], k]), torch.cat([kv[i][1], v]))
            K, V = kv[i]
            K = K.repeat_interleave(H // Hkv, dim=1).permute(1, 0, 2)
            V = V.repeat_interleave(H // Hkv, dim=1).permute(1, 0, 2)
            s = torch.matmul(q.permute(1, 0, 2), K.transpose(1, 2)) / math.sqrt(D)
            qpos = pos.unsqueeze(1)
            kpos = torch.arange(K.shape[1]).unsqueeze(0)
            s = s.masked_fill((kpos > qpos).unsqueeze(0), float("-inf"))
            a = torch.matmul(F.softmax(s, dim=-1), V).permute(1, 0, 2).reshape(T, H * D)
            x = x + a @ w[p + "self_attn.o_proj.weight"].t()
            h = self._rms(x, w[p + "post_attention_layernorm.weight"])
            gu = h @ w[p + "mlp.gate_up_proj.weight"].t()
            g, u = gu.split(c.intermediate_size, dim=-1)
            x = x + (F.silu(g) * u) @ w[p + "mlp.down_proj.weight"].t()
        x = self._rms(x[-1:], w["model.norm.weight"])
        head = w.get("lm_head.weight", w["model.embed_tokens.weight"])
        return (x @ head.t())[0]

    def decode_batch(self, tokens: list[int], positions: list[int], kvs: list[list]) -> torch.Tensor:
        """One decode step for B sequences at once, the way the reference's
        CPU path batches decodes (model_runner.py:217-250, attention.py:
        91-139): projections and MLP over the B rows together, attention per
        sequence over its own history.  kvs[b] is sequence b's K/V list (as
        forward builds it); returns the logits [B, V]."""
        c, w = self.cfg, self.w
        H, Hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        B = len(tokens)
        pos = torch.tensor(positions)
        x = w["model.embed_tokens.weight"][torch.tensor(tokens)]
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}."
            h = self._rms(x, w[p + "input_layernorm.weight"])
            q, k, v = (h @ w[p + "self_attn.qkv_proj.weight"].t()).split([H * D, Hkv * D, Hkv * D],
                                                                          dim=-1)
            q, k, v = q.view(B, H, D), k.view(B, Hkv, D), v.view(B, Hkv, D)
            if self.use_qk_norm:
                q = self._rms(q, w[p + "self_attn.q_norm.weight"])
                k = self._rms(k, w[p + "self_attn.k_norm.weight"])
            q, k = self._rope(q, pos), self._rope(k, pos)
            outs = []
            for b in range(B):
                K0, V0 = kvs[b][i]
                K = torch.cat([K0, k[b:b + 1]])
                V = torch.cat([V0, v[b:b + 1]])
                kvs[b][i] = (K, V)
                Kr = K.repeat_interleave(H // Hkv, dim=1).permute(1, 0, 2)
                Vr = V.repeat_interleave(H // Hkv, dim=1).permute(1, 0, 2)
                s = torch.matmul(q[b].unsqueeze(1), Kr.transpose(1, 2)) / math.sqrt(D)
                outs.append(torch.matmul(F.softmax(s, dim=-1), Vr).reshape(H * D))
            x = x + torch.stack(outs) @ w[p + "self_attn.o_proj.weight"].t()
            h = self._rms(x, w[p + "post_attention_layernorm.weight"])
            g, u = (h @ w[p + "mlp.gate_up_proj.weight"].t()).split(c.intermediate_size, dim=-1)
            x = x + (F.silu(g) * u) @ w[p + "mlp.down_proj.weight"].t()
        x = self._rms(x, w["model.norm.weight"])
        head = w.get("lm_head.weight", w["model.embed_tokens.weight"])
        return x @ head.t()

    def greedy(self, prompt: list[int], n: int) -> tuple[list[int], list[float]]:
        """n greedy tokens; also the top-1 minus top-2 logit margin of each."""
        kv: list = []
        logits = self.forward(prompt, 0, kv)
        out, margins = [], []
        pos = len(prompt)
        for _ in range(n):
            top = torch.topk(logits, 2)
            tok = int(torch.argmax(logits))
            out.append(tok)
            margins.append(float(top.values[0] - top.values[1]))
            logits = self.forward([tok], pos, kv)
            pos += 1
        return out, margins
