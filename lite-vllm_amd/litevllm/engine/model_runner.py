"""ModelRunner: weights, KV cache, per-step packing and the forward pass.

Interface of the reference (engine/model_runner.py:84-280): InputMetadata,
ModelRunner.load_model / init_kv_cache / profile_num_gpu_blocks /
prepare_inputs / execute_model.

prepare_inputs no longer builds per-token Python lists and synchronous
torch.tensor copies (model_runner.py:196-250).  It writes one descriptor per
sequence (lv_seq_desc: num_computed, query_len, table length and offsets)
plus the flat block ids and the fed token ids into pinned staging memory,
issues two asynchronous copies, and lv_pack_inputs expands them on the GPU
into input_ids / positions / slot_mapping / cu_seqlens / context_lens /
block tables (the reference's rules, bit-exact).  A batch is one mixed
forward: decodes first, then prefill chunks; only the rows that are sampled
(every decode, and a chunk that completes its prompt) go through the LM head.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .. import ops
from ..cache.kv_cache import KVCache
from ..config import EngineConfig
from ..layers.attention import AttentionMetadata
from ..models.base import BaseModelForCausalLM
from .sequence import Sequence, SequenceGroup


def _resolve_model_dir(model_name_or_path: str) -> str:
    if os.path.isdir(model_name_or_path):
        return model_name_or_path
    raise FileNotFoundError(f"Cannot find model weights at {model_name_or_path}: give a local "
                            "directory or load_format='dummy'")


@torch.inference_mode()
def _load_model_weights(model: BaseModelForCausalLM, model_dir: str, dtype: torch.dtype) -> None:
    """safetensors first, then *.bin (weights_only), as the reference
    (model_runner.py:40-81)."""
    from glob import glob
    st_files = sorted(glob(os.path.join(model_dir, "*.safetensors")))
    weights: dict[str, torch.Tensor] = {}
    if st_files:
        from safetensors import safe_open
        for f in st_files:
            with safe_open(f, framework="pt", device="cpu") as sf:
                for key in sf.keys():
                    weights[key] = sf.get_tensor(key).to(dtype)
    else:
        for f in sorted(glob(os.path.join(model_dir, "*.bin"))):
            for k, v in torch.load(f, map_location="cpu", weights_only=True).items():
                weights[k] = v.to(dtype)
    if not weights:
        raise FileNotFoundError(f"No safetensors or pytorch checkpoint found in {model_dir}")
    model.load_weights(weights)


class InputMetadata:
    """Packed tensors of one forward step (reference model_runner.py:84-103)
    plus what the mixed-batch attention and the sampler need."""

    def __init__(self, input_ids, positions, slot_mapping, block_tables, context_lens,
                 is_prefill, seq_ids, attn_metadata: Optional[AttentionMetadata] = None,
                 logits_indices: Optional[torch.Tensor] = None,
                 sample_seqs: Optional[list[Sequence]] = None,
                 sample_groups: Optional[list[SequenceGroup]] = None,
                 num_decodes: int = 0, num_context_tokens: int = 0,
                 num_context_blocks: int = 0) -> None:
        self.input_ids = input_ids
        self.positions = positions
        self.slot_mapping = slot_mapping
        self.block_tables = block_tables
        self.context_lens = context_lens
        self.is_prefill = is_prefill
        self.seq_ids = seq_ids
        self.attn_metadata = attn_metadata
        self.logits_indices = logits_indices
        self.sample_seqs = sample_seqs or []
        self.sample_groups = sample_groups or []
        self.num_decodes = num_decodes                 # leading 1-token sequences
        self.num_context_tokens = num_context_tokens   # sum of context lengths (host)
        self.num_context_blocks = num_context_blocks   # sum of block-table lengths (host)


@dataclass
class StepDescriptors:
    """Host side of one step's packing (what lv_pack_inputs consumes)."""
    descs: np.ndarray            # int32 [B, 6], lv_seq_desc rows
    block_ids: np.ndarray        # int32 flat block tables
    tokens: list[int]            # fed token ids, packed order
    logits_rows: list[int]       # packed rows whose logits are sampled
    sample_seqs: list[Sequence]
    sample_groups: list[SequenceGroup]
    seq_ids: list[int]
    num_decodes: int             # leading 1-token sequences
    max_blocks: int
    max_query_len: int
    is_prefill: bool


def build_step(seq_groups: list[SequenceGroup], block_manager) -> StepDescriptors:
    """Descriptors of the scheduled sequences in order.  A prefill feeds
    prompt[nc : nc + q] with q = num_scheduled_tokens (or, outside the
    scheduler, the rest of the prompt as the reference does,
    model_runner.py:201-205) and samples when it reaches the prompt's end; a
    decode feeds its last token at position total_len - 1
    (model_runner.py:217-229)."""
    seqs = [(sg, s) for sg in seq_groups for s in sg.get_unfinished_seqs()]
    B = len(seqs)
    descs = np.empty((B, 6), dtype=np.int32)
    tables: list[list[int]] = []
    tokens: list[int] = []
    logits_rows: list[int] = []
    sample_seqs: list[Sequence] = []
    sample_groups: list[SequenceGroup] = []
    seq_ids: list[int] = []
    n_blocks = n_tok = max_blocks = max_q = num_decodes = 0
    is_prefill = False
    for i, (sg, seq) in enumerate(seqs):
        ids = block_manager.get_block_table(seq.seq_id).ids
        seq_ids.append(seq.seq_id)
        if seq.is_prefill:
            is_prefill = True
            nc = seq.num_computed_tokens
            q = seq.num_scheduled_tokens or (seq.data.prompt_len - nc)
            tokens.extend(seq.data.prompt_token_ids[nc:nc + q])
            samples = nc + q >= seq.data.prompt_len
        else:
            if i == num_decodes:
                num_decodes += 1
            nc = seq.data.total_len - 1
            q = 1
            tokens.append(seq.data.last_token)
            samples = True
        descs[i] = (nc, q, len(ids), n_blocks, n_tok, -1)
        tables.append(ids)
        n_blocks += len(ids)
        n_tok += q
        max_blocks = max(max_blocks, len(ids))
        max_q = max(max_q, q)
        if samples:
            logits_rows.append(n_tok - 1)
            sample_seqs.append(seq)
            sample_groups.append(sg)
    block_ids = np.fromiter((b for t in tables for b in t), dtype=np.int32, count=n_blocks)
    return StepDescriptors(descs, block_ids, tokens, logits_rows, sample_seqs, sample_groups,
                           seq_ids, num_decodes, max_blocks, max_q, is_prefill)


class _Staging:
    """Grow-only pinned host buffers for one step's packing inputs."""

    def __init__(self) -> None:
        self.i32 = torch.empty(0, dtype=torch.int32).pin_memory() if torch.cuda.is_available() \
            else torch.empty(0, dtype=torch.int32)
        self.i64 = torch.empty(0, dtype=torch.int64).pin_memory() if torch.cuda.is_available() \
            else torch.empty(0, dtype=torch.int64)

    def get(self, n32: int, n64: int) -> tuple[torch.Tensor, torch.Tensor]:
        if self.i32.numel() < n32:
            self.i32 = torch.empty(max(n32, 2 * self.i32.numel()), dtype=torch.int32,
                                   pin_memory=torch.cuda.is_available())
        if self.i64.numel() < n64:
            self.i64 = torch.empty(max(n64, 2 * self.i64.numel()), dtype=torch.int64,
                                   pin_memory=torch.cuda.is_available())
        return self.i32[:n32], self.i64[:n64]


class ModelRunner:
    def __init__(self, engine_config: EngineConfig) -> None:
        self.config = engine_config
        self.model_config = engine_config.model_config
        self.device = engine_config.device
        self.model: Optional[BaseModelForCausalLM] = None
        self.kv_cache: Optional[KVCache] = None
        self._staging = _Staging()

    def load_model(self) -> None:
        mc = self.model_config
        model = BaseModelForCausalLM.get_model_cls(mc.model_type)(mc)
        if mc.load_format == "dummy":
            model.init_dummy_weights(seed=self.config.seed)
            model = model.to(dtype=mc.torch_dtype, device=self.device)
        else:
            model = model.to(dtype=mc.torch_dtype, device=self.device)
            _load_model_weights(model, _resolve_model_dir(mc.model), mc.torch_dtype)
        self.model = model.eval()

    def init_kv_cache(self, num_gpu_blocks: int) -> None:
        mc = self.model_config
        self.kv_cache = KVCache(mc.num_hidden_layers, num_gpu_blocks,
                                self.config.cache_config.block_size, mc.num_key_value_heads,
                                mc.head_dim, mc.torch_dtype, self.device)

    def profile_num_gpu_blocks(self) -> int:
        """KV blocks fitting in gpu_memory_utilization of the device memory
        after the weights (the reference also runs a dummy forward first,
        model_runner.py:142-178; the decode step's activations here are a few
        hundred MB and are covered by the remaining fraction)."""
        fallback = self.config.cache_config.num_gpu_blocks or 256
        if not torch.cuda.is_available() or self.device == "cpu":
            return fallback
        mc = self.model_config
        torch.cuda.synchronize()
        free, total = torch.cuda.mem_get_info()
        used = total - free
        available = int(total * self.config.cache_config.gpu_memory_utilization) - used
        n = KVCache.profile_num_blocks(available, mc.num_hidden_layers,
                                       self.config.cache_config.block_size,
                                       mc.num_key_value_heads, mc.head_dim, mc.torch_dtype)
        return max(n, 16)

    # ------------------------------------------------------------------
    def prepare_inputs(self, seq_groups: list[SequenceGroup], block_manager) -> InputMetadata:
        """Pack the scheduled sequences (decodes first, then prefill chunks)."""
        st = build_step(seq_groups, block_manager)
        B, n_blocks, n_tok = st.descs.shape[0], st.block_ids.shape[0], len(st.tokens)
        dev = torch.device(self.device)
        n32 = B * 6 + n_blocks
        st32, st64 = self._staging.get(n32, n_tok + len(st.logits_rows))
        a32 = st32.numpy()
        a32[:B * 6] = st.descs.reshape(-1)
        a32[B * 6:n32] = st.block_ids
        a64 = st64.numpy()
        a64[:n_tok] = st.tokens
        a64[n_tok:] = st.logits_rows
        d32 = st32.to(dev, non_blocking=True)
        d64 = st64.to(dev, non_blocking=True)
        packed = ops.pack_inputs(d32[:B * 6].view(B, 6), d32[B * 6:], d64[:n_tok], n_tok,
                                 self.config.cache_config.block_size, max(st.max_blocks, 1))
        attn = AttentionMetadata(block_tables=packed["block_tables"],
                                 context_lens=packed["context_lens"],
                                 cu_seqlens=packed["cu_seqlens"], num_decodes=st.num_decodes,
                                 max_query_len=st.max_query_len)
        return InputMetadata(packed["input_ids"], packed["positions"], packed["slot_mapping"],
                             packed["block_tables"], packed["context_lens"], st.is_prefill,
                             st.seq_ids, attn_metadata=attn, logits_indices=d64[n_tok:],
                             sample_seqs=st.sample_seqs, sample_groups=st.sample_groups,
                             num_decodes=st.num_decodes,
                             num_context_tokens=int(st.descs[:, 0].sum() + st.descs[:, 1].sum()),
                             num_context_blocks=int(n_blocks))

    @torch.inference_mode()
    def execute_model(self, metadata: InputMetadata) -> torch.Tensor:
        """Forward pass; logits of the sampled rows only ([len(sample_seqs), V])."""
        kv_caches = None
        if self.kv_cache is not None:
            kv_caches = [self.kv_cache.get_kv(i) for i in range(self.model_config.num_hidden_layers)]
        return self.model(input_ids=metadata.input_ids, positions=metadata.positions,
                          kv_caches=kv_caches, slot_mapping=metadata.slot_mapping,
                          block_tables=metadata.block_tables, context_lens=metadata.context_lens,
                          is_prefill=metadata.is_prefill, attn_metadata=metadata.attn_metadata,
                          logits_indices=metadata.logits_indices)
