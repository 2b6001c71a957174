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
                 num_context_blocks: int = 0, graph_batch: Optional[int] = None,
                 prefix_stats: tuple[int, int] = (0, 0)) -> None:
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
        self.graph_batch = graph_batch                 # padded batch of a graph replay
        # shared-prefix pass of this step: block reads it saves, and the
        # (member row, 128-key split) partials it writes and merges
        self.prefix_saved_blocks, self.prefix_partial_rows = prefix_stats


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
    num_tokens: int = 0          # packed tokens (host-fed + device-fed)
    uses_device_tokens: bool = False


def build_step(seq_groups: list[SequenceGroup], block_manager) -> StepDescriptors:
    """Descriptors of the scheduled sequences in order.  A prefill feeds
    prompt[nc : nc + q] with q = num_scheduled_tokens (or, outside the
    scheduler, the rest of the prompt as the reference does,
    model_runner.py:201-205) and samples when it reaches the prompt's end; a
    decode feeds its last token at position total_len - 1
    (model_runner.py:217-229).  When that last token is still in flight
    (sampled by the previous step, not yet on the host) the descriptor
    points at its row of the previous step's sampled ids (token_index) and
    the position is total_len + num_inflight - 1."""
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
    uses_device_tokens = False
    for i, (sg, seq) in enumerate(seqs):
        ids = block_manager.get_block_table(seq.seq_id).ids
        seq_ids.append(seq.seq_id)
        tok_off, tok_index = len(tokens), -1
        if seq.is_prefill:
            is_prefill = True
            nc = seq.num_computed_tokens
            q = seq.num_scheduled_tokens or (seq.data.prompt_len - nc)
            tokens.extend(seq.data.prompt_token_ids[nc:nc + q])
            samples = nc + q >= seq.data.prompt_len
        else:
            if i == num_decodes:
                num_decodes += 1
            nc = seq.data.total_len + seq.num_inflight - 1
            q = 1
            if seq.num_inflight > 0:
                tok_index = seq.inflight_row
                uses_device_tokens = True
            else:
                tokens.append(seq.data.last_token)
            samples = True
        descs[i] = (nc, q, len(ids), n_blocks, tok_off, tok_index)
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
                           seq_ids, num_decodes, max_blocks, max_q, is_prefill, n_tok,
                           uses_device_tokens)


# Shared-prefix attention: work items per step (graph-static) and the block
# reads a step must save before the extra pass pays for itself (the pass
# costs about what reading a thousand 16-token blocks of all kv heads does).
PREFIX_MAX_ITEMS = 64
PREFIX_MIN_SAVED_BLOCKS = int(os.environ.get("LV_PREFIX_MIN_BLOCKS", "1024"))


def find_shared_prefixes(descs: np.ndarray, block_ids: np.ndarray, num_decodes: int,
                         block_size: int, group_size: int, max_items: int = PREFIX_MAX_ITEMS,
                         min_saved: Optional[int] = None) -> list[tuple[np.ndarray, int]]:
    """Groups of decode rows whose block tables start with the same physical
    blocks (prefix-cache hits on a common prompt, forked sequences) and the
    length of each group's common run of blocks: at most
    ops.PREFIX_MAX_BLOCKS and never past any member's context
    (prefix * block_size <= context length).  Returns [] unless reading each
    prefix once saves at least ``min_saved`` block reads (default
    PREFIX_MIN_SAVED_BLOCKS); keeps the groups with the largest savings
    within ``max_items`` work items."""
    if min_saved is None:
        min_saved = PREFIX_MIN_SAVED_BLOCKS
    if num_decodes < 2 or block_ids.size == 0:
        return []
    d = descs[:num_decodes].astype(np.int64)
    nblk, off = d[:, 2], d[:, 3]
    cap_row = np.minimum(np.minimum((d[:, 0] + d[:, 1]) // block_size, nblk),
                         ops.PREFIX_MAX_BLOCKS)
    rows = np.nonzero(cap_row > 0)[0]
    if rows.size < 2:
        return []
    first = block_ids[off[rows]]
    order = np.argsort(first, kind="stable")
    rows, first = rows[order], first[order]
    head = np.ones(rows.size, dtype=bool)
    head[1:] = first[1:] != first[:-1]
    gid = np.cumsum(head) - 1
    sizes = np.bincount(gid)
    keep = sizes[gid] >= 2
    if not keep.any():
        return []
    rows, first = rows[keep], first[keep]
    head = np.ones(rows.size, dtype=bool)
    head[1:] = first[1:] != first[:-1]
    starts = np.nonzero(head)[0]
    gid = np.cumsum(head) - 1
    sizes = np.diff(np.append(starts, rows.size))
    leader = rows[starts][gid]
    cap_g = np.minimum.reduceat(cap_row[rows], starts)
    j = np.arange(int(cap_g.max()))
    last = block_ids.size - 1
    mine = block_ids[np.minimum(off[rows][:, None] + j, last)]
    lead = block_ids[np.minimum(off[leader][:, None] + j, last)]
    eq = (mine == lead) | (j >= cap_g[gid][:, None])
    lcp = np.where(eq.all(1), j.size, np.argmin(eq, axis=1))
    lcp_g = np.minimum(np.minimum.reduceat(lcp, starts), cap_g)
    saved = (sizes - 1) * lcp_g
    if int(saved.sum()) < min_saved:
        return []
    groups, items = [], 0
    for g in np.argsort(-saved, kind="stable"):
        if lcp_g[g] <= 0:
            break
        grp = (rows[starts[g]:starts[g] + sizes[g]], int(lcp_g[g]))
        need = ops.prefix_items_needed([grp], group_size, block_size)
        if items + need <= max_items:
            groups.append(grp)
            items += need
    return groups


def prefix_stats(groups, block_size: int) -> tuple[int, int]:
    """(block reads saved, member-split partials) of a list of groups."""
    saved = sum((len(rows) - 1) * pb for rows, pb in groups)
    parts = sum(len(rows) * -(-pb * block_size // ops.PREFIX_KEYS_PER_SPLIT)
                for rows, pb in groups)
    return saved, parts


class _Staging:
    """Grow-only pinned host buffers for one step's packing inputs.  The
    copies out of them are asynchronous, so get() first waits for the
    previous step's copies (record() marks them) before the host rewrites
    the buffers."""

    def __init__(self) -> None:
        self._event: Optional[torch.cuda.Event] = None
        self.i32 = torch.empty(0, dtype=torch.int32).pin_memory() if torch.cuda.is_available() \
            else torch.empty(0, dtype=torch.int32)
        self.i64 = torch.empty(0, dtype=torch.int64).pin_memory() if torch.cuda.is_available() \
            else torch.empty(0, dtype=torch.int64)

    def record(self) -> None:
        if torch.cuda.is_available():
            if self._event is None:
                self._event = torch.cuda.Event()
            self._event.record()

    def get(self, n32: int, n64: int) -> tuple[torch.Tensor, torch.Tensor]:
        if self._event is not None:
            self._event.synchronize()
        if self.i32.numel() < n32:
            self.i32 = torch.empty(max(n32, 2 * self.i32.numel()), dtype=torch.int32,
                                   pin_memory=torch.cuda.is_available())
        if self.i64.numel() < n64:
            self.i64 = torch.empty(max(n64, 2 * self.i64.numel()), dtype=torch.int64,
                                   pin_memory=torch.cuda.is_available())
        return self.i32[:n32], self.i64[:n64]


GRAPH_BATCHES = (1, 2, 4, 8, 16, 24, 32, 48, 64, 80, 96, 112, 128, 144, 160, 176, 192, 208,
                 224, 240, 256, 320, 384, 448, 512)


class DecodeGraphs:
    """HIP graphs of the decode-only forward, one per padded batch size.

    All graphs read one set of static buffers: the packing kernel runs
    eagerly before a replay and writes input ids, positions, slots, context
    lengths and block tables (max_blocks = max_model_len / block_size wide)
    into them.  A batch of B decodes replays the graph of the smallest
    captured size b >= B; the b - B padding rows are one-token sequences
    without blocks, so their slot is 0 -- block 0 is reserved as scratch
    (the reference's convention, cache/block_manager.py:20-27) -- and their
    logits are dropped.  The attention workspace is sized for the largest
    batch and owned here, so no replay reads memory another call may free.
    """

    def __init__(self, runner: "ModelRunner", max_batch: int) -> None:
        mc = runner.model_config
        cc = runner.config.cache_config
        dev = torch.device(runner.device)
        self.runner = runner
        self.block_size = cc.block_size
        self.max_blocks = (mc.max_model_len + cc.block_size - 1) // cc.block_size
        self.batches = [b for b in GRAPH_BATCHES if b < max_batch] + [max_batch]
        n = max_batch
        self.descs = torch.zeros((n, 6), dtype=torch.int32, device=dev)
        self.block_ids = torch.zeros(n * self.max_blocks, dtype=torch.int32, device=dev)
        self.token_ids = torch.zeros(n, dtype=torch.int64, device=dev)
        self.packed = {
            "input_ids": torch.zeros(n, dtype=torch.int64, device=dev),
            "positions": torch.zeros(n, dtype=torch.int64, device=dev),
            "slot_mapping": torch.zeros(n, dtype=torch.int64, device=dev),
            "cu_seqlens": torch.zeros(n + 1, dtype=torch.int32, device=dev),
            "seq_start": torch.zeros(n, dtype=torch.int32, device=dev),
            "context_lens": torch.zeros(n, dtype=torch.int32, device=dev),
            "block_tables": torch.zeros((n, self.max_blocks), dtype=torch.int32, device=dev),
        }
        ws = max(ops.paged_attention_workspace_size(b, b, b, mc.num_attention_heads, mc.head_dim,
                                                    cc.block_size, self.max_blocks, 1,
                                                    mc.torch_dtype) for b in self.batches)
        self.workspace = torch.empty(max(ws, 256), dtype=torch.uint8, device=dev)
        # Shared-prefix plan, one static int32 buffer: blocks [n] (padded to
        # a multiple of 4 so the items stay 16-byte aligned), items
        # [PREFIX_MAX_ITEMS, 4], members [n].  Every graph reads all of it;
        # rows and items beyond a graph's batch are skipped by the kernel.
        self.group_size = mc.num_attention_heads // mc.num_key_value_heads
        self.use_prefix = cc.shared_prefix_attention and ops.prefix_attention_supported(
            mc.num_attention_heads, mc.num_key_value_heads, mc.head_dim, cc.block_size,
            mc.torch_dtype)
        self._pfx_active = False
        if self.use_prefix:
            npad = (n + 3) // 4 * 4
            self.pfx_buf = torch.zeros(npad + 4 * PREFIX_MAX_ITEMS + n, dtype=torch.int32,
                                       device=dev)
            self.pfx_buf[npad:npad + 4 * PREFIX_MAX_ITEMS].view(-1, 4)[:, 0] = -1
            self.pfx_plan = ops.PrefixPlan(
                self.pfx_buf[:n], self.pfx_buf[npad:npad + 4 * PREFIX_MAX_ITEMS].view(-1, 4),
                self.pfx_buf[npad + 4 * PREFIX_MAX_ITEMS:])
            self.pfx_npad = npad
            self.pfx_workspace = torch.empty(
                max(ops.prefix_workspace_size(n, mc.num_attention_heads, mc.head_dim), 256),
                dtype=torch.uint8, device=dev)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.logits: dict[int, torch.Tensor] = {}
        tmpl = torch.zeros((n, 6), dtype=torch.int32)
        tmpl[:, 1] = 1                                   # query_len 1
        tmpl[:, 4] = torch.arange(n, dtype=torch.int32)  # token_offset = row
        tmpl[:, 5] = -1                                  # ids from token_ids
        self._pad_template = tmpl.to(dev)

    def _views(self, b: int) -> dict[str, torch.Tensor]:
        p = self.packed
        return {"input_ids": p["input_ids"][:b], "positions": p["positions"][:b],
                "slot_mapping": p["slot_mapping"][:b], "cu_seqlens": p["cu_seqlens"][:b + 1],
                "seq_start": p["seq_start"][:b], "context_lens": p["context_lens"][:b],
                "block_tables": p["block_tables"][:b]}

    def _forward(self, b: int) -> torch.Tensor:
        v = self._views(b)
        meta = AttentionMetadata(block_tables=v["block_tables"], context_lens=v["context_lens"],
                                 cu_seqlens=v["cu_seqlens"], num_decodes=b, max_query_len=1,
                                 workspace=self.workspace)
        if self.use_prefix:
            p = self.pfx_plan
            meta.prefix = ops.PrefixPlan(p.blocks[:b], p.items, p.members)
            meta.prefix_workspace = self.pfx_workspace
        r = self.runner
        kv = [r.kv_cache.get_kv(i) for i in range(r.model_config.num_hidden_layers)]
        return r.model(input_ids=v["input_ids"], positions=v["positions"], kv_caches=kv,
                       slot_mapping=v["slot_mapping"], block_tables=v["block_tables"],
                       context_lens=v["context_lens"], is_prefill=False, attn_metadata=meta,
                       logits_indices=None)

    def _pack(self, b: int, num_block_ids: int,
              device_tokens: Optional[torch.Tensor] = None) -> None:
        ops.pack_inputs(self.descs[:b], self.block_ids[:max(num_block_ids, 1)],
                        self.token_ids[:b], b, self.block_size, self.max_blocks,
                        device_tokens=device_tokens, out=self._views(b))

    @torch.inference_mode()
    def capture(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        for b in sorted(self.batches, reverse=True):
            self._pad_rows(0, b)
            self._pack(b, 1)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._forward(b)
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self.logits[b] = self._forward(b)
            self.graphs[b] = g
        torch.cuda.synchronize()

    def accepts(self, st: StepDescriptors) -> bool:
        B = st.descs.shape[0]
        return (B > 0 and st.num_decodes == B and B <= self.batches[-1]
                and st.max_blocks <= self.max_blocks and bool(self.graphs))

    def prepare(self, st: StepDescriptors, staging: "_Staging",
                device_tokens: Optional[torch.Tensor], may_share: bool = True) -> InputMetadata:
        B = st.descs.shape[0]
        b = next(x for x in self.batches if x >= B)
        nb = st.block_ids.shape[0]
        n_host = len(st.tokens)
        groups = find_shared_prefixes(st.descs, st.block_ids, B, self.block_size,
                                      self.group_size) if self.use_prefix and may_share else []
        n_pfx = self.pfx_buf.numel() if (groups or self._pfx_active) else 0
        st32, st64 = staging.get(B * 6 + nb + n_pfx, max(n_host, 1))
        a32 = st32.numpy()
        a32[:B * 6] = st.descs.reshape(-1)
        a32[B * 6:B * 6 + nb] = st.block_ids
        st64.numpy()[:n_host] = st.tokens
        self.descs[:B].view(-1).copy_(st32[:B * 6], non_blocking=True)
        self.block_ids[:nb].copy_(st32[B * 6:B * 6 + nb], non_blocking=True)
        if n_pfx:
            # a new plan, or the empty one replacing the previous step's
            n = self.batches[-1]
            blocks, items, members = ops.prefix_plan_arrays(
                groups, n, self.group_size, self.block_size, max_items=PREFIX_MAX_ITEMS,
                max_members=n)
            r = a32[B * 6 + nb:]
            r[:n] = blocks
            r[n:self.pfx_npad] = 0
            r[self.pfx_npad:self.pfx_npad + items.size] = items.reshape(-1)
            r[self.pfx_npad + items.size:] = members
            self.pfx_buf.copy_(st32[B * 6 + nb:], non_blocking=True)
            self._pfx_active = bool(groups)
        if n_host:
            self.token_ids[:n_host].copy_(st64[:n_host], non_blocking=True)
        staging.record()
        if b > B:
            self._pad_rows(B, b)
        self._pack(b, nb, device_tokens)
        return InputMetadata(None, None, None, None, None, False, st.seq_ids,
                             sample_seqs=st.sample_seqs, sample_groups=st.sample_groups,
                             num_decodes=B,
                             num_context_tokens=int(st.descs[:, 0].sum() + st.descs[:, 1].sum()),
                             num_context_blocks=int(nb), graph_batch=b,
                             prefix_stats=prefix_stats(groups, self.block_size))

    def _pad_rows(self, start: int, b: int) -> None:
        """Descriptors start..b-1 become padding: one token (id 0) at
        position 0 with no blocks, i.e. slot 0 in the scratch block."""
        self.descs[start:b].copy_(self._pad_template[start:b])
        self.token_ids[start:b].zero_()

    def replay(self, meta: InputMetadata) -> torch.Tensor:
        self.graphs[meta.graph_batch].replay()
        return self.logits[meta.graph_batch][:meta.num_decodes]


class ModelRunner:
    def __init__(self, engine_config: EngineConfig) -> None:
        self.config = engine_config
        self.model_config = engine_config.model_config
        self.device = engine_config.device
        self.model: Optional[BaseModelForCausalLM] = None
        self.kv_cache: Optional[KVCache] = None
        self._staging = _Staging()
        self.graphs: Optional[DecodeGraphs] = None

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

    def capture_decode_graphs(self) -> None:
        """Capture the decode-only forward for every padded batch size up to
        the scheduler's max_num_seqs (block 0 must be reserved as scratch)."""
        max_batch = min(self.config.max_graph_batch, self.config.scheduler_config.max_num_seqs)
        graphs = DecodeGraphs(self, max_batch)
        graphs.capture()
        self.graphs = graphs

    # ------------------------------------------------------------------
    def prepare_inputs(self, seq_groups: list[SequenceGroup], block_manager,
                       device_tokens: Optional[torch.Tensor] = None) -> InputMetadata:
        """Pack the scheduled sequences (decodes first, then prefill chunks).
        ``device_tokens``: the previous step's sampled ids, read by decodes
        whose last token is still in flight."""
        st = build_step(seq_groups, block_manager)
        if st.uses_device_tokens and device_tokens is None:
            raise RuntimeError("a decode's last token is in flight but no device tokens were given")
        if self.graphs is not None and self.graphs.accepts(st):
            return self.graphs.prepare(st, self._staging, device_tokens,
                                       self._may_share(block_manager))
        B, n_blocks = st.descs.shape[0], st.block_ids.shape[0]
        n_host, T = len(st.tokens), st.num_tokens
        h = max(n_host, 1)                   # keep the id array non-empty
        dev = torch.device(self.device)
        n32 = B * 6 + n_blocks
        plan_arrays = self._prefix_arrays(st) if self._may_share(block_manager) else None
        p0 = (n32 + 3) // 4 * 4              # plan after the tables, 16-byte aligned
        n_all = p0 + sum(a.size for a in plan_arrays[:3]) + 4 if plan_arrays else n32
        st32, st64 = self._staging.get(n_all, h + len(st.logits_rows))
        a32 = st32.numpy()
        a32[:B * 6] = st.descs.reshape(-1)
        a32[B * 6:n32] = st.block_ids
        stats = (0, 0)
        if plan_arrays:
            blocks, items, members, stats = plan_arrays
            nd = blocks.size
            i0 = p0 + (nd + 3) // 4 * 4
            a32[p0:p0 + nd] = blocks
            a32[i0:i0 + items.size] = items.reshape(-1)
            a32[i0 + items.size:i0 + items.size + members.size] = members
        a64 = st64.numpy()
        a64[:n_host] = st.tokens
        a64[h:] = st.logits_rows
        d32 = st32.to(dev, non_blocking=True)
        d64 = st64.to(dev, non_blocking=True)
        self._staging.record()
        packed = ops.pack_inputs(d32[:B * 6].view(B, 6), d32[B * 6:], d64[:h], T,
                                 self.config.cache_config.block_size, max(st.max_blocks, 1),
                                 device_tokens=device_tokens)
        attn = AttentionMetadata(block_tables=packed["block_tables"],
                                 context_lens=packed["context_lens"],
                                 cu_seqlens=packed["cu_seqlens"], num_decodes=st.num_decodes,
                                 max_query_len=st.max_query_len)
        if plan_arrays:
            attn.prefix = ops.PrefixPlan(d32[p0:p0 + nd], d32[i0:i0 + items.size].view(-1, 4),
                                         d32[i0 + items.size:i0 + items.size + members.size])
        return InputMetadata(packed["input_ids"], packed["positions"], packed["slot_mapping"],
                             packed["block_tables"], packed["context_lens"], st.is_prefill,
                             st.seq_ids, attn_metadata=attn, logits_indices=d64[h:],
                             sample_seqs=st.sample_seqs, sample_groups=st.sample_groups,
                             num_decodes=st.num_decodes,
                             num_context_tokens=int(st.descs[:, 0].sum() + st.descs[:, 1].sum()),
                             num_context_blocks=int(n_blocks), prefix_stats=stats)

    def _may_share(self, block_manager) -> bool:
        """Whether block tables can share leading blocks: only prefix-cache
        hits and forked tables do (otherwise the group search is skipped)."""
        return (self.config.cache_config.enable_prefix_caching
                or getattr(block_manager, "num_forks", 1) > 0)

    def _prefix_arrays(self, st: StepDescriptors):
        """Host plan of the step's shared decode prefixes, or None."""
        cc = self.config.cache_config
        mc = self.model_config
        if not cc.shared_prefix_attention or not 2 <= st.num_decodes <= ops.PREFIX_MAX_DECODES:
            return None
        if not ops.prefix_attention_supported(mc.num_attention_heads, mc.num_key_value_heads,
                                              mc.head_dim, cc.block_size, mc.torch_dtype):
            return None
        g = mc.num_attention_heads // mc.num_key_value_heads
        groups = find_shared_prefixes(st.descs, st.block_ids, st.num_decodes, cc.block_size, g)
        if not groups:
            return None
        return (*ops.prefix_plan_arrays(groups, st.num_decodes, g, cc.block_size),
                prefix_stats(groups, cc.block_size))

    @torch.inference_mode()
    def execute_model(self, metadata: InputMetadata) -> torch.Tensor:
        """Forward pass; logits of the sampled rows only ([len(sample_seqs), V])."""
        if metadata.graph_batch is not None:
            return self.graphs.replay(metadata)
        kv_caches = None
        if self.kv_cache is not None:
            kv_caches = [self.kv_cache.get_kv(i) for i in range(self.model_config.num_hidden_layers)]
        return self.model(input_ids=metadata.input_ids, positions=metadata.positions,
                          kv_caches=kv_caches, slot_mapping=metadata.slot_mapping,
                          block_tables=metadata.block_tables, context_lens=metadata.context_lens,
                          is_prefill=metadata.is_prefill, attn_metadata=metadata.attn_metadata,
                          logits_indices=metadata.logits_indices)
