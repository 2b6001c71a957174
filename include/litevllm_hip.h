/*
 * litevllm_hip.h — C ABI of the MI355X (gfx950) continuous-batching hot path.
 *
 * One shared library, liblitevllm_hip.so, exports these entry points.  They
 * replace the per-step tensor work of lite-vllm 0.1.0 (pure Python/torch +
 * two Triton kernels); each declaration below cites the reference function
 * it replaces.
 *
 * Conventions (all entry points):
 *   - Every pointer argument named *_dev is device (HBM) memory owned by the
 *     caller.  The library never allocates device memory; scratch space is
 *     passed in as a workspace.
 *   - `stream` is a hipStream_t passed as void* (NULL = legacy default
 *     stream).  All work is enqueued asynchronously on it; nothing
 *     synchronises the host.
 *   - Return 0 on success, a negative lv_status on failure.  lv_last_error()
 *     returns a thread-local, NUL-terminated description of the last failure
 *     on the calling thread.  Argument checks happen on the host before any
 *     launch, so a failed call has enqueued nothing.
 *   - Entry points keep no mutable global state and are safe to call from
 *     any host thread (the reference runs engine steps on an executor thread,
 *     litevllm/entrypoints/async_llm.py:96-116).
 */
#ifndef LITEVLLM_HIP_H
#define LITEVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of logits / q / k / v / caches. */
typedef enum lv_dtype {
  LV_F32 = 0,
  LV_F16 = 1,
  LV_BF16 = 2
} lv_dtype;

typedef enum lv_status {
  LV_OK = 0,
  LV_ERR_INVALID = -1,     /* bad shape, stride, alignment or pointer */
  LV_ERR_HIP = -2,         /* a HIP runtime call or launch failed */
  LV_ERR_WORKSPACE = -3,   /* workspace missing or too small */
  LV_ERR_UNSUPPORTED = -4, /* valid request this build has no kernel for */
  LV_ERR_DEVICE_INDEX = -5 /* lv_device_errors: a kernel met an out-of-range index */
} lv_status;

/* Thread-local description of the last error on this thread ("" if none). */
const char* lv_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int lv_abi_version(void);
#define LV_ABI_VERSION 7

/* Out-of-range indices met by the kernels on the current device.
 *
 * The reference's torch indexing raises on an index outside its tensor
 * (litevllm/layers/attention.py:80-84 slot_mapping into the caches,
 * 111-119 block_table into the caches).  The kernels here never access
 * memory outside a buffer: they clamp such an index (a block id outside
 * [0, num_cache_blocks) reads block 0; a slot >= num_blocks * block_size is
 * not written) and raise a bit in a device-side error word:
 *   LV_DEVERR_BLOCK_ID  a block-table entry outside [0, num_cache_blocks)
 *                       (lv_paged_attention, lv_paged_attention_prefix)
 *   LV_DEVERR_SLOT      a slot_mapping entry >= num_blocks * block_size
 *                       (lv_kv_scatter, lv_qk_norm_rope_cache)
 * Negative slots are padding (skipped, no bit).
 * lv_device_errors waits for the current device (hipDeviceSynchronize), so
 * every kernel enqueued before the call has reported, then stores the bits
 * raised since the last clear in *flags_out (may be NULL) and, if clear is
 * nonzero, resets them.  Returns LV_OK when no bit is set,
 * LV_ERR_DEVICE_INDEX (with lv_last_error naming the bits) when one is, or
 * LV_ERR_HIP.  The word is per device and per process, shared by every
 * stream: a clear races with kernels another thread enqueues meanwhile.
 */
#define LV_DEVERR_BLOCK_ID 1u
#define LV_DEVERR_SLOT 2u
int lv_device_errors(uint32_t* flags_out, int32_t clear);

/* ------------------------------------------------------------------------
 * (1) Ragged-batch packing.
 *
 * Replaces ModelRunner.prepare_inputs
 *   (reference litevllm/engine/model_runner.py:180-260, InputMetadata 84-103,
 *    Sequence.is_prefill / num_new_tokens engine/sequence.py:95-104,
 *    BlockTable.physical_block_ids cache/block_manager.py:76-77).
 *
 * One descriptor per scheduled sequence, in batch order.  For sequence i
 * with n = num_computed, q = query_len:
 *   tokens cu[i] .. cu[i]+q-1 of the packed batch get
 *     position  p = n + j                                (j = 0..q-1)
 *     input id  = token_ids[token_offset + j]            (token_index < 0)
 *               = device_tokens[token_index]             (token_index >= 0, q == 1)
 *     slot      = block_ids[block_offset + p / bs] * bs + p % bs
 *                 if p / bs < num_blocks, else 0          (model_runner.py:210-215)
 *   cu_seqlens[i] = sum of query_len over sequences < i, cu_seqlens[B] = T
 *   seq_start[i]  = n
 *   context_lens[i] = n + q
 *   block_tables[i, :] = block_ids[block_offset .. +num_blocks], padded
 *                        with 0 to max_blocks              (model_runner.py:243-247)
 * A reference decode sequence is n = total_len - 1, q = 1; a reference
 * prefill is n = num_computed_tokens, q = prompt_len - n.
 * num_seqs <= 8192.  The descriptors live in device memory, so the host
 * cannot check them: a descriptor that points outside block_ids /
 * token_ids / device_tokens (sizes given) yields 0 in the affected entries
 * instead of an out-of-bounds read.  Callers validate descriptors on the
 * host before uploading them.
 */
typedef struct lv_seq_desc {
  int32_t num_computed;  /* tokens of this sequence already in the KV cache */
  int32_t query_len;     /* tokens fed this step (>= 1)                      */
  int32_t num_blocks;    /* length of this sequence's block table           */
  int32_t block_offset;  /* start of its block table inside block_ids       */
  int32_t token_offset;  /* start of its input ids inside token_ids         */
  int32_t token_index;   /* >= 0: single input id read from device_tokens   */
} lv_seq_desc;

int lv_pack_inputs(const lv_seq_desc* descs_dev, int32_t num_seqs,
                   const int32_t* block_ids_dev,      /* flat block tables   */
                   int64_t num_block_ids,
                   const int64_t* token_ids_dev,      /* flat host-fed ids   */
                   int64_t num_token_ids,
                   const int64_t* device_tokens_dev,  /* may be NULL         */
                   int64_t num_device_tokens,
                   int64_t num_tokens,                /* T = sum query_len   */
                   int32_t block_size, int32_t max_blocks,
                   int64_t* input_ids_dev,            /* [T]                 */
                   int64_t* positions_dev,            /* [T]                 */
                   int64_t* slot_mapping_dev,         /* [T]                 */
                   int32_t* cu_seqlens_dev,           /* [B+1]               */
                   int32_t* seq_start_dev,            /* [B]                 */
                   int32_t* context_lens_dev,         /* [B]                 */
                   int32_t* block_tables_dev,         /* [B, max_blocks]     */
                   void* stream);

/* ------------------------------------------------------------------------
 * (2) KV-cache scatter keyed by slot_mapping.
 *
 * Replaces the inline scatter in Attention.forward
 *   (reference litevllm/layers/attention.py:79-84) and
 *   PagedAttention.write_to_cache (attention.py:17-33):
 *     key_cache[slot / bs, slot % bs, :, :] = key[t]   (same for value)
 * key/value: [T, num_kv_heads, head_dim] with token stride *_stride_t
 * (elements), heads contiguous.  Caches: contiguous
 * [num_blocks, block_size, num_kv_heads, head_dim].  Slots < 0 are skipped
 * (padding); slots >= num_blocks*block_size are skipped so no write leaves
 * the cache, and raise LV_DEVERR_SLOT (see lv_device_errors).  Duplicate slots in one call: last writer undefined (torch's
 * index_put is undefined there too).
 */
int lv_kv_scatter(const void* key_dev, int64_t key_stride_t,
                  const void* value_dev, int64_t value_stride_t,
                  void* key_cache_dev, void* value_cache_dev,
                  const int64_t* slot_mapping_dev, int64_t num_tokens,
                  int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                  int64_t num_blocks, lv_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * (3) Paged attention over a mixed batch.
 *
 * Replaces Attention._decode_fast (reference litevllm/layers/attention.py:
 * 91-139) for 1-token decodes and Attention._prefill (attention.py:141-151)
 * for prefill chunks, extended to chunks that start at an offset and read
 * the cached prefix from the paged cache.
 *
 * Sequence i owns query rows cu_seqlens[i] .. cu_seqlens[i+1]-1 and has
 * context_lens[i] tokens in the cache (including this step's tokens, which
 * must already be scattered).  Query row j of sequence i sits at position
 * p = context_lens[i] - q_i + j and attends keys 0..p (causal; for a decode
 * this is the reference mask pos < context_len, attention.py:132).  Query
 * head h reads kv head h / (num_heads / num_kv_heads) (attention.py:124).
 * Softmax is taken in fp32 of (q.k) * scale; out is written in `dtype`.
 *
 * The first num_decodes sequences must have exactly one query row each
 * (decode); the rest are prefill chunks of any length <= max_query_len.
 * cu_seqlens_dev may be NULL when num_decodes == num_seqs (row i = seq i).
 * query: [T, num_heads, head_dim], token stride q_stride_t; out likewise
 * with out_stride_t.  Caches as in lv_kv_scatter.  block_tables:
 * [num_seqs, max_blocks] int32.
 * num_cache_blocks bounds every block id read from block_tables (an id
 * outside [0, num_cache_blocks) reads block 0 instead of faulting and raises
 * LV_DEVERR_BLOCK_ID, see lv_device_errors); context lengths are clamped to
 * max_blocks * block_size.
 * workspace: at least lv_paged_attention_workspace_size(...) bytes, 256-B
 * aligned; contents need not be initialised.  Calls that overlap on one
 * workspace race (use one workspace per stream).
 * Supported: head_dim 64 or 128, block_size 16, num_heads / num_kv_heads in
 * {1, 2, 4, 8}; anything else returns LV_ERR_UNSUPPORTED.  Decode rows run on
 * the persistent kernel (num_kv_heads <= 8, num_decodes <= 15000), which
 * indexes its flattened block list in 32 bits: there num_decodes *
 * max_blocks above 2^31 - 2^16 returns LV_ERR_INVALID (the row kernel,
 * LV_ATTN_DECODE_KERNEL=rows, has no such limit).
 */
size_t lv_paged_attention_workspace_size(int32_t num_seqs, int32_t num_decodes,
                                         int64_t num_tokens, int32_t num_heads,
                                         int32_t head_dim, int32_t block_size,
                                         int32_t max_blocks, int32_t max_query_len,
                                         lv_dtype dtype);

int lv_paged_attention(const void* query_dev, int64_t q_stride_t,
                       const void* key_cache_dev, const void* value_cache_dev,
                       int64_t num_cache_blocks,
                       const int32_t* block_tables_dev, int32_t max_blocks,
                       const int32_t* cu_seqlens_dev,
                       const int32_t* context_lens_dev,
                       int32_t num_seqs, int32_t num_decodes, int64_t num_tokens,
                       int32_t max_query_len,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t block_size, float scale,
                       void* out_dev, int64_t out_stride_t,
                       void* workspace_dev, size_t workspace_bytes,
                       lv_dtype dtype, void* stream);

/* Shared-prefix (cascade) variant of lv_paged_attention for the decode rows.
 *
 * Replaces the same reference code as lv_paged_attention (attention.py:
 * 91-139); the reference has no shared-prefix pass: every decode row reads
 * its whole context.  Here decode rows whose block tables start with the
 * same physical blocks (a prefix-cache hit on a common prompt) form a group;
 * the group's prefix keys are read once for all its members (MFMA kernel,
 * members as the query rows), each row's remaining blocks are walked as in
 * lv_paged_attention, and the two softmax partials are merged.  Results
 * equal lv_paged_attention's to fp32 rounding.
 *
 * prefix_blocks: int32 [num_decodes], leading blocks of row i attended by
 * the prefix pass (0 = none); for a member of a group it is the group's
 * prefix length, at most 128 blocks, and prefix_blocks[i] * block_size <=
 * context_lens[i].  prefix_members: int32 [num_members], the member rows of
 * each group listed together.  prefix_items: int32 [max_items][4], 16-byte
 * aligned (may be NULL when max_items is 0): one work item per (group,
 * slice of up to 128 / G members, 128-key split of the prefix): {leader row, index of the slice's first member in
 * prefix_members, members in the slice, split}; leader row < 0 marks an
 * unused item.  Every member's prefix rows must be covered by exactly one
 * item per split, and the first prefix_blocks[leader] entries of every
 * member's block table must equal the leader's (the pass reads the
 * leader's table).  Items are skipped when their leader is outside
 * [0, num_decodes), their split outside [0, 16), their slice empty, wider
 * than 128 / G members or outside prefix_members [0, num_members); member
 * rows outside [0, num_decodes) are skipped.  (litevllm.ops.
 * prefix_plan_arrays builds and checks such arrays on the host.)
 * prefix_workspace: at least lv_paged_attention_prefix_workspace_size(...)
 * bytes, 256-B aligned, contents need not be initialised; one per stream.
 * Supported: bf16 / fp16, head_dim 64 / 128, block_size 16, G in
 * {1, 2, 4, 8}, at most 8 kv heads, 1 <= num_decodes <= 7000 (else
 * LV_ERR_UNSUPPORTED).  Prefill-chunk rows (num_decodes < num_seqs) are
 * handled exactly as by lv_paged_attention.
 */
size_t lv_paged_attention_prefix_workspace_size(int32_t num_decodes, int32_t num_heads,
                                                int32_t head_dim);

int lv_paged_attention_prefix(const void* query_dev, int64_t q_stride_t,
                              const void* key_cache_dev, const void* value_cache_dev,
                              int64_t num_cache_blocks,
                              const int32_t* block_tables_dev, int32_t max_blocks,
                              const int32_t* cu_seqlens_dev,
                              const int32_t* context_lens_dev,
                              int32_t num_seqs, int32_t num_decodes, int64_t num_tokens,
                              int32_t max_query_len,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, float scale,
                              void* out_dev, int64_t out_stride_t,
                              void* workspace_dev, size_t workspace_bytes,
                              const int32_t* prefix_blocks_dev,
                              const int32_t* prefix_items_dev, int32_t max_items,
                              const int32_t* prefix_members_dev, int32_t num_members,
                              void* prefix_workspace_dev, size_t prefix_workspace_bytes,
                              lv_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * (4) Fused greedy / temperature sampler.
 *
 * Replaces Sampler.sample's greedy branch (_triton_argmax / _argmax_kernel,
 * reference litevllm/layers/sampler.py:60-84, 111-124, 175-176) and its
 * temperature branch without top-k/top-p (_triton_softmax_temp +
 * torch.multinomial, sampler.py:86-108, 127-144, 177-187).
 *
 * Row r of logits [B, V] (row stride row_stride elements):
 *   temperature[r] == 0 : out[r] = first index of the fp32 maximum.
 *   temperature[r] >  0 : out[r] = inverse-CDF draw of softmax(x / T) at the
 *                         caller-supplied uniform[r] in [0, 1), with the
 *                         fixed-order fp32 arithmetic defined in sampler.hip
 *                         (bit-reproducible; the CPU restatement matches it
 *                         bit for bit).
 * temperature_dev / uniform_dev: fp32 [B] (uniform is read only for rows with
 * temperature > 0; pass zeros when every row is greedy).  out_ids_dev:
 * int64 [B].  workspace: device scratch of at least
 * lv_sample_workspace_size(num_rows, vocab_size) bytes (no initialisation
 * needed; calls that overlap on one workspace race: use one per stream).
 * Two kernels are enqueued on `stream`.
 */
size_t lv_sample_workspace_size(int64_t num_rows, int64_t vocab_size);

int lv_sample(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
              int64_t row_stride, const float* temperature_dev,
              const float* uniform_dev, int64_t* out_ids_dev, void* workspace_dev,
              size_t workspace_bytes, lv_dtype dtype, void* stream);

/* lv_sample without a workspace argument: it allocates nothing (no
 * hipMalloc / hipFree, no allocating library call).  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it).
 * Arguments, results and errors are those of lv_sample.  Its scratch is a
 * fixed 4 MiB array in the library's device code, one copy per GPU, looked
 * up (hipGetSymbolAddress) on the first call on each device -- make that
 * first call outside any stream capture (a warm-up call), so the lookup is
 * not made while a graph is being recorded; calls needing more than
 * lv_sample_workspace_size(num_rows, vocab_size) <= 4 MiB (e.g. above 1765
 * rows at vocab 151936) are rejected with LV_ERR_WORKSPACE.  Every call on a
 * GPU uses that GPU's one copy: calls that overlap on one GPU (two streams,
 * two threads) race.
 */
int lv_sample_noalloc(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
                      int64_t row_stride, const float* temperature_dev,
                      const float* uniform_dev, int64_t* out_ids_dev, lv_dtype dtype,
                      void* stream);

/* ------------------------------------------------------------------------
 * Fused layer prologue / epilogue work (the elementwise ops the reference
 * runs as separate torch ops around its GEMMs).  Rounding follows the
 * reference op by op: each intermediate the reference materialises in the
 * model dtype is rounded to that dtype.  The fp32 sum of squares is reduced
 * in a different order than torch's, so results agree within 1-2 ulp of the
 * dtype, not bit for bit.
 * ---------------------------------------------------------------------- */

/* Residual add + RMSNorm.  Replaces LlamaRMSNorm.forward
 * (litevllm/models/llama.py:24-27) together with the residual adds of the
 * decoder layer (models/qwen3.py:131-140, llama.py:133-142):
 *   if residual != NULL:  residual[t] = x[t] + residual[t];  src = residual[t]
 *   else                  src = x[t]
 *   out[t] = weight * to_dtype(src * rsqrt(mean(src^2) + eps))
 * Rows are [num_tokens, hidden] with the given element strides; every row
 * must start on a 16-byte boundary and hidden must be a multiple of 16 bytes
 * worth of elements.  out may not alias x or residual. */
int lv_add_rms_norm(const void* x_dev, int64_t x_stride_t, void* residual_dev,
                    int64_t residual_stride_t, const void* weight_dev, void* out_dev,
                    int64_t out_stride_t, int64_t num_tokens, int32_t hidden, float eps,
                    lv_dtype dtype, void* stream);

/* Attention prologue of one layer.  Replaces, for a fused q|k|v projection
 * row qkv[t] = [q (H*D) | k (Hkv*D) | v (Hkv*D)], the sequence
 * q_norm/k_norm (models/qwen3.py:75-77; pass NULL weights for Llama),
 * rotary_emb + apply_rotary_emb (layers/rotary_emb.py:92-117, with the
 * module's cos/sin caches, [max_position, D/2] in the model dtype) and the
 * K/V cache write (layers/attention.py:79-84, PagedAttention.write_to_cache
 * attention.py:17-33):
 *   q_out[t, h]                     = rope(norm_q(q[t, h]), positions[t])
 *   key_cache  row slot_mapping[t]  = rope(norm_k(k[t]), positions[t])
 *   value_cache row slot_mapping[t] = v[t]
 * Tokens with slot < 0 (padding) or slot >= num_blocks*block_size write no
 * cache row (the latter raise LV_DEVERR_SLOT, see lv_device_errors); a
 * position outside [0, max_position) yields NaN rows.
 * head_dim in {64, 128, 256}. */
int lv_qk_norm_rope_cache(const void* qkv_dev, int64_t qkv_stride_t,
                          const void* q_norm_weight_dev, const void* k_norm_weight_dev,
                          const void* cos_dev, const void* sin_dev, int64_t max_position,
                          const int64_t* positions_dev, const int64_t* slot_mapping_dev,
                          void* q_out_dev, int64_t q_out_stride_t, void* key_cache_dev,
                          void* value_cache_dev, int64_t num_blocks, int32_t block_size,
                          int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, float eps, lv_dtype dtype, void* stream);

/* Gated-MLP activation.  Replaces F.silu(gate) * up of LlamaMLP.forward
 * (models/llama.py:37-38) for a fused gate|up row:
 *   out[t, i] = to_dtype(silu(gate_up[t, i])) * gate_up[t, intermediate + i]
 * Rows 16-byte aligned; intermediate a multiple of 16 bytes of elements. */
int lv_silu_mul(const void* gate_up_dev, int64_t in_stride_t, void* out_dev,
                int64_t out_stride_t, int64_t num_tokens, int32_t intermediate,
                lv_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * Linear layers of decode-sized batches (MFMA, weight-streaming tiles).
 *
 * Replaces nn.Linear without bias -- ColumnParallelLinear /
 * RowParallelLinear (reference litevllm/layers/linear.py:15-65) as used for
 * the q/k/v, o, gate/up and down projections (models/qwen3.py:45-48,
 * models/llama.py:33-35, 58-61) of decode steps -- and, with
 * LV_ACT_SILU_MUL, the gated-MLP input of down_proj
 * F.silu(gate_proj(x)) * up_proj(x) (llama.py:38):
 *   LV_ACT_NONE      y[m, n] = to_dtype(sum_k x[m, k] * weight[n, k])
 *   LV_ACT_SILU_MUL  g, u = the same sums with weight rows n and N + n;
 *                    y[m, n] = to_dtype(to_dtype(silu(to_dtype(g))) * to_dtype(u))
 * fp32 accumulation; the k order of the sums is the same for both forms, so
 * the silu_mul form equals lv_silu_mul applied to the plain form's output
 * over the [2N, K] weight.  weight is [N, K] ([2N, K] for LV_ACT_SILU_MUL)
 * with row stride weight_stride_n; x [M, K] and y [M, N] with row strides in
 * elements; x/weight rows 16-byte aligned, y rows 8-byte aligned.  bf16/fp16
 * with N % 32 == 0 and K % 128 == 0 have a kernel (lv_linear_supported);
 * anything else returns LV_ERR_UNSUPPORTED and the caller uses a library
 * GEMM.  Meant for M up to a few hundred; larger M belong to the library
 * GEMM. */
typedef enum lv_activation {
  LV_ACT_NONE = 0,
  LV_ACT_SILU_MUL = 1
} lv_activation;

int lv_linear_supported(int64_t m, int64_t n, int64_t k, int32_t activation, lv_dtype dtype);

int lv_linear(const void* x_dev, int64_t x_stride_t, const void* weight_dev,
              int64_t weight_stride_n, void* y_dev, int64_t y_stride_t, int64_t m, int64_t n,
              int64_t k, int32_t activation, lv_dtype dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LITEVLLM_HIP_H */
