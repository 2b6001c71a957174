// Ragged-batch packing on the GPU: per-sequence descriptors -> the packed
// per-token arrays and padded block tables of one engine step.
//
// Semantics follow ModelRunner.prepare_inputs (reference
// litevllm/engine/model_runner.py:180-260): position = num_computed + j,
// slot = block_id[pos / bs] * bs + pos % bs or 0 past the table (210-215),
// block tables padded with 0 (243-247).  cu_seqlens / seq_start /
// context_lens for every sequence are additions the mixed-batch attention
// kernel consumes.
#include "lv_common.h"

namespace lv {

constexpr int kPackThreads = 256;
constexpr int kPackMaxSeqs = 8192;

// Exclusive scan of query_len into s_cu[0..n] by one workgroup (integer
// arithmetic, so any order gives the same result).
__device__ void scan_query_lens(const lv_seq_desc* __restrict__ descs, int n, int32_t* s_cu) {
  __shared__ int32_t s_part[kPackThreads];
  const int t = threadIdx.x;
  const int per = (n + kPackThreads - 1) / kPackThreads;
  const int lo = min(n, t * per);
  const int hi = min(n, lo + per);
  int32_t sum = 0;
  for (int i = lo; i < hi; ++i) sum += descs[i].query_len;
  s_part[t] = sum;
  __syncthreads();
  // Hillis-Steele over the 256 partial sums.
  for (int d = 1; d < kPackThreads; d <<= 1) {
    int32_t v = (t >= d) ? s_part[t - d] : 0;
    __syncthreads();
    s_part[t] += v;
    __syncthreads();
  }
  int32_t run = (t == 0) ? 0 : s_part[t - 1];
  for (int i = lo; i < hi; ++i) {
    s_cu[i] = run;
    run += descs[i].query_len;
  }
  if (t == kPackThreads - 1) s_cu[n] = s_part[kPackThreads - 1];
  __syncthreads();
}

__global__ __launch_bounds__(kPackThreads) void pack_kernel(
    const lv_seq_desc* __restrict__ descs, int num_seqs,
    const int32_t* __restrict__ block_ids, int64_t num_block_ids,
    const int64_t* __restrict__ token_ids, int64_t num_token_ids,
    const int64_t* __restrict__ device_tokens, int64_t num_device_tokens,
    int64_t num_tokens, int block_size, int max_blocks,
    int64_t* __restrict__ input_ids, int64_t* __restrict__ positions,
    int64_t* __restrict__ slot_mapping, int32_t* __restrict__ cu_seqlens,
    int32_t* __restrict__ seq_start, int32_t* __restrict__ context_lens,
    int32_t* __restrict__ block_tables) {
  extern __shared__ int32_t s_cu[];  // num_seqs + 1 entries
  scan_query_lens(descs, num_seqs, s_cu);

  const int64_t n_table = (int64_t)num_seqs * max_blocks;
  const int64_t n_work = num_tokens + n_table + num_seqs + 1;
  for (int64_t idx = (int64_t)blockIdx.x * kPackThreads + threadIdx.x; idx < n_work;
       idx += (int64_t)gridDim.x * kPackThreads) {
    if (idx < num_tokens) {
      // Sequence owning packed token idx: largest i with s_cu[i] <= idx.
      int lo = 0, hi = num_seqs - 1;
      while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (s_cu[mid] <= idx) lo = mid; else hi = mid - 1;
      }
      const lv_seq_desc d = descs[lo];
      const int64_t j = idx - s_cu[lo];
      int64_t tok = 0, pos = 0, slot = 0;
      if (j < d.query_len) {
        pos = (int64_t)d.num_computed + j;
        if (d.token_index >= 0) {
          if (d.token_index < num_device_tokens && device_tokens != nullptr)
            tok = device_tokens[d.token_index];
        } else {
          const int64_t ti = (int64_t)d.token_offset + j;
          if (ti >= 0 && ti < num_token_ids) tok = token_ids[ti];
        }
        const int64_t bi = pos / block_size;
        const int64_t src = (int64_t)d.block_offset + bi;
        if (bi < d.num_blocks && src >= 0 && src < num_block_ids)
          slot = (int64_t)block_ids[src] * block_size + pos % block_size;
      }
      input_ids[idx] = tok;
      positions[idx] = pos;
      slot_mapping[idx] = slot;
    } else if (idx < num_tokens + n_table) {
      const int64_t e = idx - num_tokens;
      const int i = (int)(e / max_blocks);
      const int c = (int)(e % max_blocks);
      const lv_seq_desc d = descs[i];
      const int64_t src = (int64_t)d.block_offset + c;
      int32_t v = 0;
      if (c < d.num_blocks && src >= 0 && src < num_block_ids) v = block_ids[src];
      block_tables[e] = v;
    } else {
      const int i = (int)(idx - num_tokens - n_table);
      if (i < num_seqs) {
        const lv_seq_desc d = descs[i];
        seq_start[i] = d.num_computed;
        context_lens[i] = d.num_computed + d.query_len;
      }
      cu_seqlens[i] = s_cu[i];
    }
  }
}

}  // namespace lv

extern "C" int lv_pack_inputs(const lv_seq_desc* descs_dev, int32_t num_seqs,
                              const int32_t* block_ids_dev, int64_t num_block_ids,
                              const int64_t* token_ids_dev, int64_t num_token_ids,
                              const int64_t* device_tokens_dev, int64_t num_device_tokens,
                              int64_t num_tokens, int32_t block_size, int32_t max_blocks,
                              int64_t* input_ids_dev, int64_t* positions_dev,
                              int64_t* slot_mapping_dev, int32_t* cu_seqlens_dev,
                              int32_t* seq_start_dev, int32_t* context_lens_dev,
                              int32_t* block_tables_dev, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(num_seqs >= 1 && num_seqs <= kPackMaxSeqs,
             "lv_pack_inputs: num_seqs=%d outside [1, %d]", num_seqs, kPackMaxSeqs);
  LV_REQUIRE(num_tokens >= num_seqs && num_tokens < (1ll << 31),
             "lv_pack_inputs: num_tokens=%lld must be in [num_seqs, 2^31)", (long long)num_tokens);
  LV_REQUIRE(block_size > 0 && max_blocks >= 0, "lv_pack_inputs: bad block_size/max_blocks");
  LV_REQUIRE(descs_dev && input_ids_dev && positions_dev && slot_mapping_dev && cu_seqlens_dev &&
                 seq_start_dev && context_lens_dev,
             "lv_pack_inputs: null required pointer");
  LV_REQUIRE(max_blocks == 0 || block_tables_dev, "lv_pack_inputs: null block_tables");
  LV_REQUIRE(num_block_ids == 0 || block_ids_dev, "lv_pack_inputs: null block_ids");
  LV_REQUIRE(num_token_ids == 0 || token_ids_dev, "lv_pack_inputs: null token_ids");
  const int64_t n_work = num_tokens + (int64_t)num_seqs * max_blocks + num_seqs + 1;
  int grid = (int)((n_work + kPackThreads - 1) / kPackThreads);
  if (grid > 2048) grid = 2048;
  const size_t lds = sizeof(int32_t) * (size_t)(num_seqs + 1);
  hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(kPackThreads), lds, (hipStream_t)stream,
                     descs_dev, num_seqs, block_ids_dev, num_block_ids, token_ids_dev,
                     num_token_ids, device_tokens_dev, num_device_tokens, num_tokens, block_size,
                     max_blocks, input_ids_dev, positions_dev, slot_mapping_dev, cu_seqlens_dev,
                     seq_start_dev, context_lens_dev, block_tables_dev);
  return check_launch("lv_pack_inputs");
}
