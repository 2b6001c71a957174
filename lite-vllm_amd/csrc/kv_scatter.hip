// KV-cache scatter: key_cache[slot / bs, slot % bs] = key[t] (and value).
//
// Follows the inline scatter of Attention.forward (reference
// litevllm/layers/attention.py:79-84) and PagedAttention.write_to_cache
// (attention.py:17-33).  The cache is contiguous [N, bs, Hkv, D], so cache
// row `slot` starts at slot * Hkv * D elements: the copy is a pure byte move
// of one Hkv*D row per token, independent of the element type.
#include "lv_common.h"

namespace lv {

constexpr int kScatterThreads = 256;  // 4 wavefronts, one token per wavefront

template <typename Chunk>
__global__ __launch_bounds__(kScatterThreads) void kv_scatter_kernel(
    const char* __restrict__ key, int64_t key_stride_bytes,
    const char* __restrict__ value, int64_t value_stride_bytes,
    char* __restrict__ key_cache, char* __restrict__ value_cache,
    const int64_t* __restrict__ slots, int64_t num_tokens, int row_chunks, int64_t num_slots) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (kScatterThreads / 64) + wave;
  if (t >= num_tokens) return;
  const int64_t slot = slots[t];
  if (slot < 0) return;                      // padding
  if (slot >= num_slots) {                   // outside the cache: not written, reported
    if (lane == 0) report_device_error(LV_DEVERR_SLOT);
    return;
  }
  const Chunk* ks = reinterpret_cast<const Chunk*>(key + t * key_stride_bytes);
  const Chunk* vs = reinterpret_cast<const Chunk*>(value + t * value_stride_bytes);
  Chunk* kd = reinterpret_cast<Chunk*>(key_cache) + slot * row_chunks;
  Chunk* vd = reinterpret_cast<Chunk*>(value_cache) + slot * row_chunks;
  for (int c = lane; c < row_chunks; c += 64) {
    const Chunk kv = ks[c];
    const Chunk vv = vs[c];
    kd[c] = kv;
    vd[c] = vv;
  }
}

LV_ERROR_WORD_READER(read_errors_scatter)

}  // namespace lv

extern "C" int lv_kv_scatter(const void* key_dev, int64_t key_stride_t, const void* value_dev,
                             int64_t value_stride_t, void* key_cache_dev, void* value_cache_dev,
                             const int64_t* slot_mapping_dev, int64_t num_tokens,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int64_t num_blocks, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16, "lv_kv_scatter: bad dtype");
  LV_REQUIRE(num_tokens >= 0, "lv_kv_scatter: negative num_tokens");
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(num_kv_heads > 0 && head_dim > 0 && block_size > 0 && num_blocks > 0,
             "lv_kv_scatter: bad cache geometry");
  LV_REQUIRE(key_dev && value_dev && key_cache_dev && value_cache_dev && slot_mapping_dev,
             "lv_kv_scatter: null pointer");
  const int64_t esize = (int64_t)dtype_size(dtype);
  const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
  LV_REQUIRE(key_stride_t >= row_elems && value_stride_t >= row_elems,
             "lv_kv_scatter: token stride smaller than num_kv_heads*head_dim");
  const int64_t row_bytes = row_elems * esize;
  const int64_t ks = key_stride_t * esize, vs = value_stride_t * esize;
  const int64_t num_slots = num_blocks * block_size;
  const int grid = (int)((num_tokens + 3) / 4);
  auto ok_for = [&](int64_t w) {
    const uintptr_t m = (uintptr_t)(w - 1);
    return (row_bytes % w) == 0 && (ks % w) == 0 && (vs % w) == 0 &&
           ((uintptr_t)key_dev & m) == 0 && ((uintptr_t)value_dev & m) == 0 &&
           ((uintptr_t)key_cache_dev & m) == 0 && ((uintptr_t)value_cache_dev & m) == 0;
  };
  hipStream_t st = (hipStream_t)stream;
  if (ok_for(16)) {
    hipLaunchKernelGGL(kv_scatter_kernel<uint4>, dim3(grid), dim3(kScatterThreads), 0, st,
                       (const char*)key_dev, ks, (const char*)value_dev, vs, (char*)key_cache_dev,
                       (char*)value_cache_dev, slot_mapping_dev, num_tokens, (int)(row_bytes / 16),
                       num_slots);
  } else if (ok_for(4)) {
    hipLaunchKernelGGL(kv_scatter_kernel<uint32_t>, dim3(grid), dim3(kScatterThreads), 0, st,
                       (const char*)key_dev, ks, (const char*)value_dev, vs, (char*)key_cache_dev,
                       (char*)value_cache_dev, slot_mapping_dev, num_tokens, (int)(row_bytes / 4),
                       num_slots);
  } else {
    LV_REQUIRE(ok_for(2), "lv_kv_scatter: pointers/strides not 2-byte aligned");
    hipLaunchKernelGGL(kv_scatter_kernel<uint16_t>, dim3(grid), dim3(kScatterThreads), 0, st,
                       (const char*)key_dev, ks, (const char*)value_dev, vs, (char*)key_cache_dev,
                       (char*)value_cache_dev, slot_mapping_dev, num_tokens, (int)(row_bytes / 2),
                       num_slots);
  }
  return check_launch("lv_kv_scatter");
}
