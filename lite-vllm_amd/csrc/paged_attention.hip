// Paged attention for a mixed batch of 1-token decodes and prefill chunks.
//
// Decode rows follow Attention._decode_fast (reference
// litevllm/layers/attention.py:91-139): scores (q.k) * scale over the
// positions < context_len of the sequence's block table (mask at 132-133),
// GQA head map h -> h / G (124), fp32 softmax (135), P.V (138).  Prefill
// chunk rows generalise Attention._prefill (attention.py:141-151) to a chunk
// at any offset: query position p attends keys 0..p read from the paged
// cache.
//
// attn_rows_kernel: one workgroup (4 wavefronts) per (query row, kv head,
// context partition).  A wavefront streams whole 16-token blocks with
// 16-byte loads: lane = (token-in-load tg, dim chunk dc), ROW_LANES lanes
// cover one token's head_dim, so one load instruction fetches TPL tokens.
// Both query heads of the GQA group are computed from the same K/V
// registers.  Each token group keeps its own online-softmax state (max, sum,
// accumulator) in fp32 and the states are merged at the end (in-wave
// shuffles, then LDS across wavefronts).  Long contexts are split into
// partitions whose normalised partial outputs and (max, sum) pairs go to the
// workspace and are merged by attn_reduce_kernel.
#include <stdlib.h>

#include "lv_common.h"

namespace lv {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr float kNegBig = -1.0e30f;

template <typename T, int D, int BS>
struct RowCfg {
  static constexpr int VEC = elem<T>::kPer16B;
  static constexpr int ROW_LANES = D / VEC;
  static constexpr int TPL = 64 / ROW_LANES;
  static constexpr int LOADS = BS / TPL;
  static_assert(ROW_LANES >= 1 && ROW_LANES <= 64 && 64 % ROW_LANES == 0, "row lanes");
  static_assert(BS % TPL == 0, "block size must be a multiple of tokens per load");
};

// Query row -> (sequence, causal key limit).  Without cu_seqlens every row
// is its own 1-token sequence.
__device__ __forceinline__ void resolve_row(int row, const int32_t* __restrict__ cu, int num_seqs,
                                            const int32_t* __restrict__ ctx, int max_tokens,
                                            int& seq, int& limit) {
  if (cu == nullptr) {
    seq = row;
    limit = ctx[row];
  } else {
    int lo = 0, hi = num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cu[mid] <= row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    const int q = cu[lo + 1] - cu[lo];
    limit = ctx[lo] - q + (row - cu[lo]) + 1;
  }
  limit = min(limit, max_tokens);
}

template <typename T, int D, int G, int BS>
__global__ __launch_bounds__(kAttnThreads) void attn_rows_kernel(
    const T* __restrict__ q, int64_t q_stride,
    const T* __restrict__ kc, const T* __restrict__ vc, int num_kv_heads, int64_t num_cache_blocks,
    const int32_t* __restrict__ block_tables, int max_blocks,
    const int32_t* __restrict__ cu, int num_seqs, const int32_t* __restrict__ ctx,
    int row_begin, int part_tokens, int max_parts, float scale_log2,
    T* __restrict__ out, int64_t out_stride,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml) {
  using C = RowCfg<T, D, BS>;
  constexpr int VEC = C::VEC, RL = C::ROW_LANES, TPL = C::TPL, LOADS = C::LOADS;
  __shared__ float s_acc[kAttnWaves][G][D];
  __shared__ float s_m[kAttnWaves][G];
  __shared__ float s_l[kAttnWaves][G];

  const int row = row_begin + (int)blockIdx.x;
  const int kvh = blockIdx.y;
  const int part = blockIdx.z;
  int seq, limit;
  resolve_row(row, cu, num_seqs, ctx, max_blocks * BS, seq, limit);
  const int start = part * part_tokens;
  if (start >= limit) return;
  const int end = min(limit, start + part_tokens);
  const int nparts = (limit + part_tokens - 1) / part_tokens;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int tg = lane / RL;
  const int dc = lane % RL;

  float qv[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const T* qp = q + (int64_t)row * q_stride + (int64_t)(kvh * G + g) * D + dc * VEC;
    elem<T>::unpack(load16(qp), qv[g]);
#pragma unroll
    for (int j = 0; j < VEC; ++j) qv[g][j] *= scale_log2;
  }

  float m[G], l[G], acc[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[g][j] = 0.0f;
  }

  const int64_t tok_stride = (int64_t)num_kv_heads * D;
  const int64_t blk_stride = (int64_t)BS * tok_stride;
  const int64_t lane_off = (int64_t)kvh * D + dc * VEC + tg * tok_stride;
  const int32_t* __restrict__ bt = block_tables + (int64_t)seq * max_blocks;
  const int b_begin = start / BS;
  const int b_end = (end + BS - 1) / BS;

  auto load_block = [&](int b, uint4* kk, uint4* vv) {
    int64_t phys = bt[b];
    if (phys < 0 || phys >= num_cache_blocks) phys = 0;
    const T* kp = kc + phys * blk_stride + lane_off;
    const T* vp = vc + phys * blk_stride + lane_off;
#pragma unroll
    for (int r = 0; r < LOADS; ++r) kk[r] = load16(kp + (int64_t)r * TPL * tok_stride);
#pragma unroll
    for (int r = 0; r < LOADS; ++r) vv[r] = load16(vp + (int64_t)r * TPL * tok_stride);
  };

  uint4 kr[LOADS], vr[LOADS];
  int blk = b_begin + wave;
  if (blk < b_end) load_block(blk, kr, vr);
  for (; blk < b_end; blk += kAttnWaves) {
    uint4 kn[LOADS], vn[LOADS];
    const int nb = blk + kAttnWaves;
    if (nb < b_end) load_block(nb, kn, vn);

    float s[G][LOADS];
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      float kf[VEC];
      elem<T>::unpack(kr[r], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < VEC; ++j) d = fmaf(qv[g][j], kf[j], d);
        s[g][r] = group_sum<RL>(d);
      }
    }
    const int pos0 = blk * BS + tg;
    const bool tail = (blk + 1) * BS > end;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = m[g];
#pragma unroll
      for (int r = 0; r < LOADS; ++r)
        if (!tail || pos0 + r * TPL < end) mx = fmaxf(mx, s[g][r]);
      const float alpha = fast_exp2(m[g] - mx);
      m[g] = mx;
      float lsum = l[g] * alpha;
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[g][j] *= alpha;
#pragma unroll
      for (int r = 0; r < LOADS; ++r) {
        const bool valid = !tail || pos0 + r * TPL < end;
        const float p = valid ? fast_exp2(s[g][r] - mx) : 0.0f;
        s[g][r] = p;
        lsum += p;
      }
      l[g] = lsum;
    }
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      float vf[VEC];
      elem<T>::unpack(vr[r], vf);
      if (tail && pos0 + r * TPL >= end) {
        // Slots past the context may hold anything (even NaN); 0 * NaN
        // would poison the accumulator, so drop them explicitly.
#pragma unroll
        for (int j = 0; j < VEC; ++j) vf[j] = 0.0f;
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[g][j] = fmaf(s[g][r], vf[j], acc[g][j]);
    }
    if (nb < b_end) {
#pragma unroll
      for (int r = 0; r < LOADS; ++r) { kr[r] = kn[r]; vr[r] = vn[r]; }
    }
  }

  // Merge the TPL token groups of this wavefront.
#pragma unroll
  for (int ofs = RL; ofs < 64; ofs <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], ofs);
      const float lo = __shfl_xor(l[g], ofs);
      const float mn = fmaxf(m[g], mo);
      const float fa = fast_exp2(m[g] - mn), fb = fast_exp2(mo - mn);
      l[g] = l[g] * fa + lo * fb;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float ao = __shfl_xor(acc[g][j], ofs);
        acc[g][j] = acc[g][j] * fa + ao * fb;
      }
      m[g] = mn;
    }
  }
  if (tg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) s_acc[wave][g][dc * VEC + j] = acc[g][j];
      if (dc == 0) { s_m[wave][g] = m[g]; s_l[wave][g] = l[g]; }
    }
  }
  __syncthreads();

  const int H = num_kv_heads * G;
  for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
    const int g = t / D, d = t % D;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float f = fast_exp2(s_m[w][g] - M);
      L = fmaf(s_l[w][g], f, L);
      O = fmaf(s_acc[w][g][d], f, O);
    }
    const float o = L > 0.0f ? O / L : 0.0f;
    const int hq = kvh * G + g;
    if (nparts == 1) {
      elem<T>::store(out + (int64_t)row * out_stride + (int64_t)hq * D + d, o);
    } else {
      const int64_t base = ((int64_t)(row - row_begin) * H + hq) * max_parts + part;
      ws_acc[base * D + d] = o;
      if (d == 0) { ws_ml[base * 2] = M; ws_ml[base * 2 + 1] = L; }
    }
  }
}

// Merge the partitions of one (row, query head); rows with a single
// partition were finished by attn_rows_kernel.
template <typename T, int D, int BS>
__global__ __launch_bounds__(D) void attn_reduce_kernel(
    const int32_t* __restrict__ cu, int num_seqs, const int32_t* __restrict__ ctx, int max_blocks,
    int row_begin, int part_tokens, int max_parts, int num_heads,
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    T* __restrict__ out, int64_t out_stride) {
  const int row = row_begin + (int)blockIdx.x;
  const int hq = blockIdx.y;
  const int d = threadIdx.x;
  int seq, limit;
  resolve_row(row, cu, num_seqs, ctx, max_blocks * BS, seq, limit);
  const int nparts = (limit + part_tokens - 1) / part_tokens;
  if (nparts <= 1) return;
  const int64_t base = ((int64_t)blockIdx.x * num_heads + hq) * max_parts;
  float M = kNegBig;
  for (int p = 0; p < nparts; ++p) M = fmaxf(M, ws_ml[(base + p) * 2]);
  float L = 0.0f, O = 0.0f;
  for (int p = 0; p < nparts; ++p) {
    const float f = ws_ml[(base + p) * 2 + 1] * fast_exp2(ws_ml[(base + p) * 2] - M);
    L += f;
    O = fmaf(ws_acc[(base + p) * D + d], f, O);
  }
  elem<T>::store(out + (int64_t)row * out_stride + (int64_t)hq * D + d, L > 0.0f ? O / L : 0.0f);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

// Context partition length (tokens) for split-K decode: a multiple of
// 4 * block_size so each wavefront gets whole blocks.
static int decode_part_tokens(int block_size) {
  int pt = 256;
  if (const char* e = getenv("LV_ATTN_PART_TOKENS")) {
    const int v = atoi(e);
    if (v > 0) pt = v;
  }
  const int unit = kAttnWaves * block_size;
  pt = ((pt + unit - 1) / unit) * unit;
  return pt;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct AttnPlan {
  int part_tokens;
  int max_parts;
  size_t acc_bytes, ml_bytes;
};

static AttnPlan plan_decode(int num_decodes, int num_heads, int head_dim, int block_size,
                            int max_blocks) {
  AttnPlan p;
  const int max_tokens = max_blocks * block_size;
  p.part_tokens = decode_part_tokens(block_size);
  p.max_parts = max_tokens > 0 ? (max_tokens + p.part_tokens - 1) / p.part_tokens : 1;
  if (p.max_parts <= 1) {
    p.max_parts = 1;
    p.acc_bytes = p.ml_bytes = 0;
  } else {
    const size_t n = (size_t)num_decodes * num_heads * p.max_parts;
    p.acc_bytes = align256(n * head_dim * sizeof(float));
    p.ml_bytes = align256(n * 2 * sizeof(float));
  }
  return p;
}

template <typename T, int D, int G, int BS>
static void launch_rows(const void* q, int64_t q_stride, const void* kc, const void* vc,
                        int num_kv_heads, int64_t num_cache_blocks, const int32_t* bt,
                        int max_blocks, const int32_t* cu, int num_seqs, const int32_t* ctx,
                        int row_begin, int n_rows, int part_tokens, int max_parts,
                        float scale_log2, void* out, int64_t out_stride, float* ws_acc,
                        float* ws_ml, hipStream_t st) {
  const dim3 grid(n_rows, num_kv_heads, max_parts);
  hipLaunchKernelGGL((attn_rows_kernel<T, D, G, BS>), grid, dim3(kAttnThreads), 0, st,
                     (const T*)q, q_stride, (const T*)kc, (const T*)vc, num_kv_heads,
                     num_cache_blocks, bt, max_blocks, cu, num_seqs, ctx, row_begin, part_tokens,
                     max_parts, scale_log2, (T*)out, out_stride, ws_acc, ws_ml);
  if (max_parts > 1) {
    hipLaunchKernelGGL((attn_reduce_kernel<T, D, BS>), dim3(n_rows, num_kv_heads * G), dim3(D), 0,
                       st, cu, num_seqs, ctx, max_blocks, row_begin, part_tokens, max_parts,
                       num_kv_heads * G, (const float*)ws_acc, (const float*)ws_ml, (T*)out,
                       out_stride);
  }
}

template <typename T, int D, int BS>
static int dispatch_g(int G, const void* q, int64_t q_stride, const void* kc, const void* vc,
                      int num_kv_heads, int64_t num_cache_blocks, const int32_t* bt, int max_blocks,
                      const int32_t* cu, int num_seqs, const int32_t* ctx, int row_begin,
                      int n_rows, int part_tokens, int max_parts, float scale_log2, void* out,
                      int64_t out_stride, float* ws_acc, float* ws_ml, hipStream_t st) {
#define LV_ROWS(GG)                                                                              \
  launch_rows<T, D, GG, BS>(q, q_stride, kc, vc, num_kv_heads, num_cache_blocks, bt, max_blocks, \
                            cu, num_seqs, ctx, row_begin, n_rows, part_tokens, max_parts,         \
                            scale_log2, out, out_stride, ws_acc, ws_ml, st)
  switch (G) {
    case 1: LV_ROWS(1); return LV_OK;
    case 2: LV_ROWS(2); return LV_OK;
    case 4: LV_ROWS(4); return LV_OK;
    case 8: LV_ROWS(8); return LV_OK;
    default:
      set_error("lv_paged_attention: num_heads/num_kv_heads=%d not in {1,2,4,8}", G);
      return LV_ERR_UNSUPPORTED;
  }
#undef LV_ROWS
}

template <typename T>
static int dispatch_d(int D, int G, int BS, const void* q, int64_t q_stride, const void* kc,
                      const void* vc, int num_kv_heads, int64_t num_cache_blocks, const int32_t* bt,
                      int max_blocks, const int32_t* cu, int num_seqs, const int32_t* ctx,
                      int row_begin, int n_rows, int part_tokens, int max_parts, float scale_log2,
                      void* out, int64_t out_stride, float* ws_acc, float* ws_ml,
                      hipStream_t st) {
  if (BS != 16) {
    set_error("lv_paged_attention: block_size=%d unsupported (16)", BS);
    return LV_ERR_UNSUPPORTED;
  }
  if (D == 128)
    return dispatch_g<T, 128, 16>(G, q, q_stride, kc, vc, num_kv_heads, num_cache_blocks, bt,
                                  max_blocks, cu, num_seqs, ctx, row_begin, n_rows, part_tokens,
                                  max_parts, scale_log2, out, out_stride, ws_acc, ws_ml, st);
  if (D == 64)
    return dispatch_g<T, 64, 16>(G, q, q_stride, kc, vc, num_kv_heads, num_cache_blocks, bt,
                                 max_blocks, cu, num_seqs, ctx, row_begin, n_rows, part_tokens,
                                 max_parts, scale_log2, out, out_stride, ws_acc, ws_ml, st);
  set_error("lv_paged_attention: head_dim=%d unsupported (64, 128)", D);
  return LV_ERR_UNSUPPORTED;
}

}  // namespace lv

extern "C" size_t lv_paged_attention_workspace_size(int32_t num_seqs, int32_t num_decodes,
                                                    int64_t num_tokens, int32_t num_heads,
                                                    int32_t head_dim, int32_t block_size,
                                                    int32_t max_blocks, int32_t max_query_len,
                                                    lv_dtype dtype) {
  (void)num_seqs; (void)num_tokens; (void)max_query_len; (void)dtype;
  if (num_decodes <= 0 || block_size <= 0 || max_blocks <= 0) return 0;
  const lv::AttnPlan p = lv::plan_decode(num_decodes, num_heads, head_dim, block_size, max_blocks);
  return p.acc_bytes + p.ml_bytes;
}

extern "C" int lv_paged_attention(const void* query_dev, int64_t q_stride_t,
                                  const void* key_cache_dev, const void* value_cache_dev,
                                  int64_t num_cache_blocks,
                                  const int32_t* block_tables_dev, int32_t max_blocks,
                                  const int32_t* cu_seqlens_dev, const int32_t* context_lens_dev,
                                  int32_t num_seqs, int32_t num_decodes, int64_t num_tokens,
                                  int32_t max_query_len, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t block_size, float scale, void* out_dev,
                                  int64_t out_stride_t, void* workspace_dev,
                                  size_t workspace_bytes, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16,
             "lv_paged_attention: bad dtype");
  LV_REQUIRE(num_seqs >= 0 && num_decodes >= 0 && num_decodes <= num_seqs,
             "lv_paged_attention: need 0 <= num_decodes <= num_seqs");
  if (num_seqs == 0) return LV_OK;
  LV_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "lv_paged_attention: num_heads must be a multiple of num_kv_heads");
  LV_REQUIRE(max_blocks > 0 && block_size > 0 && num_cache_blocks > 0,
             "lv_paged_attention: bad block geometry");
  LV_REQUIRE(query_dev && key_cache_dev && value_cache_dev && block_tables_dev &&
                 context_lens_dev && out_dev,
             "lv_paged_attention: null pointer");
  LV_REQUIRE(cu_seqlens_dev || num_decodes == num_seqs,
             "lv_paged_attention: cu_seqlens required when prefill chunks are present");
  LV_REQUIRE(num_tokens >= num_seqs && num_tokens <= 0x7fffffff,
             "lv_paged_attention: num_tokens=%lld invalid", (long long)num_tokens);
  const size_t es = dtype_size(dtype);
  LV_REQUIRE(aligned16(query_dev) && aligned16(key_cache_dev) && aligned16(value_cache_dev) &&
                 ((q_stride_t * (int64_t)es) % 16) == 0 && ((head_dim * es) % 16) == 0,
             "lv_paged_attention: q/k/v must be 16-byte aligned (strides too)");
  LV_REQUIRE(q_stride_t >= (int64_t)num_heads * head_dim &&
                 out_stride_t >= (int64_t)num_heads * head_dim,
             "lv_paged_attention: token strides smaller than num_heads*head_dim");
  LV_REQUIRE((int64_t)max_blocks * block_size <= (1ll << 24),
             "lv_paged_attention: max_blocks * block_size above 2^24 tokens");

  const int G = num_heads / num_kv_heads;
  const float scale_log2 = scale * 0x1.715476p+0f;
  hipStream_t st = (hipStream_t)stream;
  int rc = LV_OK;

  auto run = [&](int row_begin, int n_rows, const int32_t* cu, int part_tokens, int max_parts,
                 float* ws_acc, float* ws_ml) -> int {
    switch (dtype) {
      case LV_BF16:
        return dispatch_d<bf16>(head_dim, G, block_size, query_dev, q_stride_t, key_cache_dev,
                                value_cache_dev, num_kv_heads, num_cache_blocks, block_tables_dev,
                                max_blocks, cu, num_seqs, context_lens_dev, row_begin, n_rows,
                                part_tokens, max_parts, scale_log2, out_dev, out_stride_t, ws_acc,
                                ws_ml, st);
      case LV_F16:
        return dispatch_d<f16>(head_dim, G, block_size, query_dev, q_stride_t, key_cache_dev,
                               value_cache_dev, num_kv_heads, num_cache_blocks, block_tables_dev,
                               max_blocks, cu, num_seqs, context_lens_dev, row_begin, n_rows,
                               part_tokens, max_parts, scale_log2, out_dev, out_stride_t, ws_acc,
                               ws_ml, st);
      default:
        return dispatch_d<float>(head_dim, G, block_size, query_dev, q_stride_t, key_cache_dev,
                                 value_cache_dev, num_kv_heads, num_cache_blocks, block_tables_dev,
                                 max_blocks, cu, num_seqs, context_lens_dev, row_begin, n_rows,
                                 part_tokens, max_parts, scale_log2, out_dev, out_stride_t, ws_acc,
                                 ws_ml, st);
    }
  };

  if (num_decodes > 0) {
    const AttnPlan p = plan_decode(num_decodes, num_heads, head_dim, block_size, max_blocks);
    float* ws_acc = nullptr;
    float* ws_ml = nullptr;
    if (p.max_parts > 1) {
      if (workspace_dev == nullptr || workspace_bytes < p.acc_bytes + p.ml_bytes ||
          !aligned16(workspace_dev)) {
        set_error("lv_paged_attention: workspace needs %zu bytes (16-B aligned), got %zu",
                  p.acc_bytes + p.ml_bytes, workspace_bytes);
        return LV_ERR_WORKSPACE;
      }
      ws_acc = (float*)workspace_dev;
      ws_ml = (float*)((char*)workspace_dev + p.acc_bytes);
    }
    // Decode rows come first, so row i is sequence i: no cu_seqlens lookup.
    rc = run(0, num_decodes, nullptr, p.part_tokens, p.max_parts, ws_acc, ws_ml);
    if (rc != LV_OK) return rc;
  }
  if (num_decodes < num_seqs) {
    // Prefill-chunk rows: one partition spanning the whole context.
    const int unit = kAttnWaves * block_size;
    const int pt = ((max_blocks * block_size + unit - 1) / unit) * unit;
    const int row_begin = num_decodes;
    const int n_rows = (int)(num_tokens - num_decodes);
    rc = run(row_begin, n_rows, cu_seqlens_dev, pt, 1, nullptr, nullptr);
    if (rc != LV_OK) return rc;
  }
  return check_launch("lv_paged_attention");
}
