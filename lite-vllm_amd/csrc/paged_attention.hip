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

#include <atomic>

#include <type_traits>

#include "lv_common.h"
#include "lv_mfma.h"
#include "lv_split.h"

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

// Online-softmax state of one wavefront for one kv head and the G query
// heads that read it.  Lane = (token-in-load tg, dim chunk dc); every value
// below is per lane.  Scores are kept in log2 units (q pre-scaled by
// scale * log2(e)).
template <typename T, int D, int G, int BS, bool NT>
struct HeadState {
  using C = RowCfg<T, D, BS>;
  static constexpr int VEC = C::VEC, RL = C::ROW_LANES, TPL = C::TPL, LOADS = C::LOADS;
  float qv[G][VEC];
  float m[G], l[G], acc[G][VEC];
  int tg, dc;

  __device__ __forceinline__ void init(const T* __restrict__ qhead, float scale_log2, int lane) {
    tg = lane / RL;
    dc = lane % RL;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      elem<T>::unpack(load16(qhead + (int64_t)g * D + dc * VEC), qv[g]);
#pragma unroll
      for (int j = 0; j < VEC; ++j) qv[g][j] *= scale_log2;
      m[g] = kNegBig;
      l[g] = 0.0f;
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[g][j] = 0.0f;
    }
  }

  // K and V rows of this lane's tokens in physical block `phys`.
  __device__ __forceinline__ void load(const T* __restrict__ kbase, const T* __restrict__ vbase,
                                       int64_t phys, int64_t blk_stride, int64_t tok_stride,
                                       uint4* kk, uint4* vv) const {
    const T* kp = kbase + phys * blk_stride;
    const T* vp = vbase + phys * blk_stride;
#pragma unroll
    for (int r = 0; r < LOADS; ++r)
      kk[r] = NT ? load16_nt(kp + (int64_t)r * TPL * tok_stride)
                 : load16(kp + (int64_t)r * TPL * tok_stride);
#pragma unroll
    for (int r = 0; r < LOADS; ++r)
      vv[r] = NT ? load16_nt(vp + (int64_t)r * TPL * tok_stride)
                 : load16(vp + (int64_t)r * TPL * tok_stride);
  }

  // Fold logical block `blk` (positions blk*BS ..) into the state; positions
  // >= end are masked.
  __device__ __forceinline__ void process(const uint4* kk, const uint4* vv, int blk, int end) {
    float s[G][LOADS];
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      float kf[VEC];
      elem<T>::unpack(kk[r], kf);
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
      elem<T>::unpack(vv[r], vf);
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
  }

  // Stream blocks first, first+stride, ... (n of them) through process().
  // Block ids are fetched 64 at a time with one vector load and handed out
  // with readlane, so no K/V load waits on a block-table read.  Two register
  // buffers alternate: block i+1 is in flight while block i is computed.
  // Every prefetch and every process() is unconditional (the index of a
  // block past the end is clamped to the last one, whose reload hits in
  // cache, and its positions are all masked), so no load sits under a branch
  // where the compiler would sink it next to its use or drain all loads at
  // the join.
  __device__ __forceinline__ void stream(const int32_t* __restrict__ bt, int first, int stride,
                                         int n, int end, const T* __restrict__ kbase,
                                         const T* __restrict__ vbase, int64_t blk_stride,
                                         int64_t tok_stride, int64_t num_cache_blocks, int lane) {
    uint4 k0[LOADS], v0[LOADS], k1[LOADS], v1[LOADS];
    for (int base = 0; base < n; base += 64) {
      const int cnt = min(64, n - base);
      int id = 0;
      if (lane < cnt) {
        id = bt[first + stride * (base + lane)];
        if (id < 0 || id >= num_cache_blocks) {   // clamped and reported
          report_device_error(LV_DEVERR_BLOCK_ID);
          id = 0;
        }
      }
      auto phys = [&](int i) { return __builtin_amdgcn_readlane(id, min(i, cnt - 1)); };
      load(kbase, vbase, phys(0), blk_stride, tok_stride, k0, v0);
      for (int i = 0; i < cnt; i += 2) {
        load(kbase, vbase, phys(i + 1), blk_stride, tok_stride, k1, v1);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the math
        process(k0, v0, first + stride * (base + i), end);
        load(kbase, vbase, phys(i + 2), blk_stride, tok_stride, k0, v0);
        __builtin_amdgcn_sched_barrier(0);
        // Unconditional, so the k1/v1 loads have a use on every path and are
        // not sunk next to it; past the last block every position is masked
        // (end = -1), which leaves the state unchanged.
        process(k1, v1, first + stride * (base + i + 1), i + 1 < cnt ? end : -1);
      }
    }
  }

  // Merge the TPL token groups of the wavefront (lanes RL apart).
  __device__ __forceinline__ void merge_token_groups() {
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
  }
};

// One workgroup (4 wavefronts) per (query row, kv head, context partition);
// wavefront w takes blocks w, w+4, ... of the partition and the four states
// are merged through LDS.
template <typename T, int D, int G, int BS, bool NT>
__global__ __launch_bounds__(kAttnThreads) void attn_rows_kernel(
    const T* __restrict__ q, int64_t q_stride,
    const T* __restrict__ kc, const T* __restrict__ vc, int num_kv_heads, int64_t num_cache_blocks,
    const int32_t* __restrict__ block_tables, int max_blocks,
    const int32_t* __restrict__ cu, int num_seqs, const int32_t* __restrict__ ctx,
    int row_begin, int part_tokens, int max_parts, float scale_log2,
    T* __restrict__ out, int64_t out_stride,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml) {
  using S = HeadState<T, D, G, BS, NT>;
  constexpr int VEC = S::VEC;
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  S st;
  st.init(q + (int64_t)row * q_stride + (int64_t)kvh * G * D, scale_log2, lane);
  const int64_t tok_stride = (int64_t)num_kv_heads * D;
  const int64_t lane_off = (int64_t)kvh * D + st.dc * VEC + st.tg * tok_stride;
  const int b_begin = start / BS;
  const int b_end = (end + BS - 1) / BS;
  const int first = b_begin + wave;
  const int n = first < b_end ? (b_end - first + kAttnWaves - 1) / kAttnWaves : 0;
  st.stream(block_tables + (int64_t)seq * max_blocks, first, kAttnWaves, n, end, kc + lane_off,
            vc + lane_off, (int64_t)BS * tok_stride, tok_stride, num_cache_blocks, lane);
  st.merge_token_groups();

  if (st.tg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) s_acc[wave][g][st.dc * VEC + j] = st.acc[g][j];
      if (st.dc == 0) { s_m[wave][g] = st.m[g]; s_l[wave][g] = st.l[g]; }
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

// ---------------------------------------------------------------------------
// Persistent decode kernel.
//
// The blocks of all decode sequences form one flattened list (sequence-major:
// sequence s owns entries off[s] .. off[s+1]-1, off = exclusive scan of
// ceil(ctx / bs)).  A fixed grid of workgroups (about two per CU) splits the
// list into equal contiguous ranges, so every workgroup streams the same
// number of blocks however ragged the contexts are.  Wavefront w of a
// workgroup owns kv head w; all wavefronts walk the same blocks, so the K/V
// rows of all heads of a block -- one contiguous run in HBM -- are read
// together.  A wavefront streams its whole range without draining: when the
// next block belongs to another sequence it finishes the current one and
// starts the next.  A sequence lying entirely inside one range is written
// straight to `out`; only the first and last piece of a range can be
// partial.  Those pieces go to workspace slots (piece_slot: the first two
// pieces of a sequence row-indexed), workgroup 0 writes one header word per
// sequence (row_header), and attn_persist_reduce_kernel merges the pieces of
// sequences that span several ranges (the kernel boundary orders the partial
// writes before their reads without any device-scope fence inside the
// streaming kernel).
// ---------------------------------------------------------------------------
// Shared-prefix (cascade) pass.  Decode sequences whose block tables begin
// with the same physical blocks (prefix-cache hits) form a group; the
// group's first P blocks are attended once for all members by the MFMA
// body in prefix mode (a launch before the decode kernel), and the decode
// kernel only walks each member's remaining blocks and merges the prefix
// partials in.  Prefix partials are indexed [row][query head][split]
// (split = 128-key slice of the prefix) and hold (m, l) in log2 units and
// acc normalised by l.
struct PrefixArgs {
  const int32_t* blocks;   // [num_decodes] leading blocks handled by the prefix units (0 = none)
  const int32_t* items;    // [max_items][4]: leader row, first member, member count, split
  const int32_t* members;  // member rows, grouped
  int max_items;
  int num_members;         // entries of `members`
  float* ml;               // [rows][H][kPrefixMaxSplits][2]
  float* acc;              // [rows][H][kPrefixMaxSplits][D]
};
constexpr int kPrefixKeysPerSplit = 128;
constexpr int kPrefixMaxSplits = 16;   // prefixes up to 2048 tokens
constexpr int kPrefixMaxBlocks = kPrefixKeysPerSplit * kPrefixMaxSplits / 16;
constexpr int kPrefixMaxRows = 7000;   // decode rows: offsets + skips stay in 56 KB of LDS


constexpr int kPersistMaxWaves = 8;  // kv heads per workgroup (one wavefront each)
constexpr int kPersistMaxSeqs = 15000;  // (B+1) ints of LDS stay under 60 KB

// Exclusive scan of ceil(min(ctx, max_tokens) / bs) into s_off[0..n] by one
// workgroup (integer, order-independent).
// With a shared-prefix pass, sequence i's first skip(i) blocks are attended
// there and left out here.
template <int BS>
__device__ __forceinline__ int walked_blocks(const int32_t* __restrict__ ctx,
                                            const int32_t* __restrict__ skip, int i,
                                            int max_tokens) {
  const int nb = (min(max(ctx[i], 0), max_tokens) + BS - 1) / BS;
  return skip ? nb - min(max(skip[i], 0), min(nb, kPrefixMaxBlocks)) : nb;
}

template <int BS>
__device__ void scan_block_counts(const int32_t* __restrict__ ctx,
                                  const int32_t* __restrict__ skip, int n, int max_tokens,
                                  int32_t* s_off, int32_t* s_part, int32_t* s_skip) {
  const int t = threadIdx.x, nt = blockDim.x;
  const int per = (n + nt - 1) / nt;
  const int lo = min(n, t * per), hi = min(n, lo + per);
  int32_t sum = 0;
  for (int i = lo; i < hi; ++i) {
    const int w = walked_blocks<BS>(ctx, skip, i, max_tokens);
    if (skip) s_skip[i] = (min(max(ctx[i], 0), max_tokens) + BS - 1) / BS - w;
    sum += w;
  }
  s_part[t] = sum;
  __syncthreads();
  for (int d = 1; d < nt; d <<= 1) {
    const int32_t v = (t >= d) ? s_part[t - d] : 0;
    __syncthreads();
    s_part[t] += v;
    __syncthreads();
  }
  int32_t run = (t == 0) ? 0 : s_part[t - 1];
  for (int i = lo; i < hi; ++i) {
    s_off[i] = run;
    run += walked_blocks<BS>(ctx, skip, i, max_tokens);
  }
  if (t == nt - 1) s_off[n] = s_part[nt - 1];
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Prefill-chunk attention on MFMA (bf16 / fp16), v_mfma_f32_32x32x16.
//
// One workgroup (4 wavefronts) per (chunk sequence, kv head, tile of 128/G
// query tokens).  Its 128 rows are (query token, GQA head) pairs sharing the
// kv head: row r -> token r % QT, group head r / QT; wavefront w owns rows
// 32w..32w+31 and holds their Q for the whole kernel.  Keys stream through
// LDS in tiles of 64 (four 16-token blocks), double buffered: the next
// tile's K/V are loaded from HBM into registers while the current tile is
// computed, then written to the other buffer; one barrier per tile.  K and V
// both stay in their natural [key][dim] layout in LDS (16-byte writes).
// Per tile and wavefront:
//   S^T = K Q^T      A = 32 key rows of K (16-byte LDS reads), B = Q^T from
//                    registers; lane l ends with query l % 32 against keys
//                    8(s/4) + 4(l/32) + s%4 of each 32-key half (s = slot);
//   causal mask (key <= query position) and online softmax in fp32 -- the
//   lane owns its query column, so max/sum need one shuffle (xor 32);
//   O^T += V^T P^T   A = V^T read with ds_read_b64_tr_b16 (the LDS transpose
//                    load: in each 16-lane group, lane j receives element
//                    j % 4 of the 4-element reads of lanes 4s + j / 4, so
//                    lanes reading 4 key rows x 16 dims get 4 keys of one dim
//                    each), B = the lane's own probabilities in bf16/fp16
//                    once the 16-key contraction index is permuted as
//                    k = 8h + m -> key 4h + m % 4 + 8 (m / 4) (+16 per step).
// O^T keeps the query as the column, so the softmax rescale is lane-local.
// Keys at or past the end of the needed range are zero-filled and masked.
// ---------------------------------------------------------------------------

// W wavefronts per workgroup: 32 W (query token, head) rows, and LDS tiles
// of 16 W keys (one 16-token block staged per wavefront), computed in
// sub-tiles of 64 keys.

// LDS tile of K or V: 16 W key rows of D elements, unpadded; 16-byte chunk j
// of row r holds the row's chunk j ^ swz(r % 16).  The XOR swizzle keeps
// both read patterns free of bank conflicts on 64 banks of 4 bytes: the K
// reads (16 consecutive rows at one chunk per LDS cycle) need swz to be a
// permutation of 0..15, and the V transpose reads (32 lanes per cycle:
// rows 4i..4i+3 at four consecutive chunks) need bits 2-3 of swz distinct
// over rows 4i..4i+3 -- and bits 1-2 as well, for the 16-lane, 32-bank
// grouping.  swz = 0 6 10 12 1 7 11 13 2 4 8 14 3 5 9 15 meets all three;
// plain r % 16 makes rows 4i..4i+3 share banks.  (D = 64 takes swz % 8.)
template <int D, int W> struct ChunkLds {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int TILE = 16 * W * D;           // elements per K or V tile
  __device__ __forceinline__ static int swz(int row) {
    return (int)((0xF953E842DB71CA60ull >> (4 * (row & 15))) & (CPR - 1));
  }
  __device__ __forceinline__ static int at(int row, int chunk) {
    return row * D + 8 * (chunk ^ swz(row));
  }
};


// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap: lanes 0-31 of
// one copy trade places with lanes 32-63 of the other, so each lane holds
// its own value and its partner's), no LDS round trip.
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ i16x4_t lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)p);
}

// Chunk sequences a chunk workgroup ranks by length (more: index order).
constexpr int kChunkRankMax = 256;

// Arguments of the MFMA attention body (prefill chunks or shared-prefix
// units).
template <typename T>
struct ChunkArgs {
  const T* __restrict__ q; int64_t q_stride;
  const T* __restrict__ kc; const T* __restrict__ vc; int num_kv_heads; int64_t num_cache_blocks;
  const int32_t* __restrict__ block_tables; int max_blocks;
  const int32_t* __restrict__ cu; const int32_t* __restrict__ ctx; int seq_begin;
  int nq_tiles, num_groups; float scale_log2; T* __restrict__ out; int64_t out_stride;
  PrefixArgs pfx;
};

// PFX = false: prefill chunks (causal, normalised output rows); `unit` is
// the workgroup id and `kvh_sel` the chunk sequence (index from seq_begin)
// the caller's longest-first order gives it.  PFX = true: one shared-prefix
// unit -- `unit` is the work item, `kvh_sel` the kv head: up to QT group
// members against one 128-key split of the group's prefix (no causal mask;
// every prefix key precedes every member's query), writing prefix partials.
// The body runs on one team of W wavefronts (`tid` = thread index in the
// team) with its own four LDS tiles.  Every early exit before the last
// barrier depends only on (unit, its item), never on the team or the lane,
// and teams that share a workgroup run the same item, so all wavefronts of
// the workgroup meet the same barriers.
template <typename T, int D, int G, int BS, int W, int BPW, bool PFX>
__device__ __forceinline__ void chunk_mfma_body(const ChunkArgs<T>& A, int unit, int kvh_sel,
                                                int tid, uint16_t* Ks0, uint16_t* Ks1,
                                                uint16_t* Vs0, uint16_t* Vs1) {
  using M = Mfma32<T>;
  using v8 = typename M::v8;
  using L = ChunkLds<D, W * BPW>;
  constexpr int kThreads = 64 * W;
  constexpr int QT = 32 * W / G;       // query tokens per workgroup
  constexpr int KT = 16 * W * BPW;     // keys per LDS tile
  constexpr int NSUB = KT / 64;        // 64-key sub-tiles per LDS tile
  static_assert(NSUB == 1 || NSUB == 2, "one or two 64-key sub-tiles");
  constexpr int QSTEPS = D / 16;       // k-steps of K Q^T
  constexpr int DBLK = D / 32;         // 32-dim blocks of O^T
  constexpr int CPR = L::CPR;
  constexpr int RPI = 64 / CPR;        // key rows per wave-wide 1 KiB load
  constexpr int LPW = BS / RPI;        // loads per wavefront per tile (one block each)
  static_assert(BS == 16 && (W == 4 || W == 8), "each wavefront stages one 16-token block");
  const T* __restrict__ q = A.q;
  const int64_t q_stride = A.q_stride;
  const T* __restrict__ kc = A.kc;
  const T* __restrict__ vc = A.vc;
  const int num_kv_heads = A.num_kv_heads;
  const int64_t num_cache_blocks = A.num_cache_blocks;
  const int max_blocks = A.max_blocks;
  const float scale_log2 = A.scale_log2;
  const PrefixArgs& pfx = A.pfx;

  // XCD-aware, longest-first order (chunks): workgroups are dispatched
  // round-robin over the XCDs (id % kXcds) and, on each XCD, in id order as
  // slots free up.  Workgroup id w serves group g = (w / kXcds / nq) *
  // kXcds + w % kXcds -- kv head g % Hkv of the (g / Hkv)-th longest chunk
  // sequence (the caller ranks them) -- and query tile nq - 1 - (w / kXcds)
  // % nq: all query tiles of one group run on one XCD and share its L2 copy
  // of the group's K/V, and each XCD starts with the longest tiles, which
  // shortens the tail of the last wave of workgroups.
  int kvh, seq, q0, qlen, qt0, pos0, kb0, kend, mbeg = 0, split = 0;
  if constexpr (PFX) {
    const int item = unit;
    kvh = kvh_sel;
    if (item >= pfx.max_items) return;
    const int4 it = *reinterpret_cast<const int4*>(pfx.items + 4 * item);
    // unused item (leader < 0), leaders beyond the decode rows (num_groups),
    // member slices outside `members` or wider than QT, splits beyond the
    // partial buffers: skipped
    if (it.x < 0 || it.x >= A.num_groups || it.w < 0 || it.w >= kPrefixMaxSplits || it.y < 0 ||
        it.z < 1 || it.z > QT || it.y > pfx.num_members - it.z)
      return;
    seq = it.x;                                 // the group leader's block table
    mbeg = it.y;
    qlen = it.z;                                // members in this item (<= QT)
    split = it.w;
    q0 = 0;
    qt0 = 0;
    const int pkeys = min(min(pfx.blocks[seq], max_blocks), kPrefixMaxBlocks) * BS;
    kb0 = split * kPrefixKeysPerSplit;
    kend = min(pkeys, kb0 + kPrefixKeysPerSplit);
    pos0 = 0x3fffffff;                          // queries follow every prefix key
    if (kb0 >= kend) return;
  } else {
    const int wg = unit;
    const int slot = wg / kXcds;
    const int grp = (slot / A.nq_tiles) * kXcds + wg % kXcds;
    if (grp >= A.num_groups) return;
    kvh = grp % num_kv_heads;
    seq = A.seq_begin + kvh_sel;
    q0 = A.cu[seq];
    qlen = A.cu[seq + 1] - q0;
    qt0 = (A.nq_tiles - 1 - slot % A.nq_tiles) * QT;
    if (qt0 >= qlen) return;
    const int ctxlen = min(A.ctx[seq], max_blocks * BS);
    pos0 = ctxlen - qlen;                                      // position of chunk row 0
    kb0 = 0;
    kend = max(0, min(ctxlen, pos0 + min(qt0 + QT, qlen)));    // keys [0, kend)
    if (kend <= 0) return;
  }
  const int ntiles = (kend - kb0 + KT - 1) / KT;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31;        // this lane's query column / key row
  const int h = lane >> 5;         // half of the wavefront
  const int64_t tok_stride = (int64_t)num_kv_heads * D;
  const int32_t* __restrict__ bt = A.block_tables + (int64_t)seq * max_blocks;

  // This lane's query row (the B-operand column of K Q^T).
  const int row = 32 * wave + lr;
  const int qtok = qt0 + row % QT;
  const int qg = row / QT;
  const int qpos = PFX ? pos0 : pos0 + qtok;
  int qrow = PFX ? pfx.members[mbeg + min(qtok, qlen - 1)] : q0 + min(qtok, qlen - 1);
  bool qrow_ok = true;
  if constexpr (PFX) {
    qrow_ok = qrow >= 0 && qrow < A.num_groups;
    qrow = qrow_ok ? qrow : seq;
  }
  v8 qf[QSTEPS];
  {
    const T* qp = q + (int64_t)qrow * q_stride + (int64_t)(kvh * G + qg) * D + 8 * h;
#pragma unroll
    for (int st = 0; st < QSTEPS; ++st) qf[st] = __builtin_bit_cast(v8, load16(qp + 16 * st));
  }

  // Staging: wavefront w loads block w of the tile (rows 16w..16w+15) with
  // LPW wave-wide loads; lane l of load u fills LDS slot l % CPR of row
  // 16w + RPI u + l / CPR, i.e. the row's chunk (l % CPR) ^ swz(row).
  int64_t goff[LPW];
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const int r = RPI * u + lane / CPR;            // row inside the block
    const int chunk = (lane % CPR) ^ L::swz(r);        // 16-row blocks keep row & 15
    goff[u] = (int64_t)r * tok_stride + (int64_t)kvh * D + 8 * chunk;
  }
  const int last_blk = (kend - 1) / BS;
  const int64_t blk_elems = (int64_t)BS * tok_stride;
  // Chunks: physical ids of this wavefront's blocks (blocks wave + W j of
  // each tile), 64 tiles at a time: lane l of bids[j] holds tile bid_tb + l,
  // loaded ahead so staging a tile never waits for a block-table read.  (A
  // shared-prefix unit has at most two tiles and reads its ids directly.)
  int bids[BPW];
  int bid_tb = 0;
  auto load_bids = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int b = bt[min((kb0 + (tb + lane) * KT) / BS + wave + W * j, last_blk)];
      const bool bad = b < 0 || b >= num_cache_blocks;   // clamped and reported
      if (bad) report_device_error(LV_DEVERR_BLOCK_ID);
      bids[j] = bad ? 0 : b;
    }
    bid_tb = tb;
  };
  if constexpr (!PFX) load_bids(0);
  // Wavefront w stages blocks w, w + W, ... (BPW of them) of the tile.
  auto stage = [&](uint16_t* Kst, uint16_t* Vst, int k0) {
    const int tile = (k0 - kb0) / KT;
    if constexpr (!PFX) {
      if (tile - bid_tb >= 64) load_bids(tile);   // contexts beyond 64 tiles
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int blk = wave + W * j;
      int b;
      if constexpr (PFX) {
        b = bt[min(k0 / BS + blk, last_blk)];
        if (b < 0 || b >= num_cache_blocks) {   // clamped and reported
          report_device_error(LV_DEVERR_BLOCK_ID);
          b = 0;
        }
      } else {
        b = __builtin_amdgcn_readlane(bids[j], tile - bid_tb);
      }
      const T* kp = kc + (int64_t)b * blk_elems;
      const T* vp = vc + (int64_t)b * blk_elems;
      uint16_t* kd = Kst + 16 * blk * D;
      uint16_t* vd = Vst + 16 * blk * D;
#pragma unroll
      for (int u = 0; u < LPW; ++u) {
        load_lds16(kp + goff[u], kd + RPI * u * D);
        load_lds16(vp + goff[u], vd + RPI * u * D);
      }
    }
  };
  // Rows at or past kend hold data of the clamped block: zero their V so a
  // zero probability never meets a NaN (their scores are masked).
  auto zero_tail = [&](uint16_t* Vst, int k0) {
    for (int c = tid; c < KT * CPR; c += kThreads)
      if (k0 + c / CPR >= kend) store16(Vst + (c / CPR) * D + 8 * (c % CPR), make_uint4(0, 0, 0, 0));
  };

  f32x16_t o[DBLK];
#pragma unroll
  for (int b = 0; b < DBLK; ++b)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[b][i] = 0.0f;
  float m_run = kNegBig, l_run = 0.0f;


  // Per-lane LDS offsets of the MFMA operands.  Rows 32 kb + lr share
  // lr's swizzle (it depends on row % 16 only), so the K offset of step st
  // is kx[st] plus the constant 32 kb D; the V rows 16 t + vrow (+ 8)
  // likewise share a swizzle across t.
  int kx[QSTEPS];
  {
    const int y = h ^ L::swz(lr);         // (2 st + h) ^ sw == 2 st ^ y
#pragma unroll
    for (int st = 0; st < QSTEPS; ++st) kx[st] = lr * D + 8 * ((2 * st) ^ y);
  }
  const int vrow = 4 * h + ((lane & 15) >> 2);
  int voff[DBLK][2];
#pragma unroll
  for (int b = 0; b < DBLK; ++b) {
    const int dim = 32 * b + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    voff[b][0] = L::at(vrow, dim >> 3) + (dim & 7);
    voff[b][1] = L::at(vrow + 8, dim >> 3) + (dim & 7);
  }

  // S^T of one 64-key sub-tile (raw scores, two 32-key halves): 16 MFMAs,
  // step j = (half j / 8, k-step j % 8), with four K operand reads in
  // flight.  The order is pinned (read j + 4 goes out right after MFMA j
  // frees its buffer): left to itself the scheduler, at this register
  // budget, gives all reads one buffer and waits out each read in turn.
  auto qk = [&](const uint16_t* kb_lds, f32x16_t* sv) {
    auto kread = [&](int j) __attribute__((always_inline)) {
      return *reinterpret_cast<const uint4*>(kb_lds + 32 * (j >> 3) * D + kx[j & 7]);
    };
    static_assert(QSTEPS == 8 || QSTEPS == 4, "head_dim 128 or 64");
    constexpr int NJ = 2 * QSTEPS;
    uint4 ka[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ka[j] = kread((j / QSTEPS) * 8 + j % QSTEPS);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      const int kb = j / QSTEPS, st = j % QSTEPS;
      sv[kb] = M::run(__builtin_bit_cast(v8, ka[j & 3]), qf[st], st ? sv[kb] : f32x16_t{});
      if (j + 4 < NJ) ka[j & 3] = kread(((j + 4) / QSTEPS) * 8 + (j + 4) % QSTEPS);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Causal / range mask (MaskT = std::true_type on tiles that may need it;
  // those run in a loop of their own so the mask is never straight-line code
  // on the others): slot i of half kb holds key k0 + 32 kb + 8 (i/4) + 4 h + i%4.
  const int lim = min(qpos, kend - 1);   // last key each row may see
  auto mask = [&](auto MaskT, f32x16_t* sv, int k0) {
    if constexpr (decltype(MaskT)::value) {
      const int d = lim - k0 - 4 * h;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kb + 8 * (i >> 2) + (i & 3) > d) sv[kb][i] = kNegBig;
    }
  };
  // Online softmax in log2 units with a lazily raised maximum: the running
  // maximum m_run moves only when a row's maximum exceeds it by more than
  // 2^8 (or on the first tile), so probabilities stay below 256 and the O
  // rescale is rare.  Returns the factor O must be scaled by (1 = none).
  auto soft = [&](const f32x16_t* sv, uint32_t (*pw)[8]) {
    float mx = kNegBig;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sv[kb][i]);
    mx = xor32_max(mx) * scale_log2;
    float alpha = 1.0f;
    if (mx > m_run + 8.0f) {
      alpha = fast_exp2(m_run - mx);
      m_run = mx;
    }
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = fast_exp2(fmaf(sv[kb][i], scale_log2, -m_run));
        const float p1 = fast_exp2(fmaf(sv[kb][i + 1], scale_log2, -m_run));
        psum += p0 + p1;
        pw[kb][i >> 1] = M::pack2(p0, p1);
      }
    l_run = l_run * alpha + psum;
    return alpha;
  };
  auto rescale = [&](float alpha) {
    if (__ballot(alpha != 1.0f)) {   // uniform branch, rare after the first tile
#pragma unroll
      for (int b = 0; b < DBLK; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[b][i] *= alpha;
    }
  };
  // O^T += V^T P^T over one 64-key sub-tile, four 16-key steps; each step's
  // transpose reads are issued together ahead of its MFMAs.
  auto pv = [&](const uint16_t* vb_lds, const uint32_t (*pw)[8]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t* pp = &pw[t >> 1][4 * (t & 1)];
      const v8 pb = __builtin_bit_cast(v8, make_uint4(pp[0], pp[1], pp[2], pp[3]));
      i16x4_t lo[DBLK], hi[DBLK];
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
        lo[b] = lds_read_tr16(vb_lds + 16 * t * D + voff[b][0]);
        hi[b] = lds_read_tr16(vb_lds + 16 * t * D + voff[b][1]);
      }
#pragma unroll
      for (int b = 0; b < DBLK; ++b) {
        const i16x8_t a = __builtin_shufflevector(lo[b], hi[b], 0, 1, 2, 3, 4, 5, 6, 7);
        o[b] = M::run(__builtin_bit_cast(v8, a), pb, o[b]);
      }
    }
  };
  // One LDS tile.  With two sub-tiles the code order lets the second
  // half's K Q^T overlap the first half's softmax and the first half's
  // P V overlap the second half's softmax (no branch between them).
  auto compute = [&](auto MaskT, const uint16_t* kb_lds, const uint16_t* vb_lds, int k0) {
    if constexpr (NSUB == 1) {
      f32x16_t sv[2];
      uint32_t pw[2][8];
      qk(kb_lds, sv);
      mask(MaskT, sv, k0);
      rescale(soft(sv, pw));
      pv(vb_lds, pw);
    } else {
      f32x16_t s0[2], s1[2];
      uint32_t p0[2][8], p1[2][8];
      qk(kb_lds, s0);
      mask(MaskT, s0, k0);
      qk(kb_lds + 64 * D, s1);
      mask(MaskT, s1, k0 + 64);
      rescale(soft(s0, p0));
      pv(vb_lds, p0);
      rescale(soft(s1, p1));
      pv(vb_lds + 64 * D, p1);
    }
  };

  // One step: start loading the next tile into the other stage, compute
  // this one, then wait for the loads and make them visible to all.
  auto step = [&](auto MaskT, uint16_t* Kc, uint16_t* Vc, uint16_t* Kn, uint16_t* Vn, int it) {
    const int k0 = kb0 + it * KT;
    const bool more = it + 1 < ntiles;
    if (more) stage(Kn, Vn, k0 + KT);
    compute(MaskT, Kc, Vc, k0);
    __builtin_amdgcn_s_waitcnt(0);   // this thread's LDS loads have landed
    __syncthreads();                 // ... and everyone's; the current stage is free
    if (more && k0 + 2 * KT > kend) {
      zero_tail(Vn, k0 + KT);
      __syncthreads();
    }
  };
  stage(Ks0, Vs0, kb0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (kb0 + KT > kend) {
    zero_tail(Vs0, kb0);
    __syncthreads();
  }
  // Tiles [0, nfull) need no mask for any row of the workgroup (its
  // earliest row sits at position pos0 + qt0); the rest may.
  const int nfull = PFX ? (kend - kb0) / KT
                        : min(ntiles, min(kend, pos0 + qt0 + 1) / KT);
  const std::false_type plain{};
  const std::true_type masked{};
  int it = 0;
  for (; it + 1 < nfull; it += 2) {
    step(plain, Ks0, Vs0, Ks1, Vs1, it);
    step(plain, Ks1, Vs1, Ks0, Vs0, it + 1);
  }
  if (it < nfull) {
    step(plain, Ks0, Vs0, Ks1, Vs1, it);
    ++it;
  }
  for (; it < ntiles; ++it) {
    if (it & 1)
      step(masked, Ks1, Vs1, Ks0, Vs0, it);
    else
      step(masked, Ks0, Vs0, Ks1, Vs1, it);
  }

  // Row sum over both halves of the wavefront, then write this lane's
  // query row: O^T slot i of block b is dim 32 b + 8 (i / 4) + 4 h + i % 4.
  l_run = xor32_sum(l_run);
  if (qtok >= qlen || !qrow_ok) return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  if constexpr (PFX) {
    const int H = num_kv_heads * G;
    const int64_t base = ((int64_t)qrow * H + kvh * G + qg) * kPrefixMaxSplits + split;
    if (h == 0) {
      pfx.ml[base * 2] = m_run;
      pfx.ml[base * 2 + 1] = l_run;
    }
    float* ap = pfx.acc + base * D + 4 * h;
#pragma unroll
    for (int b = 0; b < DBLK; ++b)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<float4*>(ap + 32 * b + 8 * g4) =
            make_float4(o[b][4 * g4] * inv, o[b][4 * g4 + 1] * inv, o[b][4 * g4 + 2] * inv,
                        o[b][4 * g4 + 3] * inv);
    return;
  }
  T* op = A.out + (int64_t)(q0 + qtok) * A.out_stride + (int64_t)(kvh * G + qg) * D + 4 * h;
#pragma unroll
  for (int b = 0; b < DBLK; ++b)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      *reinterpret_cast<uint2*>(op + 32 * b + 8 * g4) =
          make_uint2(M::pack2(o[b][4 * g4] * inv, o[b][4 * g4 + 1] * inv),
                     M::pack2(o[b][4 * g4 + 2] * inv, o[b][4 * g4 + 3] * inv));
}


// The chunk sequence a chunk workgroup of group g serves: group rank
// r = g / Hkv names the r-th chunk sequence by descending context length
// (ties by index), so the longest sequences' tiles are dispatched first.
// Every workgroup ranks the sequences itself (kChunkRankMax of them at
// most; beyond that the order is the index order).  All threads of the
// workgroup call it (it may hold two barriers).
template <typename T>
__device__ __forceinline__ int chunk_rank_pick(const ChunkArgs<T>& a, int grp, int* s_ctx,
                                               int* s_pick) {
  const int nseq = a.num_groups / a.num_kv_heads;
  int pick = grp / a.num_kv_heads;
  if (grp < a.num_groups && nseq > 1 && nseq <= kChunkRankMax) {
    for (int t = threadIdx.x; t < nseq; t += blockDim.x) s_ctx[t] = a.ctx[a.seq_begin + t];
    __syncthreads();
    for (int t = threadIdx.x; t < nseq; t += blockDim.x) {
      const int c = s_ctx[t];
      int rank = 0;
      for (int u = 0; u < nseq; ++u) {
        const int cu = s_ctx[u];
        rank += (cu > c || (cu == c && u < t)) ? 1 : 0;
      }
      if (rank == pick) *s_pick = t;
    }
    __syncthreads();
    pick = *s_pick;
  }
  return pick;
}

// Prefill chunks (PFX = false) or the shared-prefix pass as a launch of its
// own (PFX = true: workgroup = (item, kv head)).
template <typename T, int D, int G, int BS, int W, int BPW, bool PFX>
__global__ __launch_bounds__(64 * W, PFX ? 1 : 8 / (W * BPW)) void attn_chunk_mfma_kernel(
    ChunkArgs<T> a) {
  using L = ChunkLds<D, W * BPW>;
  // One LDS object per stage and operand: a load in flight into one stage
  // provably does not alias the reads of the other, so the compiler does not
  // make those reads wait for it.
  __shared__ __align__(16) uint16_t Ks0[L::TILE], Ks1[L::TILE], Vs0[L::TILE], Vs1[L::TILE];
  const int wg = (int)blockIdx.x;
  if constexpr (PFX) {
    chunk_mfma_body<T, D, G, BS, W, BPW, true>(a, wg / a.num_kv_heads, wg % a.num_kv_heads,
                                               (int)threadIdx.x, Ks0, Ks1, Vs0, Vs1);
  } else {
    __shared__ int s_ctx[kChunkRankMax];
    __shared__ int s_pick;
    const int grp = (wg / kXcds / a.nq_tiles) * kXcds + wg % kXcds;
    const int pick = chunk_rank_pick(a, grp, s_ctx, &s_pick);
    chunk_mfma_body<T, D, G, BS, W, BPW, false>(a, wg, pick, (int)threadIdx.x, Ks0, Ks1, Vs0,
                                                Vs1);
  }
}

template <typename T, int D, int G, int BS, bool NT, int NBUF>
__global__ __launch_bounds__(kPersistMaxWaves * 64) void attn_decode_persistent_kernel(
    const T* __restrict__ q, int64_t q_stride,
    const T* __restrict__ kc, const T* __restrict__ vc, int num_kv_heads, int64_t num_cache_blocks,
    const int32_t* __restrict__ block_tables, int max_blocks, const int32_t* __restrict__ ctx,
    int num_seqs, float scale_log2, T* __restrict__ out, int64_t out_stride,
    int32_t* __restrict__ ws_off, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    PrefixArgs pfx, int sync_mask) {
  using S = HeadState<T, D, G, BS, NT>;
  constexpr int VEC = S::VEC;
  // LDS: s_off [num_seqs + 1], then (shared prefixes only) s_skip [num_seqs]
  extern __shared__ int32_t s_off[];
  int32_t* s_skip = s_off + num_seqs + 1;
  __shared__ int32_t s_part[kPersistMaxWaves * 64];
  const int max_tokens = max_blocks * BS;
  const bool has_pfx = pfx.blocks != nullptr;
  scan_block_counts<BS>(ctx, pfx.blocks, num_seqs, max_tokens, s_off, s_part, s_skip);
  const int total = s_off[num_seqs];
  const int H = num_kv_heads * G;
  const int grid = (int)gridDim.x;

  const RangeSplit rs = make_range_split(total, grid);
  // ws_off: offsets [num_seqs + 1], each sequence's skipped blocks
  // [num_seqs], then its header word [num_seqs]
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i <= num_seqs; i += blockDim.x) {
      ws_off[i] = s_off[i];
      if (i < num_seqs) {
        const int skip = has_pfx ? s_skip[i] : 0;
        if (has_pfx) ws_off[num_seqs + 1 + i] = skip;
        const int nsplit = (skip * BS + kPrefixKeysPerSplit - 1) / kPrefixKeysPerSplit;
        ws_off[2 * num_seqs + 1 + i] = row_header(s_off[i], s_off[i + 1], rs, nsplit);
      }
    }
  if (total == 0) return;
  const int r0 = rs.start((int)blockIdx.x);
  const int r1 = rs.start((int)blockIdx.x + 1);
  if (r0 >= r1) return;

  const int lane = threadIdx.x & 63;
  const int kvh = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (kvh >= num_kv_heads) return;
  const int64_t tok_stride = (int64_t)num_kv_heads * D;
  const int64_t blk_stride = (int64_t)BS * tok_stride;

  S st;
  st.tg = lane / S::RL;
  st.dc = lane % S::RL;
  const int64_t lane_off = (int64_t)kvh * D + st.dc * VEC + st.tg * tok_stride;
  const T* kbase = kc + lane_off;
  const T* vbase = vc + lane_off;

  int cur = -1;     // sequence whose state st holds (uniform)
  int cur_end = 0;  // its context length
  int cur_skip = 0; // its leading blocks attended by the shared-prefix units

  // Finish sequence sq: a piece covering the whole sequence goes straight
  // to `out` (merged with the row's shared-prefix partials, which the
  // prefix launch before this one wrote), any other piece to its workspace
  // slot (piece_slot), for the reduce kernel.
  auto finish = [&](int sq) __attribute__((always_inline)) {
    st.merge_token_groups();
    const int a = s_off[sq], b = s_off[sq + 1];
    const bool whole = a >= r0 && b <= r1;
    if (st.tg != 0) return;
    {
      if (whole && cur_skip > 0) {
        // fold in the prefix partials (splits of 128 keys), then normalise
        const int nsplit = (cur_skip * BS + kPrefixKeysPerSplit - 1) / kPrefixKeysPerSplit;
        if constexpr (G <= 2) {
          if (nsplit <= 4) {
            // up to four splits: every partial is loaded in one round trip,
            // then merged in the order of the general loop below
            float qm[G][4], ql[G][4], qa[G][4][S::VEC];
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const int64_t pb = ((int64_t)sq * H + kvh * G + g) * kPrefixMaxSplits;
#pragma unroll
              for (int sp = 0; sp < 4; ++sp) {
                qm[g][sp] = kNegBig;
                ql[g][sp] = 0.0f;
#pragma unroll
                for (int j = 0; j < S::VEC; ++j) qa[g][sp][j] = 0.0f;
                if (sp < nsplit) {
                  qm[g][sp] = pfx.ml[(pb + sp) * 2];
                  ql[g][sp] = pfx.ml[(pb + sp) * 2 + 1];
                  const float* ap = pfx.acc + (pb + sp) * D + st.dc * VEC;
#pragma unroll
                  for (int j = 0; j < S::VEC; ++j) qa[g][sp][j] = ap[j];
                }
              }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const int hq = kvh * G + g;
              float mx = st.m[g];
#pragma unroll
              for (int sp = 0; sp < 4; ++sp)
                if (sp < nsplit) mx = fmaxf(mx, qm[g][sp]);
              const float fs = fast_exp2(st.m[g] - mx);
              float L = st.l[g] * fs;
              float o[S::VEC];
#pragma unroll
              for (int j = 0; j < S::VEC; ++j) o[j] = st.acc[g][j] * fs;
#pragma unroll
              for (int sp = 0; sp < 4; ++sp)
                if (sp < nsplit) {
                  const float f = ql[g][sp] * fast_exp2(qm[g][sp] - mx);
                  L += f;
#pragma unroll
                  for (int j = 0; j < S::VEC; ++j) o[j] = fmaf(qa[g][sp][j], f, o[j]);
                }
              const float inv = L > 0.0f ? 1.0f / L : 0.0f;
              T* op = out + (int64_t)sq * out_stride + (int64_t)hq * D + st.dc * VEC;
#pragma unroll
              for (int j = 0; j < VEC; ++j) elem<T>::store(op + j, o[j] * inv);
            }
            return;
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const int hq = kvh * G + g;
          const int64_t pb = ((int64_t)sq * H + hq) * kPrefixMaxSplits;
          float mx = st.m[g];
          for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, pfx.ml[(pb + sp) * 2]);
          const float fs = fast_exp2(st.m[g] - mx);
          float L = st.l[g] * fs;
          float o[S::VEC];
#pragma unroll
          for (int j = 0; j < S::VEC; ++j) o[j] = st.acc[g][j] * fs;
          for (int sp = 0; sp < nsplit; ++sp) {
            const float f = pfx.ml[(pb + sp) * 2 + 1] * fast_exp2(pfx.ml[(pb + sp) * 2] - mx);
            L += f;
            const float* ap = pfx.acc + (pb + sp) * D + st.dc * VEC;
#pragma unroll
            for (int j = 0; j < S::VEC; ++j) o[j] = fmaf(ap[j], f, o[j]);
          }
          const float inv = L > 0.0f ? 1.0f / L : 0.0f;
          T* op = out + (int64_t)sq * out_stride + (int64_t)hq * D + st.dc * VEC;
#pragma unroll
          for (int j = 0; j < VEC; ++j) elem<T>::store(op + j, o[j] * inv);
        }
        return;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int hq = kvh * G + g;
      const float inv = st.l[g] > 0.0f ? 1.0f / st.l[g] : 0.0f;
      if (whole) {
        T* op = out + (int64_t)sq * out_stride + (int64_t)hq * D + st.dc * VEC;
#pragma unroll
        for (int j = 0; j < VEC; ++j) elem<T>::store(op + j, st.acc[g][j] * inv);
      } else {
        const int slot = piece_slot(sq, rs.piece_rank(a, (int)blockIdx.x), (int)blockIdx.x,
                                    num_seqs);
        const int64_t base = (int64_t)slot * H + hq;
        float* wp = ws_acc + base * D + st.dc * VEC;
#pragma unroll
        for (int j = 0; j < VEC; ++j) wp[j] = st.acc[g][j] * inv;
        if (st.dc == 0) { ws_ml[base * 2] = st.m[g]; ws_ml[base * 2 + 1] = st.l[g]; }
      }
    }
  };

  static_assert(NBUF == 2 || NBUF == 4, "NBUF");
  uint4 k0[S::LOADS], v0[S::LOADS], k1[S::LOADS], v1[S::LOADS];
  uint4 k2[NBUF == 4 ? S::LOADS : 1], v2[NBUF == 4 ? S::LOADS : 1];
  uint4 k3[NBUF == 4 ? S::LOADS : 1], v3[NBUF == 4 ? S::LOADS : 1];
  for (int base = r0; base < r1; base += 64) {
    const int cnt = min(64, r1 - base);
    // Lane i resolves flattened entry base + i: its sequence, logical block
    // and physical block id.
    int lseq = 0, lblk = 0, id = 0;
    if (lane < cnt) {
      const int j = base + lane;
      int lo = 0, hi = num_seqs - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= j) lo = mid; else hi = mid - 1;
      }
      lseq = lo;
      lblk = j - s_off[lo] + (has_pfx ? s_skip[lo] : 0);   // block index in the table
      id = block_tables[(int64_t)lo * max_blocks + lblk];
      if (id < 0 || id >= num_cache_blocks) {   // clamped and reported
        report_device_error(LV_DEVERR_BLOCK_ID);
        id = 0;
      }
    }
    auto phys = [&](int i) { return __builtin_amdgcn_readlane(id, min(i, cnt - 1)); };
    // Start (or continue) the sequence of entry i, then fold its block in;
    // i >= cnt is a fully masked no-op so process() always runs.
    auto visit = [&](const uint4* kk, const uint4* vv, int i) {
      const bool real = i < cnt;
      const int sq = __builtin_amdgcn_readlane(lseq, min(i, cnt - 1));
      const int lb = __builtin_amdgcn_readlane(lblk, min(i, cnt - 1));
      if (real && sq != cur) {
        if (cur >= 0) finish(cur);
        cur = sq;
        cur_end = min(max(ctx[sq], 0), max_tokens);
        cur_skip = has_pfx ? s_skip[sq] : 0;
        st.init(q + (int64_t)sq * q_stride + (int64_t)kvh * G * D, scale_log2, lane);
      }
      st.process(kk, vv, lb, real ? cur_end : -1);
    };
    // NBUF register buffers rotate: NBUF - 1 blocks are in flight while one
    // is folded in.  Loads past the group end reload its last block (cache
    // hit) and their visits are masked no-ops.
    //
    // Every sync_mask + 1 blocks the workgroup's wavefronts (one per kv
    // head, all walking the same blocks) meet at a plain barrier (no memory
    // fence: loads stay in flight across it).  Left alone they drift apart
    // by up to a quarter of the kernel (the CU's memory pipeline does not
    // serve its eight wavefronts evenly) and the last one finishes alone;
    // in step, all of them end together.  Every wavefront runs the same
    // loop trip counts, so each reaches the same barriers.
    if constexpr (NBUF == 2) {
      st.load(kbase, vbase, phys(0), blk_stride, tok_stride, k0, v0);
      for (int i = 0; i < cnt; i += 2) {
        if (sync_mask >= 0 && (i & sync_mask) == 0) __builtin_amdgcn_s_barrier();
        st.load(kbase, vbase, phys(i + 1), blk_stride, tok_stride, k1, v1);
        __builtin_amdgcn_sched_barrier(0);
        visit(k0, v0, i);
        st.load(kbase, vbase, phys(i + 2), blk_stride, tok_stride, k0, v0);
        __builtin_amdgcn_sched_barrier(0);
        visit(k1, v1, i + 1);
      }
    } else {
      st.load(kbase, vbase, phys(0), blk_stride, tok_stride, k0, v0);
      st.load(kbase, vbase, phys(1), blk_stride, tok_stride, k1, v1);
      st.load(kbase, vbase, phys(2), blk_stride, tok_stride, k2, v2);
      for (int i = 0; i < cnt; i += 4) {
        if (sync_mask >= 0 && (i & sync_mask) == 0) __builtin_amdgcn_s_barrier();
        st.load(kbase, vbase, phys(i + 3), blk_stride, tok_stride, k3, v3);
        __builtin_amdgcn_sched_barrier(0);
        visit(k0, v0, i);
        st.load(kbase, vbase, phys(i + 4), blk_stride, tok_stride, k0, v0);
        __builtin_amdgcn_sched_barrier(0);
        visit(k1, v1, i + 1);
        st.load(kbase, vbase, phys(i + 5), blk_stride, tok_stride, k1, v1);
        __builtin_amdgcn_sched_barrier(0);
        visit(k2, v2, i + 2);
        st.load(kbase, vbase, phys(i + 6), blk_stride, tok_stride, k2, v2);
        __builtin_amdgcn_sched_barrier(0);
        visit(k3, v3, i + 3);
      }
    }
  }
  if (cur >= 0) finish(cur);
}

// Merge the pieces of every sequence that spans several workgroup ranges
// (same flattened split as the persistent kernel), together with its
// shared-prefix partials if it has any; write zeros for a sequence with no
// tokens.  Partials are merged in a fixed order: walked pieces in range
// order, then prefix splits in key order.  Thread = (query head, 4 dims).
template <typename T, int D>
__global__ __launch_bounds__(512) void attn_persist_reduce_kernel(
    const int32_t* __restrict__ ws_off, int num_seqs, int num_wgs, int num_heads,
    const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
    T* __restrict__ out, int64_t out_stride, PrefixArgs pfx) {
  constexpr int LPH = D / 4;          // lanes per query head
  constexpr int HPW = 512 / LPH;      // query heads per workgroup
  const int sq = blockIdx.x;
  const int hq = blockIdx.y * HPW + (int)threadIdx.x / LPH;
  const int d = ((int)threadIdx.x % LPH) * 4;
  if (hq >= num_heads) return;
  T* op = out + (int64_t)sq * out_stride + (int64_t)hq * D + d;
  const int64_t pb = ((int64_t)sq * num_heads + hq) * kPrefixMaxSplits;
  // The header word and both row-indexed pieces are loaded together,
  // whether or not the row needs the pieces (their slots always exist); the
  // header then says which of them count and which prefix splits to load.
  const int hdr = ws_off[2 * num_seqs + 1 + sq];
  float2 pml[2], qml[4];
  float4 pa[2], qa[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t base = ((int64_t)sq * 2 + i) * num_heads + hq;
    pml[i] = *reinterpret_cast<const float2*>(ws_ml + base * 2);
    pa[i] = *reinterpret_cast<const float4*>(ws_acc + base * D + d);
  }
  int np = header_pieces(hdr);
  const int nsplit = header_splits(hdr);
  const bool need_pfx = pfx.blocks != nullptr && np != 1;
#pragma unroll
  for (int sp = 0; sp < 4; ++sp) {
    qml[sp] = make_float2(kNegBig, 0.0f);
    qa[sp] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (need_pfx && sp < nsplit) {
      qml[sp] = *reinterpret_cast<const float2*>(pfx.ml + (pb + sp) * 2);
      qa[sp] = *reinterpret_cast<const float4*>(pfx.acc + (pb + sp) * D + d);
    }
  }
  // keep every load above the branches below
#pragma unroll
  for (int i = 0; i < 2; ++i)
    asm volatile("" ::"v"(pml[i].x), "v"(pml[i].y), "v"(pa[i].x), "v"(pa[i].y), "v"(pa[i].z),
                 "v"(pa[i].w));
#pragma unroll
  for (int sp = 0; sp < 4; ++sp)
    asm volatile("" ::"v"(qml[sp].x), "v"(qml[sp].y), "v"(qa[sp].x), "v"(qa[sp].y),
                 "v"(qa[sp].z), "v"(qa[sp].w));
  if (np == 1) return;     // finished (with its prefix) by the decode kernel
  auto put = [&](float l, const float o[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) elem<T>::store(op + j, l > 0.0f ? o[j] / l : 0.0f);
  };
  if (np <= 2 && nsplit <= 4) {
    // at most two pieces and four prefix splits (the common case): merged
    // from the registers, in the order of the general loop below
    float M = kNegBig;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (i < np) M = fmaxf(M, pml[i].x);
#pragma unroll
    for (int sp = 0; sp < 4; ++sp)
      if (sp < nsplit) M = fmaxf(M, qml[sp].x);
    float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (i < np) {
        const float f = pml[i].y * fast_exp2(pml[i].x - M);
        L += f;
        O[0] = fmaf(pa[i].x, f, O[0]); O[1] = fmaf(pa[i].y, f, O[1]);
        O[2] = fmaf(pa[i].z, f, O[2]); O[3] = fmaf(pa[i].w, f, O[3]);
      }
#pragma unroll
    for (int sp = 0; sp < 4; ++sp)
      if (sp < nsplit) {
        const float f = qml[sp].y * fast_exp2(qml[sp].x - M);
        L += f;
        O[0] = fmaf(qa[sp].x, f, O[0]); O[1] = fmaf(qa[sp].y, f, O[1]);
        O[2] = fmaf(qa[sp].z, f, O[2]); O[3] = fmaf(qa[sp].w, f, O[3]);
      }
    put(L, O);
    return;
  }
  // three or more pieces, or more than four splits: pieces from their slots
  int g0 = 0;
  if (np == 3) {
    const int a = ws_off[sq], b = ws_off[sq + 1];
    const RangeSplit rs = make_range_split(ws_off[num_seqs], num_wgs);
    g0 = rs.owner(a);
    np = rs.owner(b - 1) - g0 + 1;
  }
  auto piece = [&](int i, float2& ml, float4& v) __attribute__((always_inline)) {
    const int64_t base = (int64_t)piece_slot(sq, min(i, 2), g0 + i, num_seqs) * num_heads + hq;
    ml = *reinterpret_cast<const float2*>(ws_ml + base * 2);
    v = *reinterpret_cast<const float4*>(ws_acc + base * D + d);
  };
  float M = kNegBig;
  for (int i = 0; i < np; ++i) {
    float2 ml; float4 v;
    piece(i, ml, v);
    M = fmaxf(M, ml.x);
  }
  for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, pfx.ml[(pb + sp) * 2]);
  float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < np; ++i) {
    float2 ml; float4 v;
    piece(i, ml, v);
    const float f = ml.y * fast_exp2(ml.x - M);
    L += f;
    O[0] = fmaf(v.x, f, O[0]); O[1] = fmaf(v.y, f, O[1]);
    O[2] = fmaf(v.z, f, O[2]); O[3] = fmaf(v.w, f, O[3]);
  }
  for (int sp = 0; sp < nsplit; ++sp) {
    const float f = pfx.ml[(pb + sp) * 2 + 1] * fast_exp2(pfx.ml[(pb + sp) * 2] - M);
    L += f;
    const float4 v = *reinterpret_cast<const float4*>(pfx.acc + (pb + sp) * D + d);
    O[0] = fmaf(v.x, f, O[0]); O[1] = fmaf(v.y, f, O[1]);
    O[2] = fmaf(v.z, f, O[2]); O[3] = fmaf(v.w, f, O[3]);
  }
  put(L, O);
}

// Merge the partitions of one (row, query head); rows with a single
// partition were finished by the attention kernel.
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

// Decode kernel choice.  Default: the persistent kernel with non-temporal
// K/V loads.  Tuning knobs (environment): LV_ATTN_DECODE_KERNEL=rows selects
// the workgroup-per-(row, kv head, partition) kernel, LV_ATTN_PART_TOKENS its
// partition length, LV_ATTN_NT=0 plain loads, LV_ATTN_PERSIST_WGS the
// persistent grid size.
static bool env_is(const char* name, char c) {
  const char* e = getenv(name);
  return e != nullptr && e[0] == c;
}

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  if (e == nullptr) return dflt;
  const int v = atoi(e);
  return v > 0 ? v : dflt;
}

// CU count of the current device (queried once per device).
static int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct AttnPlan {
  bool persistent;
  bool nt;
  int nbuf;         // persistent kernel: blocks in flight per wavefront + 1
  int part_tokens;  // rows kernel
  int max_parts;    // rows kernel
  int num_wgs;      // persistent kernel
  int sync_mask;    // persistent kernel: barrier every sync_mask + 1 blocks (-1: none)
  size_t off_bytes, ml_bytes, acc_bytes;  // off_bytes: flattened block offsets
  size_t bytes() const { return off_bytes + ml_bytes + acc_bytes; }
};

static AttnPlan plan_decode(int num_decodes, int num_heads, int num_kv_heads, int head_dim,
                            int block_size, int max_blocks) {
  AttnPlan p{};
  p.nt = !env_is("LV_ATTN_NT", '0');
  p.persistent = !env_is("LV_ATTN_DECODE_KERNEL", 'r') && num_kv_heads <= kPersistMaxWaves &&
                 num_decodes <= kPersistMaxSeqs;
  if (p.persistent) {
    // One workgroup of num_kv_heads wavefronts per CU; each wavefront keeps
    // NBUF - 1 blocks (8 KiB each at the Qwen3 shape) in flight.
    p.nbuf = env_int("LV_ATTN_NBUF", 2) == 4 ? 4 : 2;
    p.num_wgs = env_int("LV_ATTN_PERSIST_WGS", device_cu_count() * (num_kv_heads == 1 ? 4 : 1));
    // wavefront lockstep interval in blocks (LV_ATTN_SYNC=0: none)
    int sync = env_is("LV_ATTN_SYNC", '0') ? 0 : env_int("LV_ATTN_SYNC", 4);
    int pow2 = 2;
    while (pow2 < sync && pow2 < 64) pow2 *= 2;
    p.sync_mask = sync > 0 ? pow2 - 1 : -1;
    // block offsets [num_decodes + 1], shared-prefix skips and header words
    // [num_decodes] each; piece slots (piece_slot): two per decode row and
    // one per workgroup, each (m, l) and head_dim floats per query head
    const size_t slots = 2 * (size_t)num_decodes + (size_t)p.num_wgs;
    p.off_bytes = align256(sizeof(int32_t) * (size_t)(3 * num_decodes + 1));
    p.ml_bytes = align256(sizeof(float) * 2 * slots * num_heads);
    p.acc_bytes = align256(sizeof(float) * slots * num_heads * head_dim);
    return p;
  }
  const int unit = kAttnWaves * block_size;
  p.part_tokens = ((env_int("LV_ATTN_PART_TOKENS", 256) + unit - 1) / unit) * unit;
  const int max_tokens = max_blocks * block_size;
  p.max_parts = max_tokens > 0 ? (max_tokens + p.part_tokens - 1) / p.part_tokens : 1;
  if (p.max_parts <= 1) {
    p.max_parts = 1;
  } else {
    const size_t n = (size_t)num_decodes * num_heads * p.max_parts;
    p.acc_bytes = align256(n * head_dim * sizeof(float));
    p.ml_bytes = align256(n * 2 * sizeof(float));
  }
  return p;
}

template <typename T, int D, int G, int BS, bool NT>
static void launch_rows(const void* q, int64_t q_stride, const void* kc, const void* vc,
                        int num_kv_heads, int64_t num_cache_blocks, const int32_t* bt,
                        int max_blocks, const int32_t* cu, int num_seqs, const int32_t* ctx,
                        int row_begin, int n_rows, int part_tokens, int max_parts,
                        float scale_log2, void* out, int64_t out_stride, float* ws_acc,
                        float* ws_ml, hipStream_t st) {
  const dim3 grid(n_rows, num_kv_heads, max_parts);
  hipLaunchKernelGGL((attn_rows_kernel<T, D, G, BS, NT>), grid, dim3(kAttnThreads), 0, st,
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

template <typename T, int D, int G, int BS, bool NT, int NBUF>
static void launch_persistent(const void* q, int64_t q_stride, const void* kc, const void* vc,
                              int num_kv_heads, int64_t num_cache_blocks, const int32_t* bt,
                              int max_blocks, const int32_t* ctx, int num_seqs, float scale_log2,
                              void* out, int64_t out_stride, const AttnPlan& p, char* ws,
                              const PrefixArgs& pfx, hipStream_t st) {
  int32_t* ws_off = (int32_t*)ws;
  float* ws_ml = (float*)(ws + p.off_bytes);
  float* ws_acc = (float*)(ws + p.off_bytes + p.ml_bytes);
  // (the entry point admits a prefix only for bf16 / fp16, head_dim 64 / 128)
  if constexpr (!std::is_same<T, float>::value && (D == 64 || D == 128) && BS == 16) {
    if (pfx.blocks && pfx.max_items > 0) {
      // shared prefixes first: their partials are read by the two kernels below
      const ChunkArgs<T> ca{(const T*)q, q_stride, (const T*)kc, (const T*)vc, num_kv_heads,
                            num_cache_blocks, bt, max_blocks, nullptr, ctx, 0, 1, num_seqs,
                            scale_log2, (T*)out, out_stride, pfx};
      hipLaunchKernelGGL((attn_chunk_mfma_kernel<T, D, G, 16, 4, 1, true>),
                         dim3((unsigned)(pfx.max_items * num_kv_heads)), dim3(256), 0, st, ca);
    }
  }
  const size_t lds = sizeof(int32_t) * (size_t)(num_seqs + 1 + (pfx.blocks ? num_seqs : 0));
  hipLaunchKernelGGL((attn_decode_persistent_kernel<T, D, G, BS, NT, NBUF>), dim3(p.num_wgs),
                     dim3(64 * num_kv_heads), lds, st, (const T*)q, q_stride, (const T*)kc,
                     (const T*)vc, num_kv_heads, num_cache_blocks, bt, max_blocks, ctx, num_seqs,
                     scale_log2, (T*)out, out_stride, ws_off, ws_acc, ws_ml, pfx, p.sync_mask);
  constexpr int kHeadsPerReduceWg = 512 / (D / 4);
  const int H = num_kv_heads * G;
  hipLaunchKernelGGL((attn_persist_reduce_kernel<T, D>),
                     dim3(num_seqs, (H + kHeadsPerReduceWg - 1) / kHeadsPerReduceWg), dim3(512),
                     0, st, (const int32_t*)ws_off, num_seqs, p.num_wgs, H,
                     (const float*)ws_acc, (const float*)ws_ml, (T*)out, out_stride, pfx);
}

// Everything one launch needs besides the dtype / shape template arguments.
struct LaunchArgs {
  const void* q; int64_t q_stride; const void* kc; const void* vc; int num_kv_heads;
  int64_t num_cache_blocks; const int32_t* bt; int max_blocks; const int32_t* cu; int num_seqs;
  const int32_t* ctx; int row_begin; int n_rows; float scale_log2; void* out; int64_t out_stride;
  hipStream_t st;
  PrefixArgs pfx;   // decode rows' shared-prefix pass (blocks == nullptr: none)
};

template <typename T, int D, int G, int BS>
static void launch(const LaunchArgs& a, const AttnPlan& p, char* ws) {
  float* ws_ml = ws ? (float*)(ws + p.off_bytes) : nullptr;
  float* ws_acc = ws ? (float*)(ws + p.off_bytes + p.ml_bytes) : nullptr;
  if (p.persistent) {
#define LV_PERSIST(NT_, NB_)                                                                    \
  launch_persistent<T, D, G, BS, NT_, NB_>(a.q, a.q_stride, a.kc, a.vc, a.num_kv_heads,        \
                                           a.num_cache_blocks, a.bt, a.max_blocks, a.ctx,       \
                                           a.n_rows, a.scale_log2, a.out, a.out_stride, p, ws,  \
                                           a.pfx, a.st)
    if (p.nt && p.nbuf == 4) LV_PERSIST(true, 4);
    else if (p.nt) LV_PERSIST(true, 2);
    else if (p.nbuf == 4) LV_PERSIST(false, 4);
    else LV_PERSIST(false, 2);
#undef LV_PERSIST
  } else if (p.nt) {
    launch_rows<T, D, G, BS, true>(a.q, a.q_stride, a.kc, a.vc, a.num_kv_heads,
                                   a.num_cache_blocks, a.bt, a.max_blocks, a.cu, a.num_seqs, a.ctx,
                                   a.row_begin, a.n_rows, p.part_tokens, p.max_parts, a.scale_log2,
                                   a.out, a.out_stride, ws_acc, ws_ml, a.st);
  } else {
    launch_rows<T, D, G, BS, false>(a.q, a.q_stride, a.kc, a.vc, a.num_kv_heads,
                                    a.num_cache_blocks, a.bt, a.max_blocks, a.cu, a.num_seqs,
                                    a.ctx, a.row_begin, a.n_rows, p.part_tokens, p.max_parts,
                                    a.scale_log2, a.out, a.out_stride, ws_acc, ws_ml, a.st);
  }
}
template <typename T, int D, int BS>
static int dispatch_g(int G, const LaunchArgs& a, const AttnPlan& p, char* ws) {
  switch (G) {
    case 1: launch<T, D, 1, BS>(a, p, ws); return LV_OK;
    case 2: launch<T, D, 2, BS>(a, p, ws); return LV_OK;
    case 4: launch<T, D, 4, BS>(a, p, ws); return LV_OK;
    case 8: launch<T, D, 8, BS>(a, p, ws); return LV_OK;
    default:
      set_error("lv_paged_attention: num_heads/num_kv_heads=%d not in {1,2,4,8}", G);
      return LV_ERR_UNSUPPORTED;
  }
}

template <typename T>
static int dispatch_d(int D, int G, int BS, const LaunchArgs& a, const AttnPlan& p, char* ws) {
  if (BS != 16) {
    set_error("lv_paged_attention: block_size=%d unsupported (16)", BS);
    return LV_ERR_UNSUPPORTED;
  }
  if (D == 128) return dispatch_g<T, 128, 16>(G, a, p, ws);
  if (D == 64) return dispatch_g<T, 64, 16>(G, a, p, ws);
  set_error("lv_paged_attention: head_dim=%d unsupported (64, 128)", D);
  return LV_ERR_UNSUPPORTED;
}

static int dispatch(lv_dtype dt, int D, int G, int BS, const LaunchArgs& a, const AttnPlan& p,
                    char* ws) {
  switch (dt) {
    case LV_BF16: return dispatch_d<bf16>(D, G, BS, a, p, ws);
    case LV_F16: return dispatch_d<f16>(D, G, BS, a, p, ws);
    default: return dispatch_d<float>(D, G, BS, a, p, ws);
  }
}

template <typename T, int D, int G, int W, int BPW>
static void launch_chunk_kernel_w(const LaunchArgs& a, const int32_t* cu, int seq_begin,
                                  int n_seqs, int max_query_len) {
  constexpr int QT = 32 * W / G;
  const int nq = (max_query_len + QT - 1) / QT;
  const int groups = a.num_kv_heads * n_seqs;
  const int64_t wgs = (int64_t)((groups + kXcds - 1) / kXcds) * kXcds * nq;
  const ChunkArgs<T> ca{(const T*)a.q, a.q_stride, (const T*)a.kc, (const T*)a.vc,
                        a.num_kv_heads, a.num_cache_blocks, a.bt, a.max_blocks, cu, a.ctx,
                        seq_begin, nq, groups, a.scale_log2, (T*)a.out, a.out_stride,
                        PrefixArgs{}};
  hipLaunchKernelGGL((attn_chunk_mfma_kernel<T, D, G, 16, W, BPW, false>), dim3((unsigned)wgs),
                     dim3(64 * W), 0, a.st, ca);
}

// Chunk workgroups: 4 wavefronts, 64-key tiles, two workgroups per CU.
template <typename T, int D, int G>
static void launch_chunk_kernel(const LaunchArgs& a, const int32_t* cu, int seq_begin, int n_seqs,
                                int max_query_len) {
  launch_chunk_kernel_w<T, D, G, 4, 1>(a, cu, seq_begin, n_seqs, max_query_len);
}

template <typename T, int D>
static int launch_chunks_g(int G, const LaunchArgs& a, const int32_t* cu, int seq_begin,
                           int n_seqs, int max_query_len) {
  switch (G) {
    case 1: launch_chunk_kernel<T, D, 1>(a, cu, seq_begin, n_seqs, max_query_len); return LV_OK;
    case 2: launch_chunk_kernel<T, D, 2>(a, cu, seq_begin, n_seqs, max_query_len); return LV_OK;
    case 4: launch_chunk_kernel<T, D, 4>(a, cu, seq_begin, n_seqs, max_query_len); return LV_OK;
    case 8: launch_chunk_kernel<T, D, 8>(a, cu, seq_begin, n_seqs, max_query_len); return LV_OK;
    default:
      set_error("lv_paged_attention: num_heads/num_kv_heads=%d not in {1,2,4,8}", G);
      return LV_ERR_UNSUPPORTED;
  }
}

static int launch_chunks(lv_dtype dt, int D, int G, const LaunchArgs& a, const int32_t* cu,
                         int seq_begin, int n_seqs, int max_query_len) {
  if (dt == LV_BF16)
    return D == 128 ? launch_chunks_g<bf16, 128>(G, a, cu, seq_begin, n_seqs, max_query_len)
                    : launch_chunks_g<bf16, 64>(G, a, cu, seq_begin, n_seqs, max_query_len);
  return D == 128 ? launch_chunks_g<f16, 128>(G, a, cu, seq_begin, n_seqs, max_query_len)
                  : launch_chunks_g<f16, 64>(G, a, cu, seq_begin, n_seqs, max_query_len);
}

LV_ERROR_WORD_READER(read_errors_attention)

}  // namespace lv

extern "C" size_t lv_paged_attention_workspace_size(int32_t num_seqs, int32_t num_decodes,
                                                    int64_t num_tokens, int32_t num_heads,
                                                    int32_t head_dim, int32_t block_size,
                                                    int32_t max_blocks, int32_t max_query_len,
                                                    lv_dtype dtype) {
  (void)num_seqs; (void)num_tokens; (void)max_query_len; (void)dtype;
  if (num_decodes <= 0 || block_size <= 0 || max_blocks <= 0 || num_heads <= 0) return 0;
  // num_kv_heads is not an argument: take the larger of the persistent plan
  // at its biggest grid (one kv head) and the workgroup-per-row plan (used
  // above kPersistMaxWaves kv heads).
  const lv::AttnPlan a = lv::plan_decode(num_decodes, num_heads, 1, head_dim, block_size, max_blocks);
  const lv::AttnPlan b = lv::plan_decode(num_decodes, num_heads, lv::kPersistMaxWaves + 1, head_dim,
                                         block_size, max_blocks);
  return a.bytes() > b.bytes() ? a.bytes() : b.bytes();
}

static int paged_attention_impl(const void* query_dev, int64_t q_stride_t,
                                const void* key_cache_dev, const void* value_cache_dev,
                                int64_t num_cache_blocks, const int32_t* block_tables_dev,
                                int32_t max_blocks, const int32_t* cu_seqlens_dev,
                                const int32_t* context_lens_dev, int32_t num_seqs,
                                int32_t num_decodes, int64_t num_tokens, int32_t max_query_len,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, float scale, void* out_dev,
                                int64_t out_stride_t, void* workspace_dev, size_t workspace_bytes,
                                lv_dtype dtype, void* stream, const lv::PrefixArgs* pfx) {
  using namespace lv;
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
  LaunchArgs a{query_dev, q_stride_t, key_cache_dev, value_cache_dev, num_kv_heads,
               num_cache_blocks, block_tables_dev, max_blocks, nullptr, num_seqs,
               context_lens_dev, 0, 0, scale_log2, out_dev, out_stride_t, (hipStream_t)stream};

  // Decode rows: plan and checks first, so a bad workspace or prefix plan
  // fails before anything is launched.
  AttnPlan pd{};
  if (num_decodes > 0) {
    pd = plan_decode(num_decodes, num_heads, num_kv_heads, head_dim, block_size, max_blocks);
    // the persistent kernel's flattened block list is indexed in 32 bits
    LV_REQUIRE(!pd.persistent || (int64_t)num_decodes * max_blocks <= (1ll << 31) - (1ll << 16),
               "lv_paged_attention: num_decodes * max_blocks above 2^31 - 2^16 (persistent "
               "decode kernel; LV_ATTN_DECODE_KERNEL=rows has no such limit)");
    if (pd.bytes() > 0 && (workspace_dev == nullptr || workspace_bytes < pd.bytes() ||
                           (reinterpret_cast<uintptr_t>(workspace_dev) & 255) != 0)) {
      set_error("lv_paged_attention: workspace needs %zu bytes (256-B aligned), got %zu",
                pd.bytes(), workspace_bytes);
      return LV_ERR_WORKSPACE;
    }
    if (pfx && (!pd.persistent || dtype == LV_F32 || (head_dim != 64 && head_dim != 128) ||
                block_size != 16 || !(G == 1 || G == 2 || G == 4 || G == 8) ||
                num_decodes > kPrefixMaxRows)) {
      set_error("lv_paged_attention_prefix: no shared-prefix path for this shape");
      return LV_ERR_UNSUPPORTED;
    }
  }
  // Chunk rows go first: the K/V rows this step just wrote are still in the
  // last-level cache for them; the decode rows' walk reads far more than it
  // holds either way.
  if (num_decodes < num_seqs && dtype != LV_F32 && (head_dim == 64 || head_dim == 128) &&
      block_size == 16 && (G == 1 || G == 2 || G == 4 || G == 8) &&
      !env_is("LV_ATTN_CHUNK_KERNEL", 'r')) {
    LV_REQUIRE(max_query_len >= 1, "lv_paged_attention: max_query_len must be >= 1");
    const int rc = launch_chunks(dtype, head_dim, G, a, cu_seqlens_dev, num_decodes,
                                 num_seqs - num_decodes, max_query_len);
    if (rc != LV_OK) return rc;
  } else if (num_decodes < num_seqs) {
    // Prefill-chunk rows without an MFMA path (fp32): one row per query
    // token, one partition spanning the whole context.
    AttnPlan p{};
    p.persistent = false;
    p.nt = false;
    const int unit = kAttnWaves * block_size;
    p.part_tokens = ((max_blocks * block_size + unit - 1) / unit) * unit;
    p.max_parts = 1;
    a.cu = cu_seqlens_dev;
    a.num_seqs = num_seqs;
    a.row_begin = num_decodes;
    a.n_rows = (int)(num_tokens - num_decodes);
    const int rc = dispatch(dtype, head_dim, G, block_size, a, p, nullptr);
    if (rc != LV_OK) return rc;
  }
  if (num_decodes > 0) {
    // Decode rows come first in the batch, so row i is sequence i: no
    // cu_seqlens lookup.
    a.cu = nullptr;
    a.num_seqs = num_decodes;
    a.row_begin = 0;
    a.n_rows = num_decodes;
    if (pfx) a.pfx = *pfx;
    const int rc = dispatch(dtype, head_dim, G, block_size, a, pd, (char*)workspace_dev);
    a.pfx = PrefixArgs{};
    if (rc != LV_OK) return rc;
  }
  return check_launch("lv_paged_attention");
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
  lv::clear_error();
  return paged_attention_impl(query_dev, q_stride_t, key_cache_dev, value_cache_dev,
                              num_cache_blocks, block_tables_dev, max_blocks, cu_seqlens_dev,
                              context_lens_dev, num_seqs, num_decodes, num_tokens, max_query_len,
                              num_heads, num_kv_heads, head_dim, block_size, scale, out_dev,
                              out_stride_t, workspace_dev, workspace_bytes, dtype, stream,
                              nullptr);
}

extern "C" size_t lv_paged_attention_prefix_workspace_size(int32_t num_decodes,
                                                           int32_t num_heads,
                                                           int32_t head_dim) {
  if (num_decodes <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  const size_t n = (size_t)num_decodes * num_heads * lv::kPrefixMaxSplits;
  return lv::align256(n * 2 * sizeof(float)) + lv::align256(n * head_dim * sizeof(float));
}

extern "C" int lv_paged_attention_prefix(
    const void* query_dev, int64_t q_stride_t, const void* key_cache_dev,
    const void* value_cache_dev, int64_t num_cache_blocks, const int32_t* block_tables_dev,
    int32_t max_blocks, const int32_t* cu_seqlens_dev, const int32_t* context_lens_dev,
    int32_t num_seqs, int32_t num_decodes, int64_t num_tokens, int32_t max_query_len,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
    void* out_dev, int64_t out_stride_t, void* workspace_dev, size_t workspace_bytes,
    const int32_t* prefix_blocks_dev, const int32_t* prefix_items_dev, int32_t max_items,
    const int32_t* prefix_members_dev, int32_t num_members, void* prefix_workspace_dev,
    size_t prefix_workspace_bytes, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(num_decodes >= 1 && num_decodes <= kPrefixMaxRows,
             "lv_paged_attention_prefix: num_decodes must be in [1, %d]", kPrefixMaxRows);
  LV_REQUIRE(prefix_blocks_dev && prefix_members_dev && max_items >= 0 && num_members >= 0 &&
                 (prefix_items_dev || max_items == 0),
             "lv_paged_attention_prefix: null prefix description");
  LV_REQUIRE((reinterpret_cast<uintptr_t>(prefix_items_dev) & 15) == 0,
             "lv_paged_attention_prefix: prefix_items must be 16-byte aligned");
  const size_t need = lv_paged_attention_prefix_workspace_size(num_decodes, num_heads, head_dim);
  if (!prefix_workspace_dev || prefix_workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(prefix_workspace_dev) & 255) != 0) {
    set_error("lv_paged_attention_prefix: prefix workspace needs %zu bytes (256-B aligned), "
              "got %zu", need, prefix_workspace_bytes);
    return LV_ERR_WORKSPACE;
  }
  const size_t n = (size_t)num_decodes * num_heads * kPrefixMaxSplits;
  PrefixArgs pa;
  pa.blocks = prefix_blocks_dev;
  pa.items = prefix_items_dev;
  pa.members = prefix_members_dev;
  pa.max_items = max_items;
  pa.num_members = num_members;
  pa.ml = (float*)prefix_workspace_dev;
  pa.acc = (float*)((char*)prefix_workspace_dev + align256(n * 2 * sizeof(float)));
  return paged_attention_impl(query_dev, q_stride_t, key_cache_dev, value_cache_dev,
                              num_cache_blocks, block_tables_dev, max_blocks, cu_seqlens_dev,
                              context_lens_dev, num_seqs, num_decodes, num_tokens, max_query_len,
                              num_heads, num_kv_heads, head_dim, block_size, scale, out_dev,
                              out_stride_t, workspace_dev, workspace_bytes, dtype, stream, &pa);
}
