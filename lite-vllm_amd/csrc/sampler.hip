// Fused greedy / temperature sampler over [B, V] logits.
//
// Two launches.  sampler_items_kernel streams the batch as "items" of two
// consecutive 512-element segments of one row, spread over a grid of a few
// workgroups per CU: wavefront w takes items w, w + nw, w + 2 nw, ... (nw
// wavefronts in all), so every wavefront meets the batch's greedy and
// temperature rows in proportion and neighbouring wavefronts read
// neighbouring segments.  The next item's loads are issued before the
// current item is folded.  Per segment it stores the maximum and, for a
// temperature row, sigma_s (defined below).  Each segment's arithmetic is
// self-contained, so how items are spread over wavefronts does not change
// any bit.  sampler_finish_kernel (one wavefront per row) finds a greedy
// row's first maximum (the first segment holding the row maximum, then its
// first element equal to it), or runs the cross-segment part and the
// search of a temperature row.
//
// Greedy rows (temperature 0) follow _argmax_kernel / torch.argmax
// (reference litevllm/layers/sampler.py:60-84, 111-124): the first index of
// the fp32 maximum.  NaN entries never win; a row with no finite-or-+inf
// maximum (all -inf / NaN) returns 0.
//
// Temperature rows replace softmax(x / T) + torch.multinomial
// (sampler.py:127-144, 177-187) by an inverse-CDF draw at a caller-supplied
// uniform u in [0, 1).  The arithmetic is fixed so that the CPU
// restatement reproduces it bit for bit:
//
//   c      = log2(e) / T                       (one correctly rounded division)
//   segment s = elements [512 s, 512 s + 512)  (last one partial)
//   m_s    = max of the segment, e_j = exp2_det((x_j - m_s) * c)
//   a_k    = e_{8k} + ... + e_{8k+7}  sequentially, lane chunk k = 0..63
//   A_k    = inclusive Hillis-Steele scan of a_k over k (step d = 1..32:
//            A_k <- A_k + A_{k-d} for k >= d, all k at once)
//   sigma_s = A_63
//   M      = max_s m_s,  w_s = sigma_s * exp2_det((m_s - M) * c)
//   R      = ceil(nseg / 64); group k holds segments [kR, kR + R)
//   b_k    = w_{kR} + w_{kR+1} + ... sequentially; B_k = Hillis-Steele scan
//   S = B_63, r = u * S
//   level 1: k* = first k with B_k > r and b_k > 0, else last k with b_k > 0
//   level 2: acc = B_{k*-1} (0 for k* = 0); walk segments of k* in order,
//            first s with (acc + w_s) > r, else the last s with w_s > 0
//            (acc advanced sequentially: acc <- acc + w_s); base = acc
//            before s
//   level 3: scale = exp2_det((m_s - M) * c); first lane chunk k with
//            base + A_k * scale > r and a_k > 0, else last k with a_k > 0
//   level 4: q = A_{k-1} (0 for k = 0); for j in the chunk: q <- q + e_j;
//            first j with e_j > 0 and base + q * scale > r, else the last j
//            with e_j > 0.
//   exp2_det(t), t <= 0 in every use: t < -200 and NaN become -200;
//            n = floor(t), f = t - n (a result of 1.0, from t in (-2^-25, 0),
//            becomes the largest float below 1: the fract instruction's
//            clamp); P(f) = 1 + f(c1 + f(c2 + f(c3 + f(c4 + f c5)))) with
//            fused multiply-adds, c1..c5 a degree-5 minimax fit of 2^f on
//            [0, 1) rounded to fp32; result ldexp(P(f), n), rounded once
//            (subnormal below 2^-126, 0 below about 2^-150).
// Every sum, product and comparison is an IEEE fp32 operation in the order
// written (this file is compiled with -ffp-contract=off).
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "lv_common.h"

namespace lv {

constexpr int kSeg = 512;
constexpr int kMaxSegs = 4096;  // vocab up to 2^21

// log2(e) rounded to fp32.
constexpr float kLog2e = 0x1.715476p+0f;

// exp2_det of the header: fract + floor-convert + five fused multiply-adds
// + ldexp.  The relative error of P against 2^f is below 2^-22.7 for every
// fp32 f in [0, 1), and P(0) = 1, so exp2_det(0) = 1 exactly.
__device__ __forceinline__ float exp2_det(float t) {
  t = fmaxf(t, -200.0f);                      // NaN -> -200
  const float f = __builtin_amdgcn_fractf(t);  // t - floor(t), clamped below 1
  int n;
  asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(t));
  float q = 0x1.e974fap-10f;
  q = fmaf(q, f, 0x1.277856p-7f);
  q = fmaf(q, f, 0x1.c91ce6p-5f);
  q = fmaf(q, f, 0x1.ebdb5ap-3f);
  q = fmaf(q, f, 0x1.62e4bap-1f);
  const float p = fmaf(q, f, 1.0f);
  return __builtin_amdgcn_ldexpf(p, n);
}

// Maximum over the 64 lanes, every lane receiving it.  The four in-row steps
// are DPP max instructions written out (lane i with i^1, i^2, 7-i within 8,
// 15-i within 16); the inputs are fmaxf results, hence never signalling
// NaNs, so no canonicalizing step is needed between them.  The cross-row
// steps go through the LDS crossbar.
__device__ __forceinline__ float wave_max64(float x) {
  asm volatile(
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(x));
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

// Maximum of a lane's 8 elements.
__device__ __forceinline__ float max8(const float x[8]) {
  float m = fmaxf(fmaxf(x[0], x[1]), x[2]);
  m = fmaxf(fmaxf(m, x[3]), x[4]);
  m = fmaxf(fmaxf(m, x[5]), x[6]);
  return fmaxf(m, x[7]);
}

// Load elements [512 s + 8 lane, +8) of a row as fp32; entries past V are
// -inf.  `vec` says the row start is 16-byte aligned.
template <typename T>
__device__ __forceinline__ void load_chunk(const T* __restrict__ row, int64_t V, int s, int lane,
                                           bool vec, float x[8]) {
  const int64_t e0 = (int64_t)s * kSeg + lane * 8;
  if (vec && e0 + 8 <= V) {
    if constexpr (elem<T>::kPer16B == 8) {
      elem<T>::unpack(load16(row + e0), x);
    } else {
      elem<T>::unpack(load16(row + e0), x);
      elem<T>::unpack(load16(row + e0 + 4), x + 4);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      x[j] = (e0 + j < V) ? elem<T>::load(row + e0 + j) : -__builtin_inff();
  }
}

// Inclusive Hillis-Steele scan across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_scan_hs(float a, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float y = __shfl_up(a, d);
    if (lane >= d) a = a + y;
  }
  return a;
}

// Per-chunk exp weights and their sequential sum (the a_k of the header).
// The sum starts from e_0 itself: 0 + e_0 = e_0, as e_0 >= +0.
__device__ __forceinline__ float chunk_weights(const float x[8], float ms, float c, float e[8]) {
  e[0] = exp2_det((x[0] - ms) * c);
  float a = e[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    e[j] = exp2_det((x[j] - ms) * c);
    a = a + e[j];
  }
  return a;
}

// Per-(row, segment) results of the first kernel, [rows, nseg] each:
// m = the segment's maximum (fp32, NaN ignored); w = sigma_s (temperature
// rows; 0 for greedy rows).
struct SampWs {
  float* m;
  float* w;
};

constexpr int kItemSegs = 2;               // segments per item
constexpr int kItemWaves = 4;              // wavefronts per workgroup
constexpr int kItemThreads = 64 * kItemWaves;
constexpr int kMaxItemsPerWave = 64;       // lane k holds the k-th item's c

// One lane's 8 elements of a segment, fetched in one step and converted in
// another so the loads stay in flight while the previous item is folded.
// VEC (16-byte aligned rows, V % 8 == 0): 16-byte loads (two for fp32) at
// a byte offset clamped into the row; a lane chunk is then either wholly
// inside the row or wholly past V, and the fold masks the latter.
template <typename T, bool VEC>
struct SegWords {
  static constexpr int kWords = elem<T>::kPer16B == 8 ? 1 : 2;
  uint4 w[kWords];

  __device__ __forceinline__ void fetch(const T* __restrict__ row, int V, int sg,
                                        uint32_t lane_bytes) {
    // lane_bytes = 0 for every lane (a placeholder fetch) reads one line
    const uint32_t lim = (uint32_t)(V - 8 - sg * kSeg) * (uint32_t)sizeof(T);
    const char* p = (const char*)row + (uint32_t)sg * (kSeg * (uint32_t)sizeof(T)) +
                    min(lane_bytes, lim);
    w[0] = load16_nt(p);
    if constexpr (kWords == 2) w[1] = load16_nt(p + 16);
  }
  __device__ __forceinline__ void unpack(float x[8]) const {
    elem<T>::unpack(w[0], x);
    if constexpr (kWords == 2) elem<T>::unpack(w[1], x + 4);
  }
};

// General rows: guarded element loads, converted at once (entries past V
// are -inf already).
template <typename T>
struct SegWords<T, false> {
  float v[8];

  __device__ __forceinline__ void fetch(const T* __restrict__ row, int V, int sg,
                                        uint32_t lane_bytes) {
    const int e0 = sg * kSeg + (int)(lane_bytes / sizeof(T));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (e0 + j < V) ? elem<T>::load(row + e0 + j) : -__builtin_inff();
  }
  __device__ __forceinline__ void unpack(float x[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = v[j];
  }
};

// Grid requirements (sample_launch): rows * ceil(nseg / 2) < 2^31, rows *
// nseg < 2^31, and at most kMaxItemsPerWave items per wavefront.
template <typename T, bool VEC>
__global__ __launch_bounds__(kItemThreads) void sampler_items_kernel(
    const T* __restrict__ logits, int V, int64_t row_stride,
    const float* __restrict__ temperature, SampWs ws, int rows, int nseg) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * kItemWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nw = gridDim.x * kItemWaves;
  const int ipr = (nseg + kItemSegs - 1) / kItemSegs;   // items per row
  const int total = rows * ipr;
  if (w >= total) return;
  // Lane k: c of the wavefront's item k (w + k nw), or -1 for a greedy row;
  // one division per wavefront instead of one per item.
  float cv;
  {
    const int ik = min(w + lane * nw, total - 1);
    const float temp = temperature[ik / ipr];
    const float c = kLog2e / temp;
    cv = (!(temp > 0.0f) || !(c <= 3.0e38f)) ? -1.0f : c;
  }
  const uint32_t lane_bytes = (uint32_t)lane * 8u * (uint32_t)sizeof(T);
  // fetch(i, live = false) is the placeholder issued past the wavefront's
  // last item: every lane reads the first 16 bytes of item i's row (one
  // cache line, no HBM stream), so the loop's loads stay unconditional.
  auto fetch = [&](int i, bool live, SegWords<T, VEC>* b) {
    const int r = i / ipr;
    const int s0 = live ? (i - r * ipr) * kItemSegs : 0;
    const uint32_t lb = live ? lane_bytes : 0u;
    const T* row = logits + (int64_t)r * row_stride;
#pragma unroll
    for (int u = 0; u < kItemSegs; ++u) b[u].fetch(row, V, min(s0 + u, nseg - 1), lb);
  };
  auto fold = [&](int i, int k, const SegWords<T, VEC>* b) {
    const int r = i / ipr;
    const int s0 = (i - r * ipr) * kItemSegs;
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv), k));
    const bool greedy = c < 0.0f;
    float mres[kItemSegs], wres[kItemSegs];
#pragma unroll
    for (int u = 0; u < kItemSegs; ++u) {
      float x[8];
      b[u].unpack(x);
      if ((s0 + u + 1) * kSeg > V) {   // uniform: the row's last segment (or past it)
        const bool past = (s0 + u) * kSeg + lane * 8 >= V;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = past ? -__builtin_inff() : x[j];
      }
      const float ms = wave_max64(max8(x));
      mres[u] = ms;
      wres[u] = 0.0f;
      if (!greedy) {
        // sigma_s = A_63 of the header's Hillis-Steele scan.  The butterfly
        // sum adds the same pairs in the same order (lane 63 holds the
        // larger index of every pair, as in A_k + A_{k-d}; fp32 addition is
        // commutative, so every lane ends with A_63's bits).
        float e[8];
        wres[u] = group_sum<64>(chunk_weights(x, ms, c, e));
      }
    }
    // Lane l stores slot l % 4 (m of segment s0 + slot, or sigma of segment
    // s0 + slot - 2); every lane stores, so no store sits under a branch and
    // the compiler keeps counting the next item's loads instead of waiting
    // for them.  A slot past the row's last segment repeats that segment's
    // store.
    const int slot = lane & (2 * kItemSegs - 1);
    const int uu = min(slot < kItemSegs ? slot : slot - kItemSegs, nseg - 1 - s0);
    float vm = mres[0], vw = wres[0];
#pragma unroll
    for (int u = 1; u < kItemSegs; ++u) {
      vm = (uu == u) ? mres[u] : vm;
      vw = (uu == u) ? wres[u] : vw;
    }
    float* dst = (slot < kItemSegs ? ws.m : ws.w) + (r * nseg + s0 + uu);
    *dst = slot < kItemSegs ? vm : vw;
  };
  // Two items in flight.  Past the wavefront's last item the prefetch is a
  // placeholder; the empty asm and the scheduling barrier keep each
  // prefetch above the fold that follows it.
  SegWords<T, VEC> ba[kItemSegs], bb[kItemSegs];
  int i = w, k = 0;
  fetch(i, true, ba);
  for (;;) {
    const int i1 = i + nw;
    const bool more1 = i1 < total;
    fetch(more1 ? i1 : i, more1, bb);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    fold(i, k, ba);
    if (!more1) break;
    const int i2 = i1 + nw;
    const bool more2 = i2 < total;
    fetch(more2 ? i2 : i1, more2, ba);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    fold(i1, k + 1, bb);
    if (!more2) break;
    i = i2;
    k += 2;
  }
}

// One wavefront per row: merge the greedy candidates, or run the
// cross-segment scan and the four-level search of the header.
template <typename T>
__global__ __launch_bounds__(64) void sampler_finish_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride,
    const float* __restrict__ temperature, const float* __restrict__ uniform, SampWs ws,
    int nseg, int64_t* __restrict__ out, int vec_ok) {
  extern __shared__ float s_mw[];   // segment maxima [nseg], then weights [nseg]
  float* s_m = s_mw;
  float* s_w = s_mw + nseg;
  const int64_t r = blockIdx.x;
  const T* row = logits + r * row_stride;
  const int lane = threadIdx.x;
  const bool vec = vec_ok != 0;
  const float temp = temperature[r];
  const float u = uniform[r];
  // The workspace rows go to LDS while the temperature load is in flight
  // (both kinds of row read the maxima).
  const float* wm = ws.m + r * nseg;
  const float* ww = ws.w + r * nseg;
  for (int i = lane; i < nseg; i += 64) {
    s_m[i] = wm[i];
    s_w[i] = ww[i];
  }
  __syncthreads();
  const float c = kLog2e / temp;
  const bool greedy = !(temp > 0.0f) || !(c <= 3.0e38f);
  if (greedy) {
    // the first index of the row maximum: the first segment whose maximum
    // is the row's, then the first element there equal to it (NaN never
    // wins; a row with nothing above -inf gives 0)
    float M = -__builtin_inff();
    for (int sg = lane; sg < nseg; sg += 64) M = fmaxf(M, s_m[sg]);
    M = group_max<64>(M);
    if (!(M > -__builtin_inff())) {
      if (lane == 0) out[r] = 0;
      return;
    }
    int first = nseg;
    for (int sg = lane; sg < nseg; sg += 64)
      if (s_m[sg] == M) { first = sg; break; }
#pragma unroll
    for (int ofs = 32; ofs >= 1; ofs >>= 1) first = min(first, __shfl_xor(first, ofs));
    float x[8];
    load_chunk(row, V, first, lane, vec, x);
    int j = 8;
#pragma unroll
    for (int jj = 7; jj >= 0; --jj)
      if (x[jj] == M) j = jj;
    const uint64_t hit = __ballot(j < 8);
    const int kk = hit ? __ffsll((unsigned long long)hit) - 1 : 0;
    const int jk = __shfl(j, kk);
    if (lane == 0) out[r] = (int64_t)first * kSeg + kk * 8 + (jk < 8 ? jk : 0);
    return;
  }

  // Segment weights, total and the search.
  float M = -__builtin_inff();
  for (int sg = lane; sg < nseg; sg += 64) M = fmaxf(M, s_m[sg]);
  M = group_max<64>(M);
  const int R = (nseg + 63) / 64;
  const int g0 = min(nseg, lane * R), g1 = min(nseg, g0 + R);
  float b = 0.0f;
  for (int sg = g0; sg < g1; ++sg) {
    const float w = s_w[sg] * exp2_det((s_m[sg] - M) * c);
    s_w[sg] = w;  // each lane owns its own segments
    b = b + w;
  }
  const float B = wave_scan_hs(b, lane);
  const float S = __shfl(B, 63);
  if (!(S > 0.0f)) {
    if (lane == 0) out[r] = 0;
    return;
  }
  const float target = u * S;

  // Level 1.
  const uint64_t hit = __ballot(B > target && b > 0.0f);
  int k;
  if (hit) {
    k = __ffsll((unsigned long long)hit) - 1;
  } else {
    const uint64_t nz = __ballot(b > 0.0f);
    k = 63 - __clzll((long long)nz);
  }
  const float Bprev = __shfl(B, k > 0 ? k - 1 : 0);
  const float base_k = (k == 0) ? 0.0f : Bprev;

  // Level 2 (uniform across lanes: every lane walks the same segments).
  const int t0 = min(nseg, k * R), t1 = min(nseg, t0 + R);
  int sstar = -1;
  float base = 0.0f;
  {
    float acc = base_k;
    for (int sg = t0; sg < t1; ++sg) {
      const float w = s_w[sg];
      const float nxt = acc + w;
      if (nxt > target) { sstar = sg; base = acc; break; }
      acc = nxt;
    }
    if (sstar < 0) {
      acc = base_k;
      for (int sg = t0; sg < t1; ++sg) {
        const float w = s_w[sg];
        if (w > 0.0f) { sstar = sg; base = acc; }
        acc = acc + w;
      }
    }
  }

  // Unreachable when S > 0 (group k* holds a positive weight); kept so a
  // logic error can never turn into an out-of-bounds read.
  if (sstar < 0) sstar = 0;

  // Level 3: recompute the segment's chunk weights exactly as in phase 1.
  float x[8], e[8];
  load_chunk(row, V, sstar, lane, vec, x);
  float ms = x[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) ms = fmaxf(ms, x[j]);
  ms = group_max<64>(ms);
  const float a = chunk_weights(x, ms, c, e);
  const float A = wave_scan_hs(a, lane);
  const float Aprev = __shfl_up(A, 1);
  const float scale = exp2_det((s_m[sstar] - M) * c);
  const uint64_t hit3 = __ballot((base + A * scale > target) && a > 0.0f);
  int kk;
  if (hit3) {
    kk = __ffsll((unsigned long long)hit3) - 1;
  } else {
    const uint64_t nz = __ballot(a > 0.0f);
    kk = nz ? 63 - __clzll((long long)nz) : 0;
  }

  // Level 4.
  if (lane == kk) {
    float q = (kk == 0) ? 0.0f : Aprev;
    int jstar = -1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      q = q + e[j];
      if (jstar < 0 && e[j] > 0.0f && base + q * scale > target) jstar = j;
    }
    if (jstar < 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (e[j] > 0.0f) jstar = j;
    }
    if (jstar < 0) jstar = 0;
    out[r] = (int64_t)sstar * kSeg + kk * 8 + jstar;
  }
}

}  // namespace lv

namespace lv {
// Workspace: per (row, segment) two floats, 256-byte aligned.
static inline size_t samp_ws_bytes(int64_t rows, int64_t V) {
  const int64_t nseg = (V + kSeg - 1) / kSeg;
  return (size_t)rows * (size_t)nseg * 8 + 256;
}

// Workgroups of the item kernel for `items` items: LV_SAMPLER_WGS_PER_CU
// (default 8, i.e. eight wavefronts per SIMD) per CU, no more wavefronts
// than items, and enough wavefronts that none has more than
// kMaxItemsPerWave items.
static int samp_grid(int64_t items) {
  static std::atomic<int> cus{0};
  int n = cus.load(std::memory_order_relaxed);
  if (n <= 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus.store(n, std::memory_order_relaxed);
  }
  static const int per_cu = [] {
    const char* e = getenv("LV_SAMPLER_WGS_PER_CU");
    const int v = e ? atoi(e) : 8;
    return (v >= 1 && v <= 32) ? v : 8;
  }();
  const int64_t by_items = (items + kItemWaves - 1) / kItemWaves;
  const int64_t at_least =
      (items + (int64_t)kMaxItemsPerWave * kItemWaves - 1) / ((int64_t)kMaxItemsPerWave * kItemWaves);
  return (int)std::max<int64_t>(at_least,
                                std::min<int64_t>((int64_t)n * per_cu, std::max<int64_t>(1, by_items)));
}
}  // namespace lv

extern "C" size_t lv_sample_workspace_size(int64_t num_rows, int64_t vocab_size) {
  using namespace lv;
  if (num_rows <= 0 || vocab_size <= 0 || vocab_size > (int64_t)kSeg * kMaxSegs) return 0;
  return samp_ws_bytes(num_rows, vocab_size);
}

namespace lv {
// Enqueue both kernels with the workspace at `base` (256-byte aligned, at
// least samp_ws_bytes(num_rows, vocab_size) - 256 bytes).
static int sample_launch(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
                         int64_t row_stride, const float* temperature_dev,
                         const float* uniform_dev, int64_t* out_ids_dev, char* base,
                         lv_dtype dtype, hipStream_t st) {
  const int vec = aligned16(logits_dev) && ((row_stride * (int64_t)dtype_size(dtype)) % 16 == 0);
  const int nseg = (int)((vocab_size + kSeg - 1) / kSeg);
  SampWs ws;
  ws.m = (float*)base;
  ws.w = ws.m + (size_t)num_rows * nseg;
  const int64_t items = num_rows * ((nseg + kItemSegs - 1) / kItemSegs);
  const int grid = samp_grid(items);
  const bool vec_items = vec && vocab_size % 8 == 0;
#define LV_SAMPLE_LAUNCH(TT)                                                                    \
  if (vec_items)                                                                                \
    hipLaunchKernelGGL((sampler_items_kernel<TT, true>), dim3(grid), dim3(kItemThreads), 0, st, \
                       (const TT*)logits_dev, (int)vocab_size, row_stride, temperature_dev, ws,  \
                       (int)num_rows, nseg);                                                     \
  else                                                                                          \
    hipLaunchKernelGGL((sampler_items_kernel<TT, false>), dim3(grid), dim3(kItemThreads), 0,    \
                       st, (const TT*)logits_dev, (int)vocab_size, row_stride, temperature_dev,  \
                       ws, (int)num_rows, nseg);                                                 \
  hipLaunchKernelGGL(sampler_finish_kernel<TT>, dim3((unsigned)num_rows), dim3(64),              \
                     sizeof(float) * 2 * (size_t)nseg, st,                                       \
                     (const TT*)logits_dev, vocab_size, row_stride, temperature_dev,             \
                     uniform_dev, ws, nseg, out_ids_dev, vec)
  switch (dtype) {
    case LV_BF16: LV_SAMPLE_LAUNCH(bf16); break;
    case LV_F16: LV_SAMPLE_LAUNCH(f16); break;
    default: LV_SAMPLE_LAUNCH(float); break;
  }
#undef LV_SAMPLE_LAUNCH
  return check_launch("sampler kernels");
}

// Argument checks shared by both entry points.
static int sample_check(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
                        int64_t row_stride, const float* temperature_dev,
                        const float* uniform_dev, const int64_t* out_ids_dev, lv_dtype dtype) {
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16, "lv_sample: bad dtype");
  LV_REQUIRE(num_rows >= 0 && num_rows <= 0x7fffffff, "lv_sample: bad num_rows");
  if (num_rows == 0) return LV_OK;
  LV_REQUIRE(vocab_size >= 1 && vocab_size <= (int64_t)kSeg * kMaxSegs,
             "lv_sample: vocab_size=%lld outside [1, %d]", (long long)vocab_size, kSeg * kMaxSegs);
  LV_REQUIRE(row_stride >= vocab_size, "lv_sample: row_stride < vocab_size");
  LV_REQUIRE(num_rows * ((vocab_size + kSeg - 1) / kSeg) <= 0x7fffffff,
             "lv_sample: num_rows x segments of 512 above 2^31 - 1");
  LV_REQUIRE(logits_dev && temperature_dev && out_ids_dev, "lv_sample: null pointer");
  LV_REQUIRE(uniform_dev, "lv_sample: uniform draws required (pass zeros for all-greedy rows)");
  return LV_OK;
}

// Scratch of lv_sample_noalloc: one copy per GPU in the code object's own
// device memory, so that entry point never allocates.  Host code must use
// the per-device address returned by hipGetSymbolAddress (scratch_device_ptr),
// never the array's name, which on the host is only a stand-in.  Every call
// on a GPU shares that GPU's copy; nothing in it needs to start at zero
// (each call writes every entry it reads before reading it).
constexpr size_t kSampleScratchBytes = size_t(4) << 20;
static __device__ __align__(256) char scratch[kSampleScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch (looked up once per
// device, with that device current); nullptr with the error set on failure.
static void* scratch_device_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("lv_sample_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p == nullptr) {
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("lv_sample_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}
}  // namespace lv

extern "C" int lv_sample(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
                         int64_t row_stride, const float* temperature_dev, const float* uniform_dev,
                         int64_t* out_ids_dev, void* workspace_dev, size_t workspace_bytes,
                         lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  const int rc = sample_check(logits_dev, num_rows, vocab_size, row_stride, temperature_dev,
                              uniform_dev, out_ids_dev, dtype);
  if (rc != LV_OK || num_rows == 0) return rc;
  const size_t need = samp_ws_bytes(num_rows, vocab_size);
  if (!workspace_dev || workspace_bytes < need) {
    set_error("lv_sample: workspace of %zu bytes required, got %zu", need, workspace_bytes);
    return LV_ERR_WORKSPACE;
  }
  char* base = (char*)(((uintptr_t)workspace_dev + 255) & ~(uintptr_t)255);
  return sample_launch(logits_dev, num_rows, vocab_size, row_stride, temperature_dev, uniform_dev,
                       out_ids_dev, base, dtype, (hipStream_t)stream);
}

extern "C" int lv_sample_noalloc(const void* logits_dev, int64_t num_rows, int64_t vocab_size,
                                 int64_t row_stride, const float* temperature_dev,
                                 const float* uniform_dev, int64_t* out_ids_dev, lv_dtype dtype,
                                 void* stream) {
  using namespace lv;
  clear_error();
  const int rc = sample_check(logits_dev, num_rows, vocab_size, row_stride, temperature_dev,
                              uniform_dev, out_ids_dev, dtype);
  if (rc != LV_OK || num_rows == 0) return rc;
  // samp_ws_bytes includes 256 bytes of alignment slack the scratch does not
  // need; the bound below is the documented one (lv_sample_workspace_size).
  const size_t need = samp_ws_bytes(num_rows, vocab_size);
  if (need > kSampleScratchBytes) {
    set_error("lv_sample_noalloc: %lld rows x vocab %lld need %zu bytes of scratch, above the "
              "fixed %zu (use lv_sample with a workspace)", (long long)num_rows,
              (long long)vocab_size, need, kSampleScratchBytes);
    return LV_ERR_WORKSPACE;
  }
  char* base = (char*)scratch_device_ptr();
  if (base == nullptr) return LV_ERR_HIP;
  return sample_launch(logits_dev, num_rows, vocab_size, row_stride, temperature_dev, uniform_dev,
                       out_ids_dev, base, dtype, (hipStream_t)stream);
}
