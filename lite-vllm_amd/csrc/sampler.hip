// Fused greedy / temperature sampler over [B, V] logits.
//
// Two launches.  sampler_segments_kernel spreads every row over
// ceil(nseg / SPW) workgroups (SPW = 4 wavefronts x UNROLL segments in
// flight x GROUPS rounds, one wavefront per segment; default 16):
// greedy rows leave one (max, index) candidate per workgroup, temperature
// rows leave (m_s, sigma_s) per segment (defined below).  Each segment's
// arithmetic is self-contained, so how segments are spread over workgroups
// does not change any bit.  sampler_search_kernel (one workgroup per row)
// merges the candidates or runs the cross-segment part and the search.
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
// Every sum, product and comparison is an IEEE fp32 operation in the order
// written (this file is compiled with -ffp-contract=off); exp2_det uses only
// fmaf, rint and exact power-of-two scaling.
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "lv_common.h"

namespace lv {

constexpr int kSeg = 512;
constexpr int kMaxSegs = 4096;  // vocab up to 2^21

// log2(e) rounded to fp32.
constexpr float kLog2e = 0x1.715476p+0f;

// exp2 for t <= 0 by range reduction t = n + f, |f| <= 1/2, and the degree-7
// Taylor polynomial of 2^f = sum_k (f ln2)^k / k! (coefficients ln2^k/k!
// rounded to fp32) evaluated by Horner with fused multiply-adds; 2^n is
// applied by an exact power-of-two multiply.  Inputs below -125 (and NaN)
// give 0, so no result is subnormal.  Relative error < 2^-22 on [-125, 0].
__device__ __forceinline__ float exp2_det(float t) {
  // Branch-free form of: t < -125 or NaN -> 0; t > 0 -> t = 0.  For t in
  // [-125, 0] the clamps leave t unchanged, so every result equals the
  // plain definition above bit for bit.
  const bool under = !(t >= -125.0f);
  t = fmaxf(fminf(t, 0.0f), -125.0f);
  const float n = rintf(t);
  const float f = t - n;  // exact (Sterbenz)
  float p = 0x1.ffcbfcp-17f;
  p = fmaf(p, f, 0x1.430912p-13f);
  p = fmaf(p, f, 0x1.5d87fep-10f);
  p = fmaf(p, f, 0x1.3b2ab6p-7f);
  p = fmaf(p, f, 0x1.c6b08ep-5f);
  p = fmaf(p, f, 0x1.ebfbep-3f);
  p = fmaf(p, f, 0x1.62e43p-1f);
  p = fmaf(p, f, 1.0f);
  const int ni = (int)n;
  const float scale = __uint_as_float((uint32_t)(ni + 127) << 23);
  return under ? 0.0f : p * scale;
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
__device__ __forceinline__ float chunk_weights(const float x[8], float ms, float c, float e[8]) {
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    e[j] = exp2_det((x[j] - ms) * c);
    a = a + e[j];
  }
  return a;
}

__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  return v > bv || (v == bv && i < bi);
}

constexpr int kSegThreads = 256;
constexpr int kSegWaves = kSegThreads / 64;


struct SampWs {
  float* m;        // [rows, nseg] segment maxima
  float* w;        // [rows, nseg] segment sums sigma_s
  float* bv;       // [rows, split] greedy candidates: value
  int64_t* bi;     //                                  index
};

template <typename T, int UNROLL, int GROUPS>
__global__ __launch_bounds__(kSegThreads) void sampler_segments_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride,
    const float* __restrict__ temperature, SampWs ws, int nseg, int split, int vec_ok) {
  constexpr int kUnroll = UNROLL, kGroups = GROUPS;
  constexpr int kSegsPerWG = kSegWaves * kUnroll * kGroups;
  __shared__ float s_gv[kSegWaves];
  __shared__ int64_t s_gi[kSegWaves];
  const int64_t r = blockIdx.x;
  const int part = blockIdx.y;
  const T* row = logits + r * row_stride;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const bool vec = vec_ok != 0;
  const float temp = temperature[r];
  const float c = kLog2e / temp;
  const bool greedy = !(temp > 0.0f) || !(c <= 3.0e38f);
  const int sbeg = part * kSegsPerWG;
  const int send = min(nseg, sbeg + kSegsPerWG);

  // Wavefront w folds segments sbeg + w + 4 i in groups of UNROLL; segment
  // index of group g, slot u: sbeg + w + 4 (UNROLL g + u).
  auto seg_of = [&](int g, int u) { return sbeg + wave + kSegWaves * (kUnroll * g + u); };
  auto load_group = [&](int g, float (*x)[8]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = seg_of(g, u);
      if (s < send) load_chunk(row, V, s, lane, vec, x[u]);
    }
  };
  float xa[kUnroll][8], xb[kUnroll][8];
  if (greedy) {
    float bv = -__builtin_inff();
    int64_t bi = INT64_MAX;
    auto fold = [&](int g, float (*x)[8]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int s = seg_of(g, u);
        if (s < send) {
          const int64_t e0 = (int64_t)s * kSeg + lane * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (x[u][j] > bv) { bv = x[u][j]; bi = e0 + j; }
        }
      }
    };
    load_group(0, xa);
#pragma unroll
    for (int g = 0; g < kGroups; g += 2) {
      if (g + 1 < kGroups) load_group(g + 1, xb);
      fold(g, xa);
      if (g + 2 < kGroups) load_group(g + 2, xa);
      if (g + 1 < kGroups) fold(g + 1, xb);
    }
    // Lanes may hold their best from a later segment than an equal value of
    // another lane, so merges are lexicographic on (value, index).
#pragma unroll
    for (int ofs = 32; ofs >= 1; ofs >>= 1) {
      const float ov = __shfl_xor(bv, ofs);
      const int64_t oi = __shfl_xor(bi, ofs);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s_gv[wave] = bv; s_gi[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kSegWaves; ++w)
        if (better(s_gv[w], s_gi[w], bv, bi)) { bv = s_gv[w]; bi = s_gi[w]; }
      ws.bv[r * split + part] = bv;
      ws.bi[r * split + part] = bi;
    }
    return;
  }
  // Per-segment max and scanned exp weights.
  auto fold = [&](int g, float (*x)[8]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = seg_of(g, u);
      if (s < send) {
        float e[8];
        float ms = x[u][0];
#pragma unroll
        for (int j = 1; j < 8; ++j) ms = fmaxf(ms, x[u][j]);
        ms = group_max<64>(ms);
        const float A = wave_scan_hs(chunk_weights(x[u], ms, c, e), lane);
        if (lane == 63) {
          ws.m[r * nseg + s] = ms;
          ws.w[r * nseg + s] = A;
        }
      }
    }
  };
  load_group(0, xa);
#pragma unroll
  for (int g = 0; g < kGroups; g += 2) {
    if (g + 1 < kGroups) load_group(g + 1, xb);
    fold(g, xa);
    if (g + 2 < kGroups) load_group(g + 2, xa);
    if (g + 1 < kGroups) fold(g + 1, xb);
  }
}

template <typename T>
__global__ __launch_bounds__(kSegThreads) void sampler_search_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride,
    const float* __restrict__ temperature, const float* __restrict__ uniform, SampWs ws,
    int nseg, int split, int64_t* __restrict__ out, int vec_ok) {
  __shared__ float s_m[kMaxSegs];
  __shared__ float s_w[kMaxSegs];
  const int64_t r = blockIdx.x;
  const T* row = logits + r * row_stride;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const bool vec = vec_ok != 0;
  const float temp = temperature[r];
  const float c = kLog2e / temp;
  const bool greedy = !(temp > 0.0f) || !(c <= 3.0e38f);
  if (greedy) {
    if (threadIdx.x == 0) {
      float bv = -__builtin_inff();
      int64_t bi = INT64_MAX;
      for (int p = 0; p < split; ++p)
        if (better(ws.bv[r * split + p], ws.bi[r * split + p], bv, bi)) {
          bv = ws.bv[r * split + p];
          bi = ws.bi[r * split + p];
        }
      out[r] = (bi == INT64_MAX) ? 0 : bi;
    }
    return;
  }
  for (int i = threadIdx.x; i < nseg; i += kSegThreads) {
    s_m[i] = ws.m[r * nseg + i];
    s_w[i] = ws.w[r * nseg + i];
  }
  __syncthreads();
  if (wave != 0) return;

  // Phase 2 (one wavefront): segment weights, total and the search.
  float M = -__builtin_inff();
  for (int s = lane; s < nseg; s += 64) M = fmaxf(M, s_m[s]);
  M = group_max<64>(M);
  const int R = (nseg + 63) / 64;
  const int g0 = min(nseg, lane * R), g1 = min(nseg, g0 + R);
  float b = 0.0f;
  for (int s = g0; s < g1; ++s) {
    const float w = s_w[s] * exp2_det((s_m[s] - M) * c);
    s_w[s] = w;  // each lane owns its own segments
    b = b + w;
  }
  const float B = wave_scan_hs(b, lane);
  const float S = __shfl(B, 63);
  if (!(S > 0.0f)) {
    if (lane == 0) out[r] = 0;
    return;
  }
  const float u = uniform[r];
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
    for (int s = t0; s < t1; ++s) {
      const float w = s_w[s];
      const float nxt = acc + w;
      if (nxt > target) { sstar = s; base = acc; break; }
      acc = nxt;
    }
    if (sstar < 0) {
      acc = base_k;
      for (int s = t0; s < t1; ++s) {
        const float w = s_w[s];
        if (w > 0.0f) { sstar = s; base = acc; }
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
// Segments per workgroup of the first kernel (LV_SAMPLER_SPW = 4, 8, 16,
// 32: a tuning knob; 16 measured best on config 4).
static inline int samp_spw() {
  static const int v = [] {
    const char* e = getenv("LV_SAMPLER_SPW");
    const int x = e ? atoi(e) : 16;
    return (x == 4 || x == 8 || x == 16 || x == 32) ? x : 16;
  }();
  return v;
}
static inline int64_t samp_split(int nseg) { return (nseg + samp_spw() - 1) / samp_spw(); }
static inline size_t samp_ws_bytes(int64_t rows, int64_t V) {
  const int64_t nseg = (V + kSeg - 1) / kSeg;
  const int64_t split = samp_split((int)nseg);
  return (size_t)rows * (size_t)(split * 16 + nseg * 8) + 256;
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
  const int split = (int)samp_split(nseg);
  SampWs ws;
  ws.bi = (int64_t*)base;
  ws.bv = (float*)(base + (size_t)num_rows * split * 8);
  ws.m = (float*)(base + (size_t)num_rows * split * 12);
  ws.w = ws.m + (size_t)num_rows * nseg;
  const dim3 grid_a((unsigned)num_rows, (unsigned)split), grid_b((unsigned)num_rows);
  const dim3 block(kSegThreads);
#define LV_SEG(TT, U, G)                                                                        \
  hipLaunchKernelGGL((sampler_segments_kernel<TT, U, G>), grid_a, block, 0, st,                 \
                     (const TT*)logits_dev, vocab_size, row_stride, temperature_dev, ws, nseg,   \
                     split, vec)
#define LV_SAMPLE_LAUNCH(TT)                                                                    \
  switch (samp_spw()) {                                                                         \
    case 4: LV_SEG(TT, 1, 1); break;                                                            \
    case 8: LV_SEG(TT, 2, 1); break;                                                            \
    case 32: LV_SEG(TT, 4, 2); break;                                                           \
    default: LV_SEG(TT, 4, 1); break;                                                           \
  }                                                                                             \
  hipLaunchKernelGGL(sampler_search_kernel<TT>, grid_b, block, 0, st, (const TT*)logits_dev,    \
                     vocab_size, row_stride, temperature_dev, uniform_dev, ws, nseg, split,      \
                     out_ids_dev, vec)
  switch (dtype) {
    case LV_BF16: LV_SAMPLE_LAUNCH(bf16); break;
    case LV_F16: LV_SAMPLE_LAUNCH(f16); break;
    default: LV_SAMPLE_LAUNCH(float); break;
  }
#undef LV_SAMPLE_LAUNCH
#undef LV_SEG
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
