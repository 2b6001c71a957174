// Linear layers of small-batch (decode) steps on the matrix cores:
//
//   plain     y[m, n] = sum_k x[m, k] w[n, k]                 (nn.Linear, no bias)
//   silu_mul  y[m, n] = to_T(to_T(silu(to_T(g))) * to_T(u))    (gated MLP)
//             g = sum_k x[m, k] w[n, k],  u = sum_k x[m, k] w[N + n, k]
//
// Reference: ColumnParallelLinear / RowParallelLinear, plain nn.Linear on one
// GPU (layers/linear.py:15-65), used for the qkv, o, gate/up and down
// projections (models/qwen3.py:45-48, models/llama.py:33-35, 58-61), and
// F.silu(gate) * up (llama.py:38).
//
// A decode step is skinny: M (sequences) <= 512 against N, K of 1024 to
// 151936, and the weights (N x K) are the bytes that matter.  A workgroup of
// four wavefronts computes a TM x TN tile of y^T with v_mfma_f32_32x32x16:
// weight rows are the A operand (32 n x 16 k), x rows the B operand (16 k x
// 32 m), so the fp32 accumulator holds, per lane, one x row and four runs of
// 4 consecutive n -- each run is one 8-byte store.
//   * Staging: per batch of 128 k, the tile's weight rows and x rows
//     (256 B each) go from global memory straight into LDS
//     (global_load_lds_dwordx4; one instruction fills 4 whole rows, i.e.
//     whole cache lines), 16-byte chunks XOR-swizzled by row so that the
//     MFMA-layout reads (32 rows at one chunk) hit distinct banks.  Three
//     stages: two batches are in flight while the third is computed.
//   * Compute: every wavefront works on the whole tile for a quarter of each
//     batch's k (2 MFMA k-steps); the four partial tiles are summed through
//     LDS in a fixed order at the end, each wavefront finishing some of the
//     32 x 32 blocks.
//   * Tiles are numbered so that all m tiles of one n tile run on one XCD
//     (workgroups are dispatched round-robin over the 8 XCDs): the weight
//     tile is read from HBM once and re-read from that XCD's L2.
//
// Rounding: y is the fp32 sum rounded once to T, as a library GEMM with
// fp32 accumulation.  Every tile shape sums k in the same order (the same
// k slice per wavefront, the same slice order in the final sum), so the
// silu_mul form sees exactly the g and u the plain form would store, and
// then rounds like silu_mul_kernel (this file is built with
// -ffp-contract=off).
#include "lv_common.h"
#include "lv_mfma.h"

namespace lv {

constexpr int kLinK = 128;                 // k per staged batch (256 B per row)
constexpr int kLinCpr = kLinK / 8;         // 16-byte chunks per staged row
constexpr int kLinWaves = 4;               // wavefronts per workgroup = k slices per batch
constexpr int kLinRowsPerLoad = 1024 / (2 * kLinK);   // rows filled by one 64-lane DMA load

// Element offset of 16-byte chunk `chunk` of staged row `row`.
__device__ __forceinline__ int lin_at(int row, int chunk) {
  return row * kLinK + 8 * (chunk ^ (row & (kLinCpr - 1)));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
  // vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8 left at their maxima)
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 16 bytes per lane from global memory into LDS at wave base + 16 lane
// (global_load_lds_dwordx4), issued from inline assembly so that the
// compiler does not track it: its own tracking of loads into LDS across the
// staging loop's back edge waits for all of them before the first LDS read
// of each iteration.  The loads a batch needs are waited for with
// wait_vmcnt before that batch's barrier.
// lds_wave_base is an LDS byte address, the same in every lane.  M0 is
// written here and nowhere else in this file's kernels (no other
// instruction of theirs reads it).
__device__ __forceinline__ void load_lds16_async(const void* g, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
               "s"(lds_wave_base)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Workgroup barrier without the memory fence of __syncthreads: the fence
// waits for every outstanding load into LDS, which would drain the staging
// pipeline at each batch.  The loads a batch depends on are waited for
// explicitly (wait_vmcnt) before the barrier, and each wavefront's LDS reads
// of the previous batch have completed because the MFMAs consumed them; the
// "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <typename T>
__device__ __forceinline__ float silu_round(float g) {
  return round_to<T>(g / (1.0f + expf(-g)));
}

template <typename T, int TM, int TN, int NS, bool SILU>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(
    const T* __restrict__ x, int64_t x_stride, const T* __restrict__ w, int64_t w_stride,
    T* __restrict__ y, int64_t y_stride, int M, int N, int K, int m_tiles, int n_tiles) {
  using Mf = Mfma32<T>;
  using v8 = typename Mf::v8;
  constexpr int NA = SILU ? 2 : 1;            // weight row sets (gate, up)
  constexpr int MB = TM / 32, NB = TN / 32;   // 32 x 32 blocks of the tile
  constexpr int WR = NA * TN;                 // staged weight rows
  constexpr int R = WR + TM;                  // staged rows per batch
  constexpr int STAGE = R * kLinK;            // elements per stage
  constexpr int NI = R / kLinRowsPerLoad / kLinWaves;   // DMA loads per wavefront per batch
  static_assert(R % (kLinRowsPerLoad * kLinWaves) == 0, "rows per stage");
  constexpr int JS = kLinK / kLinWaves / 16;  // MFMA k-steps per wavefront per batch
  constexpr int NQ = NB * MB;                 // 32 x 32 output blocks (NA accumulators each)
  static_assert(2 * NQ * NA * 16 * 64 * 4 <= STAGE * 2, "reduction fits two stages");
  static_assert(NS >= 2 && NS <= 4, "stages");
  __shared__ __attribute__((aligned(16))) uint16_t S[NS * STAGE];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wg = blockIdx.x, slot = wg / kXcds;
  const int nt = (slot / m_tiles) * kXcds + wg % kXcds;
  const int mt = slot % m_tiles;
  if (nt >= n_tiles) return;                  // padding of the XCD-ordered grid: whole workgroup
  const int n0 = nt * TN, m0 = mt * TM;
  // LDS byte address of this wavefront's first DMA row block in each stage
  const uint32_t wofs = (uint32_t)(wave * NI * kLinRowsPerLoad * kLinK * 2);
  const uint32_t L0 = __builtin_amdgcn_readfirstlane(lds_address(S)) + wofs;

  // DMA sources: load i of this wavefront fills staged rows 4 (wave NI + i) .. +3;
  // the lane's 16 bytes land in chunk slot lane % 16 of row 4 (...) + lane / 16,
  // which holds logical chunk slot ^ (row % 16).
  const T* src[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (wave * NI + i) * kLinRowsPerLoad + lane / kLinCpr;
    const int chunk = (lane % kLinCpr) ^ (row & (kLinCpr - 1));
    const T* base;
    if (row < TN) base = w + (int64_t)(n0 + row) * w_stride;
    else if (SILU && row < WR) base = w + (int64_t)(N + n0 + row - TN) * w_stride;
    else base = x + (int64_t)min(m0 + row - WR, M - 1) * x_stride;  // rows >= M: not stored
    src[i] = base + 8 * chunk;
  }
  auto stage = [&](uint32_t dst, int k0) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      load_lds16_async(src[i] + k0, dst + (uint32_t)(i * kLinRowsPerLoad * kLinK * 2));
  };

  f32x16_t acc[NA][NB][MB];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[a][nb][mb] = f32x16_t{};
  const int r32 = lane & 31;
  auto compute = [&](const uint16_t* S) {
#pragma unroll
    for (int j = 0; j < JS; ++j) {
      const int chunk = (wave * JS + j) * 2 + (lane >> 5);
      v8 af[NA][NB], bf[MB];
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          af[a][nb] = __builtin_bit_cast(
              v8, *reinterpret_cast<const uint4*>(S + lin_at(a * TN + nb * 32 + r32, chunk)));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        bf[mb] = __builtin_bit_cast(
            v8, *reinterpret_cast<const uint4*>(S + lin_at(WR + mb * 32 + r32, chunk)));
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[a][nb][mb] = Mf::run(af[a][nb], bf[mb], acc[a][nb][mb]);
    }
  };
  // batch b lives in stage b % NS; before computing it, its loads have
  // landed (only the loads of the next NS - 2 batches may be outstanding)
  // and every wavefront is done with batch b - 1, whose stage then takes
  // batch b + NS - 1
  const int nbat = K / kLinK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nbat) stage(L0 + (uint32_t)(s * STAGE * 2), s * kLinK);
  int cur = 0;   // b % NS
  for (int b = 0; b < nbat; ++b) {
    const int pending = min(NS - 2, nbat - 1 - b);   // batches loaded after b
    if (pending >= 2) wait_vmcnt<2 * NI>();
    else if (pending == 1) wait_vmcnt<NI>();
    else wait_vmcnt<0>();
    lds_barrier();
    const int prev = cur == 0 ? NS - 1 : cur - 1;    // (b + NS - 1) % NS
    if (b + NS - 1 < nbat) stage(L0 + (uint32_t)(prev * STAGE * 2), (b + NS - 1) * kLinK);
    compute(S + cur * STAGE);
    cur = cur == NS - 1 ? 0 : cur + 1;
  }

  // Sum the four k slices: partial block q (accumulator a) of wavefront v
  // goes to stage v / 2 at float offset (((v % 2) NQ + q) NA + a) 1024; the
  // final sums run over v = 0..3 in order.
  __syncthreads();
  {
    float* red = reinterpret_cast<float*>(S + (wave / 2) * STAGE) + (wave % 2) * NQ * NA * 1024;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            red[((nb * MB + mb) * NA + a) * 1024 + e * 64 + lane] = acc[a][nb][mb][e];
  }
  __syncthreads();
  // Each block's 16 accumulator elements per lane are 4 runs of 4 outputs;
  // with fewer blocks than wavefronts the runs are shared out, so every
  // wavefront takes part in the final sum and the epilogue.
  constexpr int SPLIT = NQ >= kLinWaves ? 1 : kLinWaves / NQ;   // wavefronts per block
  constexpr int RUNS = 4 / SPLIT;                                // runs per wavefront
  static_assert(NQ * SPLIT == kLinWaves || NQ % kLinWaves == 0, "blocks per wavefront");
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int part = 0; part < SPLIT; ++part) {
      if ((q * SPLIT + part) % kLinWaves != wave) continue;
      const int nb = q / MB, mb = q % MB;
      const int m = m0 + mb * 32 + r32;
      float sum[NA][4 * RUNS];
#pragma unroll
      for (int v = 0; v < kLinWaves; ++v) {
        const float* red =
            reinterpret_cast<const float*>(S + (v / 2) * STAGE) + (v % 2) * NQ * NA * 1024;
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int i = 0; i < 4 * RUNS; ++i) {
            const int e = 4 * RUNS * part + i;
            const float p = red[(q * NA + a) * 1024 + e * 64 + lane];
            sum[a][i] = v == 0 ? p : sum[a][i] + p;
          }
      }
      if (m >= M) continue;
      T* yr = y + (int64_t)m * y_stride + n0 + nb * 32 + 4 * (lane >> 5);
#pragma unroll
      for (int r = 0; r < RUNS; ++r) {
        const int g = RUNS * part + r;   // run g: outputs n = 8 g + 4 (lane / 32) + 0..3
        float v4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (SILU) {
            const float gt = round_to<T>(sum[0][4 * r + e]);
            const float up = round_to<T>(sum[1][4 * r + e]);
            v4[e] = round_to<T>(silu_round<T>(gt) * up);
          } else {
            v4[e] = sum[0][4 * r + e];
          }
        }
        *reinterpret_cast<uint2*>(yr + 8 * g) =
            make_uint2(Mf::pack2(v4[0], v4[1]), Mf::pack2(v4[2], v4[3]));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.  Configurations (tile TM x TN, NS stages, LDS per workgroup):
//   0: 64 x 64, 3 stages (96 KB)    1: 64 x 64, 2 stages (64 KB, 2 per CU)
//   2: 32 x 32, 4 stages (64 KB)    3: 32 x 64, 4 stages (96 KB)
// Measured on decode shapes (M 64..256, N 1024..6144, K 1024..3072): 64 x 64
// tiles when they make about one workgroup per CU, 2-stage ones when they
// make more (two resident per CU cover the second round), else the narrower
// tiles.  LV_LINEAR_CFG forces one.
// ---------------------------------------------------------------------------
struct LinCfg { int tm, tn; };
constexpr LinCfg kLinCfgs[] = {{64, 64}, {64, 64}, {32, 32}, {32, 64}};
constexpr int kLinNumCfgs = 4;

// silu_mul: tiles of 64 x 32 outputs (64 staged weight rows: 32 gate, 32 up),
// 2 stages (64 KB, two workgroups per CU) or 3 stages (96 KB) when the grid
// fits one round.
static int lin_pick_silu(int64_t m, int64_t n, int64_t k) {
  if (k % kLinK != 0 || n % 32 != 0) return -1;
  if (const char* e = getenv("LV_LINEAR_SILU_CFG")) {
    const int i = atoi(e);
    if (i == 0 || i == 1) return i;
  }
  return ((m + 63) / 64) * (n / 32) > 256 ? 1 : 0;
}

static int lin_pick(int64_t m, int64_t n, int64_t k) {
  if (k % kLinK != 0 || n % 32 != 0) return -1;
  auto fits = [&](int i) { return n % kLinCfgs[i].tn == 0; };
  auto wgs = [&](int i) { return ((m + kLinCfgs[i].tm - 1) / kLinCfgs[i].tm) * (n / kLinCfgs[i].tn); };
  if (const char* e = getenv("LV_LINEAR_CFG")) {
    const int i = atoi(e);
    if (i >= 0 && i < kLinNumCfgs && fits(i)) return i;
  }
  if (fits(0) && wgs(0) > 256) return 1;
  if (fits(0) && wgs(0) >= 200) return 0;
  if (fits(3) && wgs(3) >= 160) return 3;
  return 2;
}

template <typename T, int TM, int TN, int NS, bool SILU>
static int launch_lin(const void* x, int64_t xs, const void* w, int64_t ws, void* y, int64_t ys,
                      int m, int n, int k, hipStream_t st) {
  const int m_tiles = (m + TM - 1) / TM;
  const int n_tiles = n / TN;
  const int64_t grid = (int64_t)(n_tiles + kXcds - 1) / kXcds * kXcds * m_tiles;
  if (grid > 0x7fffffff) {
    set_error("lv_linear: grid of %lld workgroups", (long long)grid);
    return LV_ERR_INVALID;
  }
  hipLaunchKernelGGL((linear_kernel<T, TM, TN, NS, SILU>), dim3((unsigned)grid),
                     dim3(64 * kLinWaves), 0, st, static_cast<const T*>(x), xs,
                     static_cast<const T*>(w), ws, static_cast<T*>(y), ys, m, n, k, m_tiles,
                     n_tiles);
  return check_launch("linear_kernel");
}

template <typename T>
static int dispatch_lin(bool silu, int cfg, const void* x, int64_t xs, const void* w, int64_t ws,
                        void* y, int64_t ys, int m, int n, int k, hipStream_t st) {
  if (silu)
    return cfg == 1 ? launch_lin<T, 64, 32, 2, true>(x, xs, w, ws, y, ys, m, n, k, st)
                    : launch_lin<T, 64, 32, 3, true>(x, xs, w, ws, y, ys, m, n, k, st);
  switch (cfg) {
    case 0: return launch_lin<T, 64, 64, 3, false>(x, xs, w, ws, y, ys, m, n, k, st);
    case 1: return launch_lin<T, 64, 64, 2, false>(x, xs, w, ws, y, ys, m, n, k, st);
    case 2: return launch_lin<T, 32, 32, 4, false>(x, xs, w, ws, y, ys, m, n, k, st);
    default: return launch_lin<T, 32, 64, 4, false>(x, xs, w, ws, y, ys, m, n, k, st);
  }
}

}  // namespace lv

extern "C" int lv_linear_supported(int64_t m, int64_t n, int64_t k, int32_t activation,
                                   lv_dtype dtype) {
  using namespace lv;
  if (dtype != LV_BF16 && dtype != LV_F16) return 0;
  if (activation != LV_ACT_NONE && activation != LV_ACT_SILU_MUL) return 0;
  if (m < 1 || m > 0x7fffffff || n < 1 || n > 0x3fffffff || k < 1 || k > 0x7fffffff) return 0;
  return (activation == LV_ACT_SILU_MUL ? lin_pick_silu(m, n, k) : lin_pick(m, n, k)) >= 0;
}

extern "C" int lv_linear(const void* x_dev, int64_t x_stride_t, const void* weight_dev,
                         int64_t weight_stride_n, void* y_dev, int64_t y_stride_t, int64_t m,
                         int64_t n, int64_t k, int32_t activation, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_BF16 || dtype == LV_F16 || dtype == LV_F32, "lv_linear: bad dtype");
  LV_REQUIRE(activation == LV_ACT_NONE || activation == LV_ACT_SILU_MUL,
             "lv_linear: bad activation %d", activation);
  LV_REQUIRE(m >= 0 && m <= 0x7fffffff && n >= 1 && n <= 0x3fffffff && k >= 1 &&
                 k <= 0x7fffffff, "lv_linear: bad shape m=%lld n=%lld k=%lld", (long long)m,
             (long long)n, (long long)k);
  if (m == 0) return LV_OK;
  LV_REQUIRE(x_dev && weight_dev && y_dev, "lv_linear: null pointer");
  LV_REQUIRE(x_stride_t >= k && weight_stride_n >= k && y_stride_t >= n,
             "lv_linear: a row stride is shorter than its row");
  LV_REQUIRE(aligned16(x_dev) && aligned16(weight_dev) && x_stride_t % 8 == 0 &&
                 weight_stride_n % 8 == 0, "lv_linear: x and weight rows must be 16-byte aligned");
  LV_REQUIRE(((uintptr_t)y_dev & 7u) == 0 && y_stride_t % 4 == 0,
             "lv_linear: y rows must be 8-byte aligned");
  const bool silu = activation == LV_ACT_SILU_MUL;
  const int cfg = (dtype == LV_F32) ? -1 : (silu ? lin_pick_silu(m, n, k) : lin_pick(m, n, k));
  if (cfg < 0) {
    set_error("lv_linear: no kernel for dtype %d, n=%lld, k=%lld (n %% 32 and k %% 128 must be 0)",
              (int)dtype, (long long)n, (long long)k);
    return LV_ERR_UNSUPPORTED;
  }
  hipStream_t st = (hipStream_t)stream;
  const int mi = (int)m, ni = (int)n, ki = (int)k;
  if (dtype == LV_BF16)
    return dispatch_lin<bf16>(silu, cfg, x_dev, x_stride_t, weight_dev, weight_stride_n, y_dev,
                              y_stride_t, mi, ni, ki, st);
  return dispatch_lin<f16>(silu, cfg, x_dev, x_stride_t, weight_dev, weight_stride_n, y_dev,
                           y_stride_t, mi, ni, ki, st);
}
