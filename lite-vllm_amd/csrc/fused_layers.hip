// Fused per-layer elementwise work around the attention and MLP GEMMs.
//
//  * add_rms_norm: optional residual add, then RMSNorm
//      (reference litevllm/models/llama.py:18-27 LlamaRMSNorm.forward and the
//      residual adds of Qwen3DecoderLayer.forward, models/qwen3.py:121-140).
//  * qk_norm_rope_cache: the attention prologue of one layer -- split of the
//      fused q|k|v projection, per-head q/k RMSNorm (qwen3.py:75-77), rotary
//      embedding (layers/rotary_emb.py:92-117, the cos/sin rows of the
//      module's cache), query written out, key and value written into the
//      paged cache at slot_mapping (layers/attention.py:79-84).
//  * silu_mul: silu(gate) * up of the gated MLP (llama.py:30-38).
//
// Rounding follows the reference op by op: every intermediate that the
// reference materialises as a tensor of the model dtype T is rounded to T
// here too (this file is built with -ffp-contract=off, so no product is
// fused into an add).  What cannot match bit for bit is the order of the
// fp32 sum of squares and the rsqrt routine, so the outputs agree with the
// reference within one or two units in the last place of T.
#include "lv_common.h"

namespace lv {

constexpr int kFusedThreads = 256;

// ---------------------------------------------------------------------------
// add_rms_norm: one single-wavefront workgroup per token row (rows spread
// over all CUs); the row stays in registers (NC chunks of 16 bytes per lane).
// ---------------------------------------------------------------------------
template <typename T, int NC>
__global__ __launch_bounds__(64) void add_rms_norm_kernel(
    const T* __restrict__ x, int64_t x_stride, T* __restrict__ residual, int64_t res_stride,
    const T* __restrict__ weight, T* __restrict__ out, int64_t out_stride, int64_t num_tokens,
    int hidden, float eps) {
  constexpr int P = elem<T>::kPer16B;
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int chunks = hidden / P;
  const T* xr = x + row * x_stride;
  T* rr = residual ? residual + row * res_stride : nullptr;
  // every load of the row is issued before the first use: one memory round
  // trip, then the reduction
  uint4 xv[NC], rv[NC], wv[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      xv[j] = load16(xr + c * P);
      if (rr) rv[j] = load16(rr + c * P);
      wv[j] = load16(weight + c * P);
    }
  }
  float v[NC][P];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      elem<T>::unpack(xv[j], v[j]);
      if (rr) {
        float r[P];
        elem<T>::unpack(rv[j], r);
#pragma unroll
        for (int i = 0; i < P; ++i) v[j][i] = round_to<T>(v[j][i] + r[i]);
        store16(rr + c * P, pack16<T>(v[j]));
      }
#pragma unroll
      for (int i = 0; i < P; ++i) ss += v[j][i] * v[j][i];
    }
  }
  ss = group_sum<64>(ss);
  const float inv = rsqrtf(ss / (float)hidden + eps);
  T* orow = out + row * out_stride;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      float w[P], o[P];
      elem<T>::unpack(wv[j], w);
#pragma unroll
      for (int i = 0; i < P; ++i) o[i] = round_to<T>(w[i] * round_to<T>(v[j][i] * inv));
      store16(orow + c * P, pack16<T>(o));
    }
  }
}

// ---------------------------------------------------------------------------
// qk_norm_rope_cache: a group of W = min(D/2, 64) lanes per (token, head
// slot); head slots are [0, H) query heads, [H, H+Hkv) key heads, then
// [H+Hkv, H+2Hkv) value heads.  Lane i of a group owns the rotation pairs
// (i + W*p, i + W*p + D/2), p < D/(2W), so the rotation never crosses lanes
// and a 16-lane..64-lane group reduction gives the per-head sum of squares.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kFusedThreads) void qk_norm_rope_cache_kernel(
    const T* __restrict__ qkv, int64_t qkv_stride, const T* __restrict__ q_norm_w,
    const T* __restrict__ k_norm_w, const T* __restrict__ cos_cache,
    const T* __restrict__ sin_cache, int64_t max_position, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ slots, T* __restrict__ q_out, int64_t q_out_stride,
    T* __restrict__ key_cache, T* __restrict__ value_cache, int64_t num_slots,
    int64_t num_tokens, int num_heads, int num_kv_heads, float eps) {
  constexpr int HALF = D / 2;
  constexpr int W = HALF < 64 ? HALF : 64;
  constexpr int PPL = HALF / W;  // rotation pairs per lane
  const int slots_per_token = num_heads + 2 * num_kv_heads;
  const int lane_in_group = threadIdx.x & (W - 1);
  const int64_t gid = ((int64_t)blockIdx.x * kFusedThreads + threadIdx.x) / W;
  const int64_t t = gid / slots_per_token;
  if (t >= num_tokens) return;  // whole groups leave together (W divides 64)
  const int hs = (int)(gid - t * slots_per_token);
  const T* src = qkv + t * qkv_stride + (int64_t)hs * D;
  // the position and slot loads go first: cos/sin depend on the position,
  // and everything else is independent, so the kernel takes two memory
  // round trips (row, weights, position, slot; then cos/sin)
  const int64_t pos = positions[t];
  const int64_t slot = slots[t];

  // a slot past the cache writes nothing and is reported (by the value
  // head's first lane); slot < 0 is padding
  const bool slot_ok = slot >= 0 && slot < num_slots;
  if (hs >= num_heads + num_kv_heads) {  // value head: plain copy into the cache
    if (slot >= num_slots && lane_in_group == 0) report_device_error(LV_DEVERR_SLOT);
    if (!slot_ok) return;
    T* dst = value_cache + slot * ((int64_t)num_kv_heads * D) +
             (int64_t)(hs - num_heads - num_kv_heads) * D;
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
      const int i = lane_in_group + W * p;
      dst[i] = src[i];
      dst[i + HALF] = src[i + HALF];
    }
    return;
  }

  const bool is_q = hs < num_heads;
  if (!is_q && !slot_ok) return;
  const T* nw = is_q ? q_norm_w : k_norm_w;
  float x1[PPL], x2[PPL], w1[PPL], w2[PPL];
#pragma unroll
  for (int p = 0; p < PPL; ++p) {
    const int i = lane_in_group + W * p;
    x1[p] = elem<T>::load(src + i);
    x2[p] = elem<T>::load(src + i + HALF);
    w1[p] = nw ? elem<T>::load(nw + i) : 0.f;
    w2[p] = nw ? elem<T>::load(nw + i + HALF) : 0.f;
  }
  // an out-of-range position has no cos/sin row: the output becomes NaN
  const bool pos_ok = pos >= 0 && pos < max_position;
  float cs[PPL], sn[PPL];
#pragma unroll
  for (int p = 0; p < PPL; ++p) {
    const int i = lane_in_group + W * p;
    cs[p] = pos_ok ? elem<T>::load(cos_cache + pos * HALF + i) : __builtin_nanf("");
    sn[p] = pos_ok ? elem<T>::load(sin_cache + pos * HALF + i) : __builtin_nanf("");
  }
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < PPL; ++p) ss += x1[p] * x1[p] + x2[p] * x2[p];
    ss = group_sum<W>(ss);
    const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
      x1[p] = round_to<T>(w1[p] * round_to<T>(x1[p] * inv));
      x2[p] = round_to<T>(w2[p] * round_to<T>(x2[p] * inv));
    }
  }
  T* dst = is_q ? q_out + t * q_out_stride + (int64_t)hs * D
                : key_cache + slot * ((int64_t)num_kv_heads * D) + (int64_t)(hs - num_heads) * D;
#pragma unroll
  for (int p = 0; p < PPL; ++p) {
    const int i = lane_in_group + W * p;
    const float o1 = round_to<T>(round_to<T>(x1[p] * cs[p]) - round_to<T>(x2[p] * sn[p]));
    const float o2 = round_to<T>(round_to<T>(x2[p] * cs[p]) + round_to<T>(x1[p] * sn[p]));
    elem<T>::store(dst + i, o1);
    elem<T>::store(dst + i + HALF, o2);
  }
}

// ---------------------------------------------------------------------------
// silu_mul: out[t, i] = silu(gate[t, i]) * up[t, i], gate|up fused per row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kFusedThreads) void silu_mul_kernel(
    const T* __restrict__ gate_up, int64_t in_stride, T* __restrict__ out, int64_t out_stride,
    int64_t num_tokens, int inter) {
  constexpr int P = elem<T>::kPer16B;
  const int chunks = inter / P;
  const int64_t total = num_tokens * chunks;
  for (int64_t k = (int64_t)blockIdx.x * kFusedThreads + threadIdx.x; k < total;
       k += (int64_t)gridDim.x * kFusedThreads) {
    const int64_t t = k / chunks;
    const int c = (int)(k - t * chunks);
    const T* row = gate_up + t * in_stride;
    float g[P], u[P], o[P];
    elem<T>::unpack(load16(row + c * P), g);
    elem<T>::unpack(load16(row + inter + c * P), u);
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const float a = round_to<T>(g[i] / (1.0f + expf(-g[i])));
      o[i] = round_to<T>(a * u[i]);
    }
    store16(out + t * out_stride + c * P, pack16<T>(o));
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
template <typename T>
int launch_add_rms_norm(const void* x, int64_t xs, void* res, int64_t rs, const void* w, void* out,
                        int64_t os, int64_t n, int hidden, float eps, hipStream_t st) {
  constexpr int P = elem<T>::kPer16B;
  const int chunks = hidden / P;
  const int nc = (chunks + 63) / 64;
  const dim3 grid((unsigned)n);
  const T* xp = static_cast<const T*>(x);
  T* rp = static_cast<T*>(res);
  const T* wp = static_cast<const T*>(w);
  T* op = static_cast<T*>(out);
#define LV_RMS_CASE(NCV)                                                                     \
  if (nc <= NCV) {                                                                           \
    add_rms_norm_kernel<T, NCV><<<grid, 64, 0, st>>>(xp, xs, rp, rs, wp, op, os, n, hidden,    \
                                                     eps);                                   \
    return check_launch("add_rms_norm_kernel");                                              \
  }
  LV_RMS_CASE(1)
  LV_RMS_CASE(2)
  LV_RMS_CASE(4)
  LV_RMS_CASE(8)
  LV_RMS_CASE(16)
  LV_RMS_CASE(32)
#undef LV_RMS_CASE
  set_error("lv_add_rms_norm: hidden %d too large", hidden);
  return LV_ERR_UNSUPPORTED;
}

template <typename T, int D>
int launch_qk_rope(const void* qkv, int64_t qs, const void* qn, const void* kn, const void* cosc,
                   const void* sinc, int64_t max_pos, const int64_t* pos, const int64_t* slots,
                   void* q_out, int64_t qos, void* kc, void* vc, int64_t num_slots, int64_t n,
                   int H, int Hkv, float eps, hipStream_t st) {
  constexpr int W = (D / 2) < 64 ? (D / 2) : 64;
  const int64_t groups = n * (int64_t)(H + 2 * Hkv);
  const int64_t blocks = (groups * W + kFusedThreads - 1) / kFusedThreads;
  qk_norm_rope_cache_kernel<T, D><<<dim3((unsigned)blocks), kFusedThreads, 0, st>>>(
      static_cast<const T*>(qkv), qs, static_cast<const T*>(qn), static_cast<const T*>(kn),
      static_cast<const T*>(cosc), static_cast<const T*>(sinc), max_pos, pos, slots,
      static_cast<T*>(q_out), qos, static_cast<T*>(kc), static_cast<T*>(vc), num_slots, n, H, Hkv,
      eps);
  return check_launch("qk_norm_rope_cache_kernel");
}

template <typename T>
int dispatch_qk_rope(int D, const void* qkv, int64_t qs, const void* qn, const void* kn,
                     const void* cosc, const void* sinc, int64_t max_pos, const int64_t* pos,
                     const int64_t* slots, void* q_out, int64_t qos, void* kc, void* vc,
                     int64_t num_slots, int64_t n, int H, int Hkv, float eps, hipStream_t st) {
  switch (D) {
    case 64:
      return launch_qk_rope<T, 64>(qkv, qs, qn, kn, cosc, sinc, max_pos, pos, slots, q_out, qos,
                                   kc, vc, num_slots, n, H, Hkv, eps, st);
    case 128:
      return launch_qk_rope<T, 128>(qkv, qs, qn, kn, cosc, sinc, max_pos, pos, slots, q_out, qos,
                                    kc, vc, num_slots, n, H, Hkv, eps, st);
    case 256:
      return launch_qk_rope<T, 256>(qkv, qs, qn, kn, cosc, sinc, max_pos, pos, slots, q_out, qos,
                                    kc, vc, num_slots, n, H, Hkv, eps, st);
    default:
      set_error("lv_qk_norm_rope_cache: head_dim %d not supported (64, 128, 256)", D);
      return LV_ERR_UNSUPPORTED;
  }
}

template <typename T>
int launch_silu_mul(const void* in, int64_t is, void* out, int64_t os, int64_t n, int inter,
                    hipStream_t st) {
  constexpr int P = elem<T>::kPer16B;
  const int64_t total = n * (inter / P);
  int64_t blocks = (total + kFusedThreads - 1) / kFusedThreads;
  if (blocks > 65536) blocks = 65536;
  silu_mul_kernel<T><<<dim3((unsigned)blocks), kFusedThreads, 0, st>>>(
      static_cast<const T*>(in), is, static_cast<T*>(out), os, n, inter);
  return check_launch("silu_mul_kernel");
}

inline bool rows_aligned(const void* p, int64_t stride_elems, size_t esize) {
  return aligned16(p) && ((stride_elems * (int64_t)esize) & 15) == 0;
}

LV_ERROR_WORD_READER(read_errors_fused)

}  // namespace lv

extern "C" int lv_add_rms_norm(const void* x_dev, int64_t x_stride_t, void* residual_dev,
                               int64_t residual_stride_t, const void* weight_dev, void* out_dev,
                               int64_t out_stride_t, int64_t num_tokens, int32_t hidden,
                               float eps, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16, "lv_add_rms_norm: bad dtype");
  LV_REQUIRE(num_tokens >= 0, "lv_add_rms_norm: negative num_tokens");
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(x_dev && weight_dev && out_dev, "lv_add_rms_norm: null pointer");
  const size_t es = dtype_size(dtype);
  const int per16 = (int)(16 / es);
  LV_REQUIRE(hidden > 0 && hidden % per16 == 0,
             "lv_add_rms_norm: hidden %d must be a positive multiple of %d", hidden, per16);
  LV_REQUIRE(x_stride_t >= hidden && out_stride_t >= hidden &&
                 (!residual_dev || residual_stride_t >= hidden),
             "lv_add_rms_norm: row stride smaller than hidden");
  LV_REQUIRE(rows_aligned(x_dev, x_stride_t, es) && rows_aligned(out_dev, out_stride_t, es) &&
                 aligned16(weight_dev) &&
                 (!residual_dev || rows_aligned(residual_dev, residual_stride_t, es)),
             "lv_add_rms_norm: rows must start on 16-byte boundaries");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LV_F32:
      return launch_add_rms_norm<float>(x_dev, x_stride_t, residual_dev, residual_stride_t,
                                        weight_dev, out_dev, out_stride_t, num_tokens, hidden, eps,
                                        st);
    case LV_F16:
      return launch_add_rms_norm<f16>(x_dev, x_stride_t, residual_dev, residual_stride_t,
                                      weight_dev, out_dev, out_stride_t, num_tokens, hidden, eps,
                                      st);
    default:
      return launch_add_rms_norm<bf16>(x_dev, x_stride_t, residual_dev, residual_stride_t,
                                       weight_dev, out_dev, out_stride_t, num_tokens, hidden, eps,
                                       st);
  }
}

extern "C" int lv_qk_norm_rope_cache(
    const void* qkv_dev, int64_t qkv_stride_t, const void* q_norm_weight_dev,
    const void* k_norm_weight_dev, const void* cos_dev, const void* sin_dev,
    int64_t max_position, const int64_t* positions_dev, const int64_t* slot_mapping_dev,
    void* q_out_dev, int64_t q_out_stride_t, void* key_cache_dev, void* value_cache_dev,
    int64_t num_blocks, int32_t block_size, int64_t num_tokens, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, float eps, lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16,
             "lv_qk_norm_rope_cache: bad dtype");
  LV_REQUIRE(num_tokens >= 0, "lv_qk_norm_rope_cache: negative num_tokens");
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(qkv_dev && cos_dev && sin_dev && positions_dev && slot_mapping_dev && q_out_dev &&
                 key_cache_dev && value_cache_dev,
             "lv_qk_norm_rope_cache: null pointer");
  LV_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "lv_qk_norm_rope_cache: bad head counts %d / %d", num_heads, num_kv_heads);
  LV_REQUIRE(num_blocks > 0 && block_size > 0 && max_position > 0,
             "lv_qk_norm_rope_cache: bad cache geometry");
  LV_REQUIRE(qkv_stride_t >= (int64_t)(num_heads + 2 * num_kv_heads) * head_dim &&
                 q_out_stride_t >= (int64_t)num_heads * head_dim,
             "lv_qk_norm_rope_cache: row stride too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t num_slots = num_blocks * block_size;
  switch (dtype) {
    case LV_F32:
      return dispatch_qk_rope<float>(head_dim, qkv_dev, qkv_stride_t, q_norm_weight_dev,
                                     k_norm_weight_dev, cos_dev, sin_dev, max_position,
                                     positions_dev, slot_mapping_dev, q_out_dev, q_out_stride_t,
                                     key_cache_dev, value_cache_dev, num_slots, num_tokens,
                                     num_heads, num_kv_heads, eps, st);
    case LV_F16:
      return dispatch_qk_rope<f16>(head_dim, qkv_dev, qkv_stride_t, q_norm_weight_dev,
                                   k_norm_weight_dev, cos_dev, sin_dev, max_position,
                                   positions_dev, slot_mapping_dev, q_out_dev, q_out_stride_t,
                                   key_cache_dev, value_cache_dev, num_slots, num_tokens,
                                   num_heads, num_kv_heads, eps, st);
    default:
      return dispatch_qk_rope<bf16>(head_dim, qkv_dev, qkv_stride_t, q_norm_weight_dev,
                                    k_norm_weight_dev, cos_dev, sin_dev, max_position,
                                    positions_dev, slot_mapping_dev, q_out_dev, q_out_stride_t,
                                    key_cache_dev, value_cache_dev, num_slots, num_tokens,
                                    num_heads, num_kv_heads, eps, st);
  }
}

extern "C" int lv_silu_mul(const void* gate_up_dev, int64_t in_stride_t, void* out_dev,
                           int64_t out_stride_t, int64_t num_tokens, int32_t intermediate,
                           lv_dtype dtype, void* stream) {
  using namespace lv;
  clear_error();
  LV_REQUIRE(dtype == LV_F32 || dtype == LV_F16 || dtype == LV_BF16, "lv_silu_mul: bad dtype");
  LV_REQUIRE(num_tokens >= 0, "lv_silu_mul: negative num_tokens");
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(gate_up_dev && out_dev, "lv_silu_mul: null pointer");
  const size_t es = dtype_size(dtype);
  const int per16 = (int)(16 / es);
  LV_REQUIRE(intermediate > 0 && intermediate % per16 == 0,
             "lv_silu_mul: intermediate %d must be a positive multiple of %d", intermediate, per16);
  LV_REQUIRE(in_stride_t >= 2 * (int64_t)intermediate && out_stride_t >= intermediate,
             "lv_silu_mul: row stride too small");
  LV_REQUIRE(rows_aligned(gate_up_dev, in_stride_t, es) && rows_aligned(out_dev, out_stride_t, es),
             "lv_silu_mul: rows must start on 16-byte boundaries");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LV_F32:
      return launch_silu_mul<float>(gate_up_dev, in_stride_t, out_dev, out_stride_t, num_tokens,
                                    intermediate, st);
    case LV_F16:
      return launch_silu_mul<f16>(gate_up_dev, in_stride_t, out_dev, out_stride_t, num_tokens,
                                  intermediate, st);
    default:
      return launch_silu_mul<bf16>(gate_up_dev, in_stride_t, out_dev, out_stride_t, num_tokens,
                                   intermediate, st);
  }
}
