// Shared helpers for the gfx950 hot-path kernels: element types, 16-byte
// vector access, wavefront reductions and host-side error reporting.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "litevllm_hip.h"

namespace lv {

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local, see lv_last_error()).
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Checks the launch that was just enqueued; returns LV_OK or LV_ERR_HIP.
int check_launch(const char* what);

#define LV_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      ::lv::set_error(__VA_ARGS__);    \
      return LV_ERR_INVALID;           \
    }                                  \
  } while (0)

// XCDs of an MI355X: workgroups are dispatched round-robin over them, and
// each XCD has its own L2.
constexpr int kXcds = 8;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t dtype_size(lv_dtype dt) { return dt == LV_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Element types.  Storage is raw bits; arithmetic is always fp32.
// ---------------------------------------------------------------------------
struct bf16 { uint16_t bits; };
struct f16 { uint16_t bits; };

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
  return __uint_as_float(b << 16);
}
// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_bits_to_float(uint32_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
  return (float)h;
}
__device__ __forceinline__ uint16_t float_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

template <typename T> struct elem;
template <> struct elem<float> {
  static constexpr int kBytes = 4;
  static constexpr int kPer16B = 4;
  __device__ __forceinline__ static void unpack(const uint4& v, float* out) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  }
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct elem<bf16> {
  static constexpr int kBytes = 2;
  static constexpr int kPer16B = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static float load(const bf16* p) { return bf16_bits_to_float(p->bits); }
  __device__ __forceinline__ static void store(bf16* p, float v) { p->bits = float_to_bf16_bits(v); }
};
template <> struct elem<f16> {
  static constexpr int kBytes = 2;
  static constexpr int kPer16B = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = f16_bits_to_float(w[i] & 0xffffu);
      out[2 * i + 1] = f16_bits_to_float(w[i] >> 16);
    }
  }
  __device__ __forceinline__ static float load(const f16* p) { return f16_bits_to_float(p->bits); }
  __device__ __forceinline__ static void store(f16* p, float v) { p->bits = float_to_f16_bits(v); }
};

// Value after a store to T and a reload (fp32 arithmetic rounded to the
// storage type, the way a torch op with a T-typed output rounds).
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<bf16>(float v) {
  return bf16_bits_to_float(float_to_bf16_bits(v));
}
template <> __device__ __forceinline__ float round_to<f16>(float v) {
  return f16_bits_to_float(float_to_f16_bits(v));
}

// Pack kPer16B fp32 values (already representable in T) into 16 bytes.
template <typename T> __device__ __forceinline__ uint4 pack16(const float* v);
template <> __device__ __forceinline__ uint4 pack16<float>(const float* v) {
  return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                    __float_as_uint(v[3]));
}
template <> __device__ __forceinline__ uint4 pack16<bf16>(const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)float_to_bf16_bits(v[2 * i]) | ((uint32_t)float_to_bf16_bits(v[2 * i + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <> __device__ __forceinline__ uint4 pack16<f16>(const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)float_to_f16_bits(v[2 * i]) | ((uint32_t)float_to_f16_bits(v[2 * i + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// Streaming 16-byte load (non-temporal hint: data read once, not cached for
// reuse).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store16(void* p, const uint4& v) {
  *reinterpret_cast<uint4*>(p) = v;
}

// ---------------------------------------------------------------------------
// Cross-lane helpers.  DPP row operations act on rows of 16 lanes.
// dpp control codes: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141 (lane i <-> 7-i in each 8-lane half row),
// row_mirror = 0x140 (lane i <-> 15-i in each row).  Each step pairs lanes
// symmetrically, so every lane of a group ends with the bit-identical total.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xf, 0xf, false);
}

// Sum over aligned groups of W lanes (W in 1,2,4,...,64); every lane of the
// group receives the same total.
template <int W>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (W >= 2) x += dpp<0xB1>(x);
  if constexpr (W >= 4) x += dpp<0x4E>(x);
  if constexpr (W >= 8) x += dpp<0x141>(x);
  if constexpr (W >= 16) x += dpp<0x140>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16);
  if constexpr (W >= 64) x += __shfl_xor(x, 32);
  return x;
}

template <int W>
__device__ __forceinline__ float group_max(float x) {
  if constexpr (W >= 2) x = fmaxf(x, dpp<0xB1>(x));
  if constexpr (W >= 4) x = fmaxf(x, dpp<0x4E>(x));
  if constexpr (W >= 8) x = fmaxf(x, dpp<0x141>(x));
  if constexpr (W >= 16) x = fmaxf(x, dpp<0x140>(x));
  if constexpr (W >= 32) x = fmaxf(x, __shfl_xor(x, 16));
  if constexpr (W >= 64) x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// Device-side report of out-of-range indices.  A kernel that meets one
// clamps it (no access leaves its buffer) and raises a bit (LV_DEVERR_*) in
// the error word of its translation unit.  Device code is not linked across
// units, so every unit has a word of its own per device; the unit's reader
// (defined with LV_ERROR_WORD_READER) copies it out and lv_device_errors()
// ORs the readers' results.
// ---------------------------------------------------------------------------
namespace {
__device__ uint32_t tu_error_word = 0;
}
__device__ __forceinline__ void report_device_error(uint32_t bit) {
  __hip_atomic_fetch_or(&tu_error_word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Readers of the units that report (the caller has synchronised the device).
int read_errors_scatter(uint32_t* bits, bool clear);
int read_errors_attention(uint32_t* bits, bool clear);
int read_errors_fused(uint32_t* bits, bool clear);

#define LV_ERROR_WORD_READER(NAME)                                                        \
  int NAME(uint32_t* bits, bool clear) {                                                   \
    hipError_t e = hipMemcpyFromSymbol(bits, HIP_SYMBOL(tu_error_word), sizeof(uint32_t), 0, \
                                       hipMemcpyDeviceToHost);                             \
    if (e == hipSuccess && clear) {                                                        \
      const uint32_t zero = 0;                                                             \
      e = hipMemcpyToSymbol(HIP_SYMBOL(tu_error_word), &zero, sizeof(uint32_t), 0,         \
                            hipMemcpyHostToDevice);                                        \
    }                                                                                      \
    if (e != hipSuccess) {                                                                 \
      set_error(#NAME ": %s", hipGetErrorString(e));                                       \
      return LV_ERR_HIP;                                                                   \
    }                                                                                      \
    return LV_OK;                                                                          \
  }

}  // namespace lv
