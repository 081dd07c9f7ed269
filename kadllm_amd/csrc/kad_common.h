// Shared definitions for the kadllm HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/kadllm_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;  // bf16 bit pattern in memory

// ---------------------------------------------------------------------------
// host-side error reporting (thread-local message, returned by kad_last_error)
void kad_set_error(const char* fmt, ...);
int kad_launch_status(const char* what);

#define KAD_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      kad_set_error(__VA_ARGS__);              \
      return KAD_ERR_INVALID_ARGUMENT;         \
    }                                          \
  } while (0)

#define KAD_UNSUPPORTED(...)                   \
  do {                                         \
    kad_set_error(__VA_ARGS__);                \
    return KAD_ERR_UNSUPPORTED;                \
  } while (0)

// ---------------------------------------------------------------------------
// device helpers
__device__ __forceinline__ float bf2f(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ bf16_t f2bf(float f) {
  __bf16 b = (__bf16)f;  // round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
  return __builtin_bit_cast(bf16_t, b);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ __bf16 f2b(float f) { return (__bf16)f; }

// load/store one element of a runtime dtype as float
__device__ __forceinline__ float load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == KAD_DTYPE_F32) return ((const float*)p)[i];
  if (dtype == KAD_DTYPE_BF16) return bf2f(((const bf16_t*)p)[i]);
  return (float)((const _Float16*)p)[i];
}
__device__ __forceinline__ float round_to_dtype(float f, int dtype) {
  if (dtype == KAD_DTYPE_F32) return f;
  if (dtype == KAD_DTYPE_BF16) return round_bf(f);
  return (float)(_Float16)f;
}

// element type traits for templated kernels
template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
  static constexpr int code = KAD_DTYPE_BF16;
  __device__ static __forceinline__ float to_f(bf16_t v) { return bf2f(v); }
  __device__ static __forceinline__ bf16_t from_f(float f) { return f2bf(f); }
};
template <> struct Elem<float> {
  static constexpr int code = KAD_DTYPE_F32;
  __device__ static __forceinline__ float to_f(float v) { return v; }
  __device__ static __forceinline__ float from_f(float f) { return f; }
};
template <> struct Elem<_Float16> {
  static constexpr int code = KAD_DTYPE_F16;
  __device__ static __forceinline__ float to_f(_Float16 v) { return (float)v; }
  __device__ static __forceinline__ _Float16 from_f(float f) { return (_Float16)f; }
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }
// SiLU with the hardware reciprocal (1 ulp) in place of the IEEE divide, for
// the VALU-bound decode kernels; within the tested bf16 tolerance of torch's
// silu once rounded
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) {
  // torch softplus (beta 1, threshold 20)
  return x > 20.0f ? x : log1pf(expf(x));
}

// MFMA wrappers (gfx950)
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

// two floats to a packed bf16 pair, each rounded to nearest even: one
// v_cvt_pk_bf16_f32 for both (a scalar conversion spends one per element)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){a, b}, bf16x2_v));
}

// split 8 floats into bf16 hi/lo parts: x ~= hi + lo with |x-hi-lo| <= 2^-16 |x|;
// the same bits as rounding each element on its own, with a packed
// conversion per pair and the pair's hi parts widened by shift / mask
__device__ __forceinline__ void split8(const float* x, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t hp = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    h[i] = hp;
    l[i] = pack_bf16x2(x[2 * i] - __uint_as_float(hp << 16),
                       x[2 * i + 1] - __uint_as_float(hp & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

// x combined with x of lane ^ 16 or lane ^ 32 by the gfx950 row / half-wave
// swaps (v_permlane16_swap, v_permlane32_swap: VALU, no LDS round trip).  The
// swap of x with itself leaves x and its partner in the two results, so
// their sum (or max) equals x + shfl_xor(x, 16 or 32) bit for bit.
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// wave-level reductions (wave64)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

static inline int64_t kad_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Map a linear workgroup id so that consecutive logical ids land on the same
// XCD (the dispatcher hands workgroup i to XCD i % 8).  Returns the logical id.
__device__ __forceinline__ int xcd_logical_id(int bid, int nblocks) {
  const int nx = 8;
  if (nblocks % nx) return bid;
  return (bid % nx) * (nblocks / nx) + bid / nx;
}
