// Shared device/host helpers for the gfx950 paged-attention kernels.
//
// Element-type traits, exact conversions, wavefront reductions and the
// thread-local error string behind mlr_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "mlr_attn.h"

namespace mlr {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------------------
// Error reporting (host side).
// ---------------------------------------------------------------------------
int set_error(int code, const char *fmt, ...);
void clear_error();

#define MLR_REQUIRE(cond, ...)                               \
  do {                                                       \
    if (!(cond)) return ::mlr::set_error(MLR_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// Reports a launch failure (bad grid, missing code object) as MLR_ERR_HIP.
int check_launch(const char *what);

// Compute units of the current device, queried once per device; 0 when the
// query fails.
int current_device_cus();

// ---------------------------------------------------------------------------
// Storage types. bf16 and fp16 are carried as raw 16-bit patterns so that the
// kernels control every rounding step themselves.
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
  return __uint_as_float(b << 16);
}

// fp32 -> bf16 with round-to-nearest-even; every NaN becomes the canonical
// quiet NaN 0x7FC0, which is what Tensor.to(torch.bfloat16) produces.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  // Add 0x7fff plus the lowest kept bit, then truncate: ties go to even.
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_float(uint16_t b) {
  return __half2float(__ushort_as_half(b));
}

// fp32 -> fp16, round-to-nearest-even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t float_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

template <typename T> struct Elem;

template <> struct Elem<float> {
  using storage = float;
  using acc = float;  // dot-product / P@V accumulation type
  static constexpr int kDtype = MLR_DTYPE_F32;
  __device__ static float to_f32(float x) { return x; }
  __device__ static double to_f64(float x) { return x; }
  __device__ static float from_f32(float x) { return x; }
  __device__ static float from_f64(double x) { return static_cast<float>(x); }
  __device__ static float to_acc(float x) { return x; }
  __device__ static float from_acc(float x) { return x; }
  // Round an accumulated value to the element type and back (identity here).
  __device__ static float round_acc(float x) { return x; }
};

template <> struct Elem<double> {
  using storage = double;
  using acc = double;
  static constexpr int kDtype = MLR_DTYPE_F64;
  __device__ static float to_f32(double x) { return static_cast<float>(x); }
  __device__ static double to_f64(double x) { return x; }
  __device__ static double from_f32(float x) { return x; }
  __device__ static double from_f64(double x) { return x; }
  __device__ static double to_acc(double x) { return x; }
  __device__ static double from_acc(double x) { return x; }
  __device__ static double round_acc(double x) { return x; }
};

template <> struct Elem<bf16_t> {
  using storage = bf16_t;
  using acc = float;
  static constexpr int kDtype = MLR_DTYPE_BF16;
  __device__ static float to_f32(bf16_t x) { return bf16_bits_to_float(x.bits); }
  __device__ static double to_f64(bf16_t x) { return bf16_bits_to_float(x.bits); }
  __device__ static bf16_t from_f32(float x) { return bf16_t{float_to_bf16_bits(x)}; }
  // double -> float -> bf16, the two roundings Tensor.to performs.
  __device__ static bf16_t from_f64(double x) {
    return bf16_t{float_to_bf16_bits(static_cast<float>(x))};
  }
  __device__ static float to_acc(bf16_t x) { return to_f32(x); }
  __device__ static bf16_t from_acc(float x) { return from_f32(x); }
  __device__ static float round_acc(float x) {
    return bf16_bits_to_float(float_to_bf16_bits(x));
  }
};

template <> struct Elem<f16_t> {
  using storage = f16_t;
  using acc = float;
  static constexpr int kDtype = MLR_DTYPE_F16;
  __device__ static float to_f32(f16_t x) { return f16_bits_to_float(x.bits); }
  __device__ static double to_f64(f16_t x) { return f16_bits_to_float(x.bits); }
  __device__ static f16_t from_f32(float x) { return f16_t{float_to_f16_bits(x)}; }
  __device__ static f16_t from_f64(double x) {
    return f16_t{float_to_f16_bits(static_cast<float>(x))};
  }
  __device__ static float to_acc(f16_t x) { return to_f32(x); }
  __device__ static f16_t from_acc(float x) { return from_f32(x); }
  __device__ static float round_acc(float x) {
    return f16_bits_to_float(float_to_f16_bits(x));
  }
};

// ---------------------------------------------------------------------------
// Wavefront reductions (64 lanes, butterfly over __shfl_xor).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o));
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

// log2(x) when x is a positive power of two, else -1.
inline int log2_if_pow2(int64_t x) {
  if (x <= 0 || (x & (x - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t(1) << s) < x) ++s;
  return s;
}

inline int dtype_size(int dtype) {
  switch (dtype) {
    case MLR_DTYPE_F32: return 4;
    case MLR_DTYPE_F16: return 2;
    case MLR_DTYPE_BF16: return 2;
    case MLR_DTYPE_F64: return 8;
    default: return 0;
  }
}

}  // namespace mlr
