// The elementwise work of a Qwen2 decoder layer around its attention and
// GEMMs, one launch each where PyTorch issues several:
//
//   mlr_rms_norm:  optional residual add, then RMSNorm (Qwen2RMSNorm, reference
//                  model/qwen2.py:88-123; the residual adds of
//                  Qwen2DecoderLayer, :794-940). PyTorch issues eight kernels
//                  for the norm of a 16-bit tensor and one for the add.
//   mlr_silu_mul:  silu(gate) * up of Qwen2MLP (:768-792) over the output of
//                  one GEMM with the gate and up projections side by side.
//
// Rounding follows the modules' PyTorch operations for each storage type
// (16-bit types keep their statistics in FP32):
//   r    = T(x + residual)                  (the add, when a residual is given)
//   s    = sum_j float(r_j) * float(r_j)    (one row, FP32)
//   var  = s * factor,  factor = float(rows) / float(rows * hidden)
//                                          (the scale torch's mean applies)
//   inv  = rsqrtf(var + float(eps))
//   out  = T(float(w_j) * float(T(float(r_j) * inv)))     (FP32: w_j * (r_j * inv))
//   silu_mul: T(float(T(g / (1 + expf(-g)))) * float(u))
// Only the order of the row sum differs from torch's reduction: each lane adds
// its chunks in order and the wave adds the 64 lane sums by a fixed butterfly,
// so a row's result is the same whether or not the add was fused.
//
// One wave per row, four rows per 256-thread workgroup; 16-byte chunks when
// the row length and every row start allow it, single elements otherwise.
// Rows of at most 256 chunks (2,048 16-bit or 1,024 FP32 elements) stay in
// registers: every chunk of x, the residual and the weight is loaded before
// anything is stored, so a wave makes one memory round trip before its
// reduction instead of three (the loads, the re-read of the summed row, the
// weight). Longer rows loop over their chunks and the second pass re-reads
// the row (from residual_out when the add was fused) from the caches. Both
// kernels are latency-bound at serving sizes (a few rows of 896 elements)
// and bandwidth-bound at prefill sizes.
#include <algorithm>
#include <type_traits>

#include "mlr_common.h"

// Every product and sum is rounded on its own, as PyTorch's separate kernels
// round them: no multiply-add contraction in this file.
#pragma clang fp contract(off)

namespace mlr {
namespace {

template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> { static constexpr int n = 8; };
template <> struct Vec16<f16_t> { static constexpr int n = 8; };
template <> struct Vec16<float> { static constexpr int n = 4; };

template <typename T, int N>
struct alignas(sizeof(T) * N) Chunk {
  T v[N];
};

template <typename T, int N>
__global__ __launch_bounds__(256) void rms_norm_kernel(
    const T *x, int64_t x_stride, const T *residual, int64_t res_stride,
    T *residual_out, int64_t res_out_stride, const T *__restrict__ weight, T *out,
    int64_t out_stride, int64_t rows, int hidden, float factor, float eps) {
  using E = Elem<T>;
  using C = Chunk<T, N>;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int chunks = hidden / N;
  const C *xr = reinterpret_cast<const C *>(x + row * x_stride);
  const bool fused = residual != nullptr;
  float sum = 0.f;
  if (fused) {
    const C *rr = reinterpret_cast<const C *>(residual + row * res_stride);
    C *ro = reinterpret_cast<C *>(residual_out + row * res_out_stride);
    for (int c = lane; c < chunks; c += kWave) {
      const C a = xr[c], b = rr[c];
      C r;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        r.v[e] = E::from_f32(E::to_f32(b.v[e]) + E::to_f32(a.v[e]));
        const float f = E::to_f32(r.v[e]);
        sum += f * f;
      }
      ro[c] = r;
    }
  } else {
    for (int c = lane; c < chunks; c += kWave) {
      const C a = xr[c];
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float f = E::to_f32(a.v[e]);
        sum += f * f;
      }
    }
  }
  sum = wave_sum(sum);
  const float inv = rsqrtf(sum * factor + eps);
  const C *src = fused ? reinterpret_cast<const C *>(residual_out + row * res_out_stride) : xr;
  const C *wr = reinterpret_cast<const C *>(weight);
  C *dst = reinterpret_cast<C *>(out + row * out_stride);
  for (int c = lane; c < chunks; c += kWave) {
    const C a = src[c], w = wr[c];
    C o;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      float p = E::to_f32(a.v[e]) * inv;
      // Keep the FP32 rounding of the product: for fp16 the compiler would
      // otherwise fold product and conversion into one instruction that
      // rounds once (torch rounds to FP32, then to fp16).
      if constexpr (std::is_same<T, f16_t>::value) asm volatile("" : "+v"(p));
      const T n = E::from_f32(p);
      o.v[e] = E::from_f32(E::to_f32(w.v[e]) * E::to_f32(n));
    }
    dst[c] = o;
  }
}

// Rows of at most kWave * K chunks of N elements, held in registers (see the
// file comment). Each lane adds its chunks and their elements in the order
// rms_norm_kernel does, so the two kernels give the same bits.
template <typename T, int N, int K>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(
    const T *x, int64_t x_stride, const T *residual, int64_t res_stride,
    T *residual_out, int64_t res_out_stride, const T *__restrict__ weight, T *out,
    int64_t out_stride, int64_t rows, int hidden, float factor, float eps) {
  using E = Elem<T>;
  using C = Chunk<T, N>;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int chunks = hidden / N;
  const C *xr = reinterpret_cast<const C *>(x + row * x_stride);
  const C *wr = reinterpret_cast<const C *>(weight);
  C r[K], w[K], b[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = lane + kWave * k;
    if (c < chunks) {
      r[k] = xr[c];
      w[k] = wr[c];
    }
  }
  if (residual != nullptr) {
    const C *rr = reinterpret_cast<const C *>(residual + row * res_stride);
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (lane + kWave * k < chunks) b[k] = rr[lane + kWave * k];
    C *ro = reinterpret_cast<C *>(residual_out + row * res_out_stride);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int c = lane + kWave * k;
      if (c < chunks) {
#pragma unroll
        for (int e = 0; e < N; ++e)
          r[k].v[e] = E::from_f32(E::to_f32(b[k].v[e]) + E::to_f32(r[k].v[e]));
        ro[c] = r[k];
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane + kWave * k < chunks) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float f = E::to_f32(r[k].v[e]);
        sum += f * f;
      }
    }
  sum = wave_sum(sum);
  const float inv = rsqrtf(sum * factor + eps);
  C *dst = reinterpret_cast<C *>(out + row * out_stride);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int c = lane + kWave * k;
    if (c < chunks) {
      C o;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        float p = E::to_f32(r[k].v[e]) * inv;
        // The FP32 rounding of the product stays, as in rms_norm_kernel.
        if constexpr (std::is_same<T, f16_t>::value) asm volatile("" : "+v"(p));
        const T n = E::from_f32(p);
        o.v[e] = E::from_f32(E::to_f32(w[k].v[e]) * E::to_f32(n));
      }
      dst[c] = o;
    }
  }
}

template <typename T, int N>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T *__restrict__ gate_up,
                                                       int64_t gu_stride, T *__restrict__ out,
                                                       int64_t out_stride, int64_t rows,
                                                       int inter) {
  using E = Elem<T>;
  using C = Chunk<T, N>;
  const int chunks = inter / N;
  const int64_t total = rows * chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / chunks;
    const int c = static_cast<int>(i - row * chunks);
    const C *g = reinterpret_cast<const C *>(gate_up + row * gu_stride);
    const C *u = reinterpret_cast<const C *>(gate_up + row * gu_stride + inter);
    const C a = g[c], b = u[c];
    C o;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float gf = E::to_f32(a.v[e]);
      const T s = E::from_f32(gf / (1.0f + expf(-gf)));
      o.v[e] = E::from_f32(E::to_f32(s) * E::to_f32(b.v[e]));
    }
    reinterpret_cast<C *>(out + row * out_stride)[c] = o;
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
int launch_norm(const void *x, int64_t xs, const void *res, int64_t rs, void *ro, int64_t ros,
                const void *w, void *out, int64_t os, int64_t rows, int64_t hidden, float factor,
                float eps, hipStream_t stream) {
  constexpr int N = Vec16<T>::n;
  const bool vec = hidden % N == 0 && xs % N == 0 && os % N == 0 && aligned16(x) &&
                   aligned16(w) && aligned16(out) &&
                   (res == nullptr || (rs % N == 0 && ros % N == 0 && aligned16(res) &&
                                       aligned16(ro)));
  const unsigned blocks = static_cast<unsigned>(ceil_div(rows, 4));
  const auto *xt = static_cast<const T *>(x);
  const auto *rt = static_cast<const T *>(res);
  auto *rot = static_cast<T *>(ro);
  const auto *wt = static_cast<const T *>(w);
  auto *ot = static_cast<T *>(out);
  const int h = static_cast<int>(hidden);
  const int64_t chunks = hidden / N;
  if (vec && chunks <= kWave)
    rms_norm_rows_kernel<T, N, 1><<<blocks, 256, 0, stream>>>(xt, xs, rt, rs, rot, ros, wt, ot,
                                                             os, rows, h, factor, eps);
  else if (vec && chunks <= 2 * kWave)
    rms_norm_rows_kernel<T, N, 2><<<blocks, 256, 0, stream>>>(xt, xs, rt, rs, rot, ros, wt, ot,
                                                             os, rows, h, factor, eps);
  else if (vec && chunks <= 4 * kWave)
    rms_norm_rows_kernel<T, N, 4><<<blocks, 256, 0, stream>>>(xt, xs, rt, rs, rot, ros, wt, ot,
                                                             os, rows, h, factor, eps);
  else if (vec)
    rms_norm_kernel<T, N><<<blocks, 256, 0, stream>>>(xt, xs, rt, rs, rot, ros, wt, ot, os, rows,
                                                     h, factor, eps);
  else
    rms_norm_kernel<T, 1><<<blocks, 256, 0, stream>>>(xt, xs, rt, rs, rot, ros, wt, ot, os, rows,
                                                     static_cast<int>(hidden), factor, eps);
  return check_launch("mlr_rms_norm");
}

template <typename T>
int launch_silu_mul(const void *gu, int64_t gs, void *out, int64_t os, int64_t rows,
                    int64_t inter, hipStream_t stream) {
  constexpr int N = Vec16<T>::n;
  const bool vec = inter % N == 0 && gs % N == 0 && os % N == 0 && aligned16(gu) &&
                   aligned16(out);
  const int n = vec ? N : 1;
  const int64_t total = rows * (inter / n);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(total, 256), 4096));
  const auto *g = static_cast<const T *>(gu);
  auto *o = static_cast<T *>(out);
  if (vec)
    silu_mul_kernel<T, N><<<blocks, 256, 0, stream>>>(g, gs, o, os, rows,
                                                     static_cast<int>(inter));
  else
    silu_mul_kernel<T, 1><<<blocks, 256, 0, stream>>>(g, gs, o, os, rows,
                                                     static_cast<int>(inter));
  return check_launch("mlr_silu_mul");
}

}  // namespace
}  // namespace mlr

using namespace mlr;

extern "C" int mlr_rms_norm(const void *x, int64_t x_stride, const void *residual,
                            int64_t residual_stride, void *residual_out,
                            int64_t residual_out_stride, const void *weight, void *out,
                            int64_t out_stride, int64_t rows, int64_t hidden, double eps,
                            int dtype, void *stream) {
  clear_error();
  MLR_REQUIRE(rows >= 0, "mlr_rms_norm: rows must be >= 0");
  MLR_REQUIRE(hidden > 0 && hidden <= (int64_t(1) << 20),
              "mlr_rms_norm: hidden must be in [1, 2^20]");
  MLR_REQUIRE(eps > 0, "mlr_rms_norm: eps must be > 0");
  if (rows == 0) return MLR_OK;
  MLR_REQUIRE(x && weight && out, "mlr_rms_norm: null x, weight or out");
  MLR_REQUIRE((residual == nullptr) == (residual_out == nullptr),
              "mlr_rms_norm: residual and residual_out go together");
  MLR_REQUIRE(x_stride >= hidden && out_stride >= hidden &&
                  (residual == nullptr ||
                   (residual_stride >= hidden && residual_out_stride >= hidden)),
              "mlr_rms_norm: a row stride is smaller than hidden");
  MLR_REQUIRE(ceil_div(rows, 4) < INT32_MAX, "mlr_rms_norm: too many rows");
  // The scale torch's mean applies: float(rows) / float(rows * hidden).
  const float factor = static_cast<float>(rows) / static_cast<float>(rows * hidden);
  const float e = static_cast<float>(eps);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MLR_DTYPE_BF16:
      return launch_norm<bf16_t>(x, x_stride, residual, residual_stride, residual_out,
                                 residual_out_stride, weight, out, out_stride, rows, hidden,
                                 factor, e, s);
    case MLR_DTYPE_F16:
      return launch_norm<f16_t>(x, x_stride, residual, residual_stride, residual_out,
                                residual_out_stride, weight, out, out_stride, rows, hidden,
                                factor, e, s);
    case MLR_DTYPE_F32:
      return launch_norm<float>(x, x_stride, residual, residual_stride, residual_out,
                                residual_out_stride, weight, out, out_stride, rows, hidden,
                                factor, e, s);
    default:
      return set_error(MLR_ERR_INVALID, "mlr_rms_norm: dtype %d not supported (bf16, fp16, "
                       "fp32)", dtype);
  }
}

extern "C" int mlr_silu_mul(const void *gate_up, int64_t gate_up_stride, void *out,
                            int64_t out_stride, int64_t rows, int64_t intermediate, int dtype,
                            void *stream) {
  clear_error();
  MLR_REQUIRE(rows >= 0, "mlr_silu_mul: rows must be >= 0");
  MLR_REQUIRE(intermediate > 0 && intermediate <= (int64_t(1) << 24),
              "mlr_silu_mul: intermediate must be in [1, 2^24]");
  if (rows == 0) return MLR_OK;
  MLR_REQUIRE(gate_up && out, "mlr_silu_mul: null gate_up or out");
  MLR_REQUIRE(gate_up_stride >= 2 * intermediate && out_stride >= intermediate,
              "mlr_silu_mul: a row stride is too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MLR_DTYPE_BF16:
      return launch_silu_mul<bf16_t>(gate_up, gate_up_stride, out, out_stride, rows,
                                     intermediate, s);
    case MLR_DTYPE_F16:
      return launch_silu_mul<f16_t>(gate_up, gate_up_stride, out, out_stride, rows,
                                    intermediate, s);
    case MLR_DTYPE_F32:
      return launch_silu_mul<float>(gate_up, gate_up_stride, out, out_stride, rows,
                                    intermediate, s);
    default:
      return set_error(MLR_ERR_INVALID, "mlr_silu_mul: dtype %d not supported (bf16, fp16, "
                       "fp32)", dtype);
  }
}
