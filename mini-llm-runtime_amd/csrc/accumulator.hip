// Batched weighted row sum out[b, d] = sum_n p[b, n] * v[b, n, d] (FP32),
// the contract of the reference's only native extension
// (kernels/cuda/paged_attention_accumulator.cu:83-100 forward(p, v), called
// through kernels/cuda/accumulator.py:21-37): p [B, 64], v [B, 64, 256].
//
// One wave per batch entry: lane l owns the four consecutive columns 4l..4l+3
// (256 = 64 lanes x 4), streams the 64 rows of v as 16-byte loads, half of
// them in flight at once, and accumulates with FP32 fma in row order. No
// cross-wave reduction, no LDS. HBM-bound: 64 KB of v per entry.
#include "mlr_common.h"

namespace mlr {
namespace {

constexpr int kRows = 64;
constexpr int kCols = 256;
constexpr int kPass = 32;  // rows in flight per lane
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void accumulate_kernel(const float *__restrict__ p,
                                                         const float *__restrict__ v,
                                                         float *__restrict__ out,
                                                         int64_t batch) {
  const int lane = threadIdx.x & 63;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (b >= batch) return;  // whole waves
  const f32x4_t *vb = reinterpret_cast<const f32x4_t *>(v + b * kRows * kCols) + lane;
  const float *pb = p + b * kRows;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n0 = 0; n0 < kRows; n0 += kPass) {
    f32x4_t rows[kPass];
#pragma unroll
    for (int i = 0; i < kPass; ++i)
      rows[i] = __builtin_nontemporal_load(vb + (n0 + i) * (kCols / 4));
#pragma unroll
    for (int i = 0; i < kPass; ++i) {
      const float w = pb[n0 + i];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(w, rows[i][e], acc[e]);
    }
  }
  reinterpret_cast<f32x4_t *>(out + b * kCols)[lane] = acc;
}

}  // namespace
}  // namespace mlr

extern "C" int mlr_pa_accumulate(const float *p, const float *v, float *out, int64_t batch,
                                 void *stream) {
  using namespace mlr;
  clear_error();
  MLR_REQUIRE(batch >= 0, "mlr_pa_accumulate: batch must be >= 0");
  MLR_REQUIRE(batch / 4 < INT32_MAX, "mlr_pa_accumulate: batch too large");
  if (batch == 0) return MLR_OK;
  MLR_REQUIRE(p && v && out, "mlr_pa_accumulate: null pointer");
  MLR_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(out) & 15u) == 0,
              "mlr_pa_accumulate: v and out must be 16-byte aligned");
  const unsigned blocks = static_cast<unsigned>((batch + 3) / 4);
  accumulate_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(p, v, out, batch);
  return check_launch("mlr_pa_accumulate");
}
