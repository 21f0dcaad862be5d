// KV-cache write: scatter [T, Hkv, D] rows of K and V into one layer's paged
// block pool at flat slots, converting the element type on the way.
//
// Replaces the two index_copy_ calls of PagedKVCache.write_slots
// (runtime/paged_kv_cache.py:243-249). The pool layer is
// [num_blocks, block_size, Hkv, D] contiguous, so slot s is the contiguous run
// of Hkv*D elements starting at s*Hkv*D; the kernel writes whole 16-byte
// chunks of that run when source and cache share one element type.
#include "mlr_common.h"

namespace mlr {
namespace {

template <typename I>
__device__ __forceinline__ int64_t load_slot(const void *slots, int64_t t) {
  return static_cast<int64_t>(static_cast<const I *>(slots)[t]);
}

// Exact element conversion S -> C (bit copy when the types match).
template <typename S, typename C>
__device__ __forceinline__ C convert_elem(S x) {
  if constexpr (std::is_same<S, C>::value) {
    return x;
  } else if constexpr (std::is_same<S, double>::value ||
                       std::is_same<C, double>::value) {
    return Elem<C>::from_f64(Elem<S>::to_f64(x));
  } else {
    return Elem<C>::from_f32(Elem<S>::to_f32(x));
  }
}

// One thread per (token, head, dim) element; any strides, any type pair.
template <typename S, typename C, typename I>
__global__ __launch_bounds__(256) void kv_write_generic_kernel(
    const S *__restrict__ k, const S *__restrict__ v, int64_t num_tokens,
    int64_t kst, int64_t ksh, int64_t ksd, int64_t vst, int64_t vsh,
    int64_t vsd, const void *__restrict__ slots, C *__restrict__ kc,
    C *__restrict__ vc, int64_t num_slots, int64_t hkv, int64_t d) {
  const int64_t n = num_tokens * hkv * d;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i % d;
    const int64_t r = i / d;
    const int64_t h = r % hkv;
    const int64_t t = r / hkv;
    const int64_t slot = load_slot<I>(slots, t);
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t dst = (slot * hkv + h) * d + e;
    kc[dst] = convert_elem<S, C>(k[t * kst + h * ksh + e * ksd]);
    vc[dst] = convert_elem<S, C>(v[t * vst + h * vsh + e * vsd]);
  }
}

// Same element type, unit stride along D, 16-byte aligned rows: one thread
// moves one 16-byte chunk of one (token, head) row for K and one for V.
template <typename I>
__global__ __launch_bounds__(256) void kv_write_vec16_kernel(
    const uint4 *__restrict__ k, const uint4 *__restrict__ v,
    int64_t num_tokens, int64_t kst, int64_t ksh, int64_t vst, int64_t vsh,
    const void *__restrict__ slots, uint4 *__restrict__ kc,
    uint4 *__restrict__ vc, int64_t num_slots, int64_t hkv,
    int64_t chunks_per_row) {
  // Strides here are in 16-byte chunks. The host launches this kernel only
  // when num_tokens * hkv * chunks_per_row fits 32 bits.
  const uint32_t n = static_cast<uint32_t>(num_tokens * hkv * chunks_per_row);
  const uint32_t cpr = static_cast<uint32_t>(chunks_per_row);
  const uint32_t nh = static_cast<uint32_t>(hkv);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += gridDim.x * blockDim.x) {
    const uint32_t c = i % cpr;
    const uint32_t r = i / cpr;
    const uint32_t h = r % nh;
    const uint32_t t = r / nh;
    // The source rows do not depend on the slot: all three loads are in
    // flight together.
    const uint4 kv = k[t * kst + h * ksh + c];
    const uint4 vv = v[t * vst + h * vsh + c];
    const int64_t slot = load_slot<I>(slots, t);
    if (slot < 0 || slot >= num_slots) continue;
    const int64_t dst = (slot * hkv + h) * chunks_per_row + c;
    kc[dst] = kv;
    vc[dst] = vv;
  }
}

int grid_for(int64_t n, int threads) {
  int64_t blocks = ceil_div(n, threads);
  if (blocks > 65536) blocks = 65536;  // grid-stride loops cover the rest
  return static_cast<int>(blocks < 1 ? 1 : blocks);
}

template <typename S, typename C>
int launch_generic(const void *k, const void *v, int64_t T, int64_t kst,
                   int64_t ksh, int64_t ksd, int64_t vst, int64_t vsh,
                   int64_t vsd, const void *slots, int index_dtype, void *kc,
                   void *vc, int64_t num_slots, int64_t hkv, int64_t d,
                   hipStream_t stream) {
  const int64_t n = T * hkv * d;
  const int threads = 256;
  const int blocks = grid_for(n, threads);
  if (index_dtype == MLR_INDEX_I32) {
    kv_write_generic_kernel<S, C, int32_t><<<blocks, threads, 0, stream>>>(
        static_cast<const S *>(k), static_cast<const S *>(v), T, kst, ksh, ksd,
        vst, vsh, vsd, slots, static_cast<C *>(kc), static_cast<C *>(vc),
        num_slots, hkv, d);
  } else {
    kv_write_generic_kernel<S, C, int64_t><<<blocks, threads, 0, stream>>>(
        static_cast<const S *>(k), static_cast<const S *>(v), T, kst, ksh, ksd,
        vst, vsh, vsd, slots, static_cast<C *>(kc), static_cast<C *>(vc),
        num_slots, hkv, d);
  }
  return check_launch("mlr_kv_write");
}

template <typename S>
int dispatch_cache(int cache_dtype, const void *k, const void *v, int64_t T,
                   int64_t kst, int64_t ksh, int64_t ksd, int64_t vst,
                   int64_t vsh, int64_t vsd, const void *slots,
                   int index_dtype, void *kc, void *vc, int64_t num_slots,
                   int64_t hkv, int64_t d, hipStream_t stream) {
  switch (cache_dtype) {
    case MLR_DTYPE_F32:
      return launch_generic<S, float>(k, v, T, kst, ksh, ksd, vst, vsh, vsd,
                                      slots, index_dtype, kc, vc, num_slots,
                                      hkv, d, stream);
    case MLR_DTYPE_F16:
      return launch_generic<S, f16_t>(k, v, T, kst, ksh, ksd, vst, vsh, vsd,
                                      slots, index_dtype, kc, vc, num_slots,
                                      hkv, d, stream);
    case MLR_DTYPE_BF16:
      return launch_generic<S, bf16_t>(k, v, T, kst, ksh, ksd, vst, vsh, vsd,
                                       slots, index_dtype, kc, vc, num_slots,
                                       hkv, d, stream);
    case MLR_DTYPE_F64:
      return launch_generic<S, double>(k, v, T, kst, ksh, ksd, vst, vsh, vsd,
                                       slots, index_dtype, kc, vc, num_slots,
                                       hkv, d, stream);
    default:
      return set_error(MLR_ERR_INVALID, "mlr_kv_write: unknown cache dtype %d",
                       cache_dtype);
  }
}

bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace
}  // namespace mlr

extern "C" int mlr_kv_write(const void *k, const void *v, int src_dtype,
                            int64_t num_tokens, int64_t k_stride_t,
                            int64_t k_stride_h, int64_t k_stride_d,
                            int64_t v_stride_t, int64_t v_stride_h,
                            int64_t v_stride_d, const void *slot_mapping,
                            int index_dtype, void *k_cache, void *v_cache,
                            int cache_dtype, int64_t num_slots,
                            int64_t num_kv_heads, int64_t head_dim,
                            void *stream) {
  using namespace mlr;
  clear_error();
  MLR_REQUIRE(num_tokens >= 0, "mlr_kv_write: num_tokens must be >= 0");
  MLR_REQUIRE(num_kv_heads > 0 && head_dim > 0,
              "mlr_kv_write: num_kv_heads and head_dim must be > 0");
  MLR_REQUIRE(num_slots >= 0, "mlr_kv_write: num_slots must be >= 0");
  MLR_REQUIRE(index_dtype == MLR_INDEX_I32 || index_dtype == MLR_INDEX_I64,
              "mlr_kv_write: slot_mapping must be int32 or int64");
  const int ssz = dtype_size(src_dtype);
  const int csz = dtype_size(cache_dtype);
  MLR_REQUIRE(ssz > 0, "mlr_kv_write: unknown source dtype %d", src_dtype);
  MLR_REQUIRE(csz > 0, "mlr_kv_write: unknown cache dtype %d", cache_dtype);
  if (num_tokens == 0) return MLR_OK;  // empty writes are allowed
  MLR_REQUIRE(k && v && slot_mapping && k_cache && v_cache,
              "mlr_kv_write: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);

  // Vector path: same type, unit D stride, whole 16-byte chunks, aligned rows.
  const int64_t row_bytes = head_dim * csz;
  const int64_t elems_per_chunk = 16 / csz;
  const bool same = src_dtype == cache_dtype;
  const bool vec_ok =
      same && k_stride_d == 1 && v_stride_d == 1 && row_bytes % 16 == 0 &&
      (k_stride_t % elems_per_chunk) == 0 &&
      (k_stride_h % elems_per_chunk) == 0 &&
      (v_stride_t % elems_per_chunk) == 0 &&
      (v_stride_h % elems_per_chunk) == 0 && aligned16(k) && aligned16(v) &&
      aligned16(k_cache) && aligned16(v_cache) &&
      num_tokens * num_kv_heads * (row_bytes / 16) < (int64_t(1) << 31);
  if (vec_ok) {
    const int64_t cpr = row_bytes / 16;
    const int64_t n = num_tokens * num_kv_heads * cpr;
    const int threads = 256;
    const int blocks = grid_for(n, threads);
    const auto *k4 = static_cast<const uint4 *>(k);
    const auto *v4 = static_cast<const uint4 *>(v);
    auto *kc4 = static_cast<uint4 *>(k_cache);
    auto *vc4 = static_cast<uint4 *>(v_cache);
    const int64_t e = elems_per_chunk;
    if (index_dtype == MLR_INDEX_I32) {
      kv_write_vec16_kernel<int32_t><<<blocks, threads, 0, s>>>(
          k4, v4, num_tokens, k_stride_t / e, k_stride_h / e, v_stride_t / e,
          v_stride_h / e, slot_mapping, kc4, vc4, num_slots, num_kv_heads,
          cpr);
    } else {
      kv_write_vec16_kernel<int64_t><<<blocks, threads, 0, s>>>(
          k4, v4, num_tokens, k_stride_t / e, k_stride_h / e, v_stride_t / e,
          v_stride_h / e, slot_mapping, kc4, vc4, num_slots, num_kv_heads,
          cpr);
    }
    return check_launch("mlr_kv_write");
  }

  switch (src_dtype) {
    case MLR_DTYPE_F32:
      return dispatch_cache<float>(cache_dtype, k, v, num_tokens, k_stride_t,
                                   k_stride_h, k_stride_d, v_stride_t,
                                   v_stride_h, v_stride_d, slot_mapping,
                                   index_dtype, k_cache, v_cache, num_slots,
                                   num_kv_heads, head_dim, s);
    case MLR_DTYPE_F16:
      return dispatch_cache<f16_t>(cache_dtype, k, v, num_tokens, k_stride_t,
                                   k_stride_h, k_stride_d, v_stride_t,
                                   v_stride_h, v_stride_d, slot_mapping,
                                   index_dtype, k_cache, v_cache, num_slots,
                                   num_kv_heads, head_dim, s);
    case MLR_DTYPE_BF16:
      return dispatch_cache<bf16_t>(cache_dtype, k, v, num_tokens, k_stride_t,
                                    k_stride_h, k_stride_d, v_stride_t,
                                    v_stride_h, v_stride_d, slot_mapping,
                                    index_dtype, k_cache, v_cache, num_slots,
                                    num_kv_heads, head_dim, s);
    case MLR_DTYPE_F64:
      return dispatch_cache<double>(cache_dtype, k, v, num_tokens, k_stride_t,
                                    k_stride_h, k_stride_d, v_stride_t,
                                    v_stride_h, v_stride_d, slot_mapping,
                                    index_dtype, k_cache, v_cache, num_slots,
                                    num_kv_heads, head_dim, s);
    default:
      return set_error(MLR_ERR_INVALID, "mlr_kv_write: unknown source dtype %d",
                       src_dtype);
  }
}
