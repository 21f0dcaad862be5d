// Fused pre-attention step: optional QKV bias, rotary embedding of Q and K,
// and the KV-cache write, in one launch.
//
// Replaces, per layer, the tail of Qwen2QKVProjection.forward (bias) and the
// Qwen2RotaryEmbedding / apply_rotary_pos_emb / write_slots sequence of the
// reference's attention callers (model/qwen2.py:125-209, :605-613, :737-746;
// runtime/paged_kv_cache.py:243-249). The input is one row per token of the
// concatenated projection [q heads | k heads | v heads] x head_dim.
//
// Numerics are the reference's operation by operation, in the model dtype:
//   f      = float(position) * inv_freq[i]                     (FP32)
//   c, s   = dtype(cos f), dtype(sin f)
//   out_lo = dtype(dtype(x_lo * c) + dtype(-x_hi * s))
//   out_hi = dtype(dtype(x_hi * c) + dtype(x_lo * s))
// for i < head_dim/2, x_lo = x[i], x_hi = x[i + head_dim/2] (rotate_half
// convention). Products and sums are single FP32 operations rounded once to
// the dtype (what torch's half-precision elementwise ops do); FP32 runs
// without contraction into fma. cos and sin are the device library's, as in
// torch's own kernels.
#include "mlr_common.h"

namespace mlr {
namespace {

// x rounded to T (nearest even) and back to FP32, for the intermediate
// roundings; stored values go through Elem<T>::from_f32, which also maps
// every NaN to the canonical one. bf16 rounds with v_cvt_pk_bf16_f32, two
// values per instruction in rnd2.
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return Elem<T>::to_f32(Elem<T>::from_f32(x));
}
template <>
__device__ __forceinline__ float rnd<bf16_t>(float x) {
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(x)))
                         << 16);
}
template <typename T>
__device__ __forceinline__ void rnd2(float &a, float &b) {
  a = rnd<T>(a);
  b = rnd<T>(b);
}
template <>
__device__ __forceinline__ void rnd2<bf16_t>(float &a, float &b) {
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{a, b}, bf16x2_v));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

template <typename T>
__device__ __forceinline__ float load_f(const T *p) {
  return Elem<T>::to_f32(*p);
}

template <typename I>
__device__ __forceinline__ int64_t load_index(const void *p, int64_t t) {
  return static_cast<int64_t>(static_cast<const I *>(p)[t]);
}

// VEC consecutive elements, moved as one load or store.
template <typename T, int VEC>
struct alignas(VEC * sizeof(T)) Vec {
  T v[VEC];
};

// One wave per token (grid-stride over tokens; a workgroup holds one wave,
// or four for large launches). A token's row is cut into
// chunks of VEC elements: a rotary chunk is VEC elements of the first half of
// a q or k head with their partners in the second half; a v chunk is VEC
// elements of a v head. A lane takes K chunks per pass. The position and the
// lane's inverse frequency are loaded first, then every chunk load of the
// pass is issued unconditionally (clamped index), so the loads are in flight
// together and the cos/sin table is built under their latency; only the
// stores depend on the chunk kind.
template <typename T, typename I, int VEC, int K>
__global__ __launch_bounds__(256) void qkv_rope_write_kernel(
    const T *__restrict__ qkv, int64_t qkv_st, const T *__restrict__ bias,
    const int64_t *__restrict__ positions, const float *__restrict__ inv_freq,
    const void *__restrict__ slots, T *__restrict__ q_out, int64_t q_st,
    T *__restrict__ kc, T *__restrict__ vc, int64_t num_slots, int64_t num_tokens, int hq,
    int hkv, int d) {
#pragma clang fp contract(off)
  using V = Vec<T, VEC>;
  // Per wave: [d/2] cos then [d/2] sin, dtype-rounded. The wave's own rows:
  // LDS operations of one wave complete in order, and the wave barriers
  // (no instruction) keep the compiler from reordering across them.
  extern __shared__ float cs_all[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  float *cs = cs_all + wv * d;
  const int half = d / 2;
  const int cph = half / VEC;  // rotary chunks per head
  const int n_rope = (hq + hkv) * cph;
  const int n_chunks = n_rope + hkv * d / VEC;
  const int v_base = (hq + hkv) * d;
  const float my_freq = lane < half ? inv_freq[lane] : 0.f;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * waves + wv; t < num_tokens;
       t += static_cast<int64_t>(gridDim.x) * waves) {
    const T *row = qkv + t * qkv_st;
    const float pos = static_cast<float>(positions[t]);
    const int64_t slot = load_index<I>(slots, t);
    const bool write_kv = slot >= 0 && slot < num_slots;
    for (int c0 = 0; c0 < n_chunks; c0 += 64 * K) {
      V lo[K], hi[K];
      int elo[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = min(c0 + 64 * k + lane, n_chunks - 1);
        const bool rope = c < n_rope;
        elo[k] = rope ? (c / cph) * d + (c % cph) * VEC : v_base + (c - n_rope) * VEC;
        lo[k] = *reinterpret_cast<const V *>(row + elo[k]);
        hi[k] = *reinterpret_cast<const V *>(row + (rope ? elo[k] + half : elo[k]));
      }
      if (c0 == 0) {
        // sincosf: one argument reduction for both; its results are those
        // of cosf and sinf.
        if (lane < half) {
          float sv, cv;
          sincosf(pos * my_freq, &sv, &cv);
          rnd2<T>(cv, sv);
          cs[lane] = cv;
          cs[half + lane] = sv;
        }
        for (int i = lane + 64; i < half; i += 64) {  // head_dim > 128
          float sv, cv;
          sincosf(pos * inv_freq[i], &sv, &cv);
          rnd2<T>(cv, sv);
          cs[i] = cv;
          cs[half + i] = sv;
        }
        __builtin_amdgcn_wave_barrier();
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = c0 + 64 * k + lane;
        if (c >= n_chunks) continue;
        if (c < n_rope) {
          const int h = c / cph, i0 = (c % cph) * VEC;
          V olo, ohi;
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float x_lo = Elem<T>::to_f32(lo[k].v[j]), x_hi = Elem<T>::to_f32(hi[k].v[j]);
            if (bias != nullptr) {
              x_lo = rnd<T>(x_lo + load_f(bias + h * d + i0 + j));
              x_hi = rnd<T>(x_hi + load_f(bias + h * d + half + i0 + j));
            }
            const float cv = cs[i0 + j], sv = cs[half + i0 + j];
            float a = x_lo * cv, b = -x_hi * sv, e = x_hi * cv, f = x_lo * sv;
            rnd2<T>(a, b);
            rnd2<T>(e, f);
            olo.v[j] = Elem<T>::from_f32(a + b);
            ohi.v[j] = Elem<T>::from_f32(e + f);
          }
          T *o = h < hq ? q_out + t * q_st + static_cast<int64_t>(h) * d
                        : kc + (slot * hkv + (h - hq)) * d;
          if (h < hq || write_kv) {
            *reinterpret_cast<V *>(o + i0) = olo;
            *reinterpret_cast<V *>(o + i0 + half) = ohi;
          }
        } else if (write_kv) {
          const int ev = elo[k] - v_base;  // element within the token's v heads
          V ov = lo[k];
          if (bias != nullptr) {
#pragma unroll
            for (int j = 0; j < VEC; ++j)
              ov.v[j] = Elem<T>::from_f32(Elem<T>::to_f32(lo[k].v[j]) +
                                          load_f(bias + v_base + ev + j));
          }
          *reinterpret_cast<V *>(vc + slot * hkv * d + ev) = ov;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // cs is rewritten for the next token
  }
}

// Head size 64 or 128 with 16-byte chunks (the same arithmetic as above,
// the chunk-to-head map by shifts). The token index is made wave-uniform, so
// its position and slot are scalar loads, and a pass's row loads are issued
// before anything waits: the cos/sin table is built while they are in flight.
template <typename T, typename I, int D, int K>
__global__ __launch_bounds__(256) void qkv_rope_write_wide_kernel(
    const T *__restrict__ qkv, int64_t qkv_st, const T *__restrict__ bias,
    const int64_t *__restrict__ positions, const float *__restrict__ inv_freq,
    const void *__restrict__ slots, T *__restrict__ q_out, int64_t q_st,
    T *__restrict__ kc, T *__restrict__ vc, int64_t num_slots, int64_t num_tokens, int hq,
    int hkv) {
#pragma clang fp contract(off)
  constexpr int kVec = 16 / sizeof(T);
  constexpr int kHalf = D / 2;
  constexpr int kCph = kHalf / kVec;  // rotary chunks per head
  static_assert(kHalf % kVec == 0 && kHalf <= 64, "head size 64 or 128");
  using V = Vec<T, kVec>;
  extern __shared__ float cs_all[];  // per wave: [D/2] cos then [D/2] sin
  const int lane = __lane_id();
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  float *cs = cs_all + wv * D;
  const int n_rope = (hq + hkv) * kCph;
  const int n_chunks = n_rope + hkv * (D / kVec);
  const int v_base = (hq + hkv) * D;
  // Lanes past D/2 load a duplicate they never use.
  const float my_freq = inv_freq[lane & (kHalf - 1)];
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * waves + wv; t < num_tokens;
       t += static_cast<int64_t>(gridDim.x) * waves) {
    const T *row = qkv + t * qkv_st;
    V lo[K], hi[K];
    // Chunk c of the row: rotary chunks first (head c / kCph, elements
    // [i0, i0 + kVec) and their partners at + D/2), then the v chunks.
    auto load_pass = [&](int c0) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = min(c0 + 64 * k + lane, n_chunks - 1);
        const bool rope = c < n_rope;
        const int e = rope ? (c / kCph) * D + (c % kCph) * kVec : v_base + (c - n_rope) * kVec;
        lo[k] = *reinterpret_cast<const V *>(row + e);
        hi[k] = *reinterpret_cast<const V *>(row + (rope ? e + kHalf : e));
      }
    };
    load_pass(0);
    const float pos = static_cast<float>(positions[t]);
    const int64_t slot = load_index<I>(slots, t);
    const bool write_kv = slot >= 0 && slot < num_slots;
    if (lane < kHalf) {
      // sincosf: one argument reduction for both; its results are those of
      // cosf and sinf.
      float sv, cv;
      sincosf(pos * my_freq, &sv, &cv);
      rnd2<T>(cv, sv);
      cs[lane] = cv;
      cs[kHalf + lane] = sv;
    }
    __builtin_amdgcn_wave_barrier();
    for (int c0 = 0;;) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = c0 + 64 * k + lane;
        if (c >= n_chunks) continue;
        if (c < n_rope) {
          const int h = c / kCph, i0 = (c % kCph) * kVec;
          V olo, ohi;
#pragma unroll
          for (int j = 0; j < kVec; ++j) {
            float x_lo = Elem<T>::to_f32(lo[k].v[j]), x_hi = Elem<T>::to_f32(hi[k].v[j]);
            if (bias != nullptr) {
              x_lo = rnd<T>(x_lo + load_f(bias + h * D + i0 + j));
              x_hi = rnd<T>(x_hi + load_f(bias + h * D + kHalf + i0 + j));
            }
            const float cv = cs[i0 + j], sv = cs[kHalf + i0 + j];
            float a = x_lo * cv, b = -x_hi * sv, e = x_hi * cv, f = x_lo * sv;
            rnd2<T>(a, b);
            rnd2<T>(e, f);
            olo.v[j] = Elem<T>::from_f32(a + b);
            ohi.v[j] = Elem<T>::from_f32(e + f);
          }
          T *o = h < hq ? q_out + t * q_st + static_cast<int64_t>(h) * D
                        : kc + (slot * hkv + (h - hq)) * D;
          if (h < hq || write_kv) {
            *reinterpret_cast<V *>(o + i0) = olo;
            *reinterpret_cast<V *>(o + i0 + kHalf) = ohi;
          }
        } else if (write_kv) {
          const int ev = (c - n_rope) * kVec;  // element within the token's v heads
          V ov = lo[k];
          if (bias != nullptr) {
#pragma unroll
            for (int j = 0; j < kVec; ++j)
              ov.v[j] = Elem<T>::from_f32(Elem<T>::to_f32(lo[k].v[j]) +
                                          load_f(bias + v_base + ev + j));
          }
          *reinterpret_cast<V *>(vc + slot * hkv * D + ev) = ov;
        }
      }
      c0 += 64 * K;
      if (c0 >= n_chunks) break;
      load_pass(c0);
    }
    __builtin_amdgcn_wave_barrier();  // cs is rewritten for the next token
  }
}

template <typename T, typename I, int VEC>
void launch_vec(const void *qkv, int64_t qkv_st, const void *bias, const int64_t *positions,
                const float *inv_freq, const void *slots, void *q_out, int64_t q_st, void *kc,
                void *vc, int64_t num_slots, int64_t num_tokens, int hq, int hkv, int d,
                hipStream_t stream) {
  // Four tokens (waves) per workgroup from 1024 tokens on, one below it.
  // Measured at a Qwen2.5-0.5B layer, bf16, in 100-call graphs: 2048
  // tokens 4.39 us against 4.53 us with one wave per workgroup (eight per
  // workgroup: 4.40 us); 48 tokens 3.30 us against 3.18 us.
  const int waves = num_tokens >= 1024 ? 4 : 1;
  const int64_t wgs = (num_tokens + waves - 1) / waves;
  const int64_t blocks = wgs < 65536 ? wgs : 65536;
  const size_t lds = static_cast<size_t>(waves) * d * sizeof(float);
  qkv_rope_write_kernel<T, I, VEC, 4><<<static_cast<unsigned>(blocks), 64 * waves, lds, stream>>>(
      static_cast<const T *>(qkv), qkv_st, static_cast<const T *>(bias), positions, inv_freq,
      slots, static_cast<T *>(q_out), q_st, static_cast<T *>(kc), static_cast<T *>(vc),
      num_slots, num_tokens, hq, hkv, d);
}

template <typename T, typename I, int D>
void launch_wide(const void *qkv, int64_t qkv_st, const void *bias, const int64_t *positions,
                 const float *inv_freq, const void *slots, void *q_out, int64_t q_st, void *kc,
                 void *vc, int64_t num_slots, int64_t num_tokens, int hq, int hkv,
                 hipStream_t stream) {
  const int waves = num_tokens >= 1024 ? 4 : 1;
  const int64_t wgs = (num_tokens + waves - 1) / waves;
  const int64_t blocks = wgs < 65536 ? wgs : 65536;
  const size_t lds = static_cast<size_t>(waves) * D * sizeof(float);
  qkv_rope_write_wide_kernel<T, I, D, 2>
      <<<static_cast<unsigned>(blocks), 64 * waves, lds, stream>>>(
          static_cast<const T *>(qkv), qkv_st, static_cast<const T *>(bias), positions,
          inv_freq, slots, static_cast<T *>(q_out), q_st, static_cast<T *>(kc),
          static_cast<T *>(vc), num_slots, num_tokens, hq, hkv);
}

template <typename T>
int launch(const void *qkv, int64_t qkv_st, const void *bias, const int64_t *positions,
           const float *inv_freq, const void *slots, int index_dtype, void *q_out,
           int64_t q_st, void *kc, void *vc, int64_t num_slots, int64_t num_tokens, int hq,
           int hkv, int d, hipStream_t stream) {
  // 16-byte chunks at head sizes 64 and 128; otherwise four-element chunks.
  // Either needs half a head to be whole chunks and every row start aligned
  // to the chunk size.
  auto aligned_to = [&](int vec) {
    const uintptr_t align = vec * sizeof(T) - 1;
    return (d / 2) % vec == 0 && qkv_st % vec == 0 && q_st % vec == 0 &&
           (reinterpret_cast<uintptr_t>(qkv) & align) == 0 &&
           (reinterpret_cast<uintptr_t>(q_out) & align) == 0 &&
           (reinterpret_cast<uintptr_t>(kc) & align) == 0 &&
           (reinterpret_cast<uintptr_t>(vc) & align) == 0;
  };
  constexpr int kWide = 16 / sizeof(T);
  constexpr int kVec = 4;
  const bool wide = (d == 64 || d == 128) && aligned_to(kWide);
  const bool vec = aligned_to(kVec);
  const bool i32 = index_dtype == MLR_INDEX_I32;
#define MLR_QKV_WIDE(I, D)                                                                  \
  launch_wide<T, I, D>(qkv, qkv_st, bias, positions, inv_freq, slots, q_out, q_st, kc, vc, \
                       num_slots, num_tokens, hq, hkv, stream)
#define MLR_QKV_LAUNCH(I, V)                                                                  \
  launch_vec<T, I, V>(qkv, qkv_st, bias, positions, inv_freq, slots, q_out, q_st, kc, vc,   \
                      num_slots, num_tokens, hq, hkv, d, stream)
  if (wide && d == 64) {
    if (i32) MLR_QKV_WIDE(int32_t, 64); else MLR_QKV_WIDE(int64_t, 64);
  } else if (wide) {
    if (i32) MLR_QKV_WIDE(int32_t, 128); else MLR_QKV_WIDE(int64_t, 128);
  } else if (vec) {
    if (i32) MLR_QKV_LAUNCH(int32_t, kVec); else MLR_QKV_LAUNCH(int64_t, kVec);
  } else {
    if (i32) MLR_QKV_LAUNCH(int32_t, 1); else MLR_QKV_LAUNCH(int64_t, 1);
  }
#undef MLR_QKV_LAUNCH
#undef MLR_QKV_WIDE
  return check_launch("mlr_qkv_rope_write");
}

}  // namespace
}  // namespace mlr

extern "C" int mlr_qkv_rope_write(const void *qkv, int64_t qkv_stride_t, const void *bias,
                                  const int64_t *positions, const float *inv_freq,
                                  const void *slot_mapping, int index_dtype, void *q_out,
                                  int64_t q_out_stride_t, void *k_cache, void *v_cache,
                                  int64_t num_slots, int64_t num_tokens, int64_t num_q_heads,
                                  int64_t num_kv_heads, int64_t head_dim, int dtype,
                                  void *stream) {
  using namespace mlr;
  clear_error();
  MLR_REQUIRE(num_tokens >= 0, "mlr_qkv_rope_write: num_tokens must be >= 0");
  MLR_REQUIRE(num_q_heads > 0 && num_kv_heads > 0,
              "mlr_qkv_rope_write: head counts must be positive");
  MLR_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024,
              "mlr_qkv_rope_write: head_dim must be even and in (0, 1024]");
  MLR_REQUIRE((num_q_heads + 2 * num_kv_heads) * head_dim < (int64_t(1) << 30),
              "mlr_qkv_rope_write: row too wide");
  MLR_REQUIRE(qkv_stride_t >= (num_q_heads + 2 * num_kv_heads) * head_dim,
              "mlr_qkv_rope_write: qkv row stride smaller than its row");
  MLR_REQUIRE(q_out_stride_t >= num_q_heads * head_dim,
              "mlr_qkv_rope_write: q_out row stride smaller than its row");
  MLR_REQUIRE(num_slots >= 0, "mlr_qkv_rope_write: num_slots must be >= 0");
  MLR_REQUIRE(index_dtype == MLR_INDEX_I32 || index_dtype == MLR_INDEX_I64,
              "mlr_qkv_rope_write: unknown index dtype %d", index_dtype);
  if (num_tokens == 0) return MLR_OK;
  MLR_REQUIRE(qkv && positions && inv_freq && slot_mapping && q_out && k_cache && v_cache,
              "mlr_qkv_rope_write: null pointer");
  const int hq = static_cast<int>(num_q_heads), hkv = static_cast<int>(num_kv_heads);
  const int d = static_cast<int>(head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MLR_DTYPE_F32:
      return launch<float>(qkv, qkv_stride_t, bias, positions, inv_freq, slot_mapping,
                           index_dtype, q_out, q_out_stride_t, k_cache, v_cache, num_slots,
                           num_tokens, hq, hkv, d, s);
    case MLR_DTYPE_F16:
      return launch<f16_t>(qkv, qkv_stride_t, bias, positions, inv_freq, slot_mapping,
                           index_dtype, q_out, q_out_stride_t, k_cache, v_cache, num_slots,
                           num_tokens, hq, hkv, d, s);
    case MLR_DTYPE_BF16:
      return launch<bf16_t>(qkv, qkv_stride_t, bias, positions, inv_freq, slot_mapping,
                            index_dtype, q_out, q_out_stride_t, k_cache, v_cache, num_slots,
                            num_tokens, hq, hkv, d, s);
    default:
      return set_error(MLR_ERR_UNSUPPORTED, "mlr_qkv_rope_write: unsupported dtype %d", dtype);
  }
}
