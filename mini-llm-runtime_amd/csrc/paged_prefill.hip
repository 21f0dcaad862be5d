// Paged chunk-prefill attention: generic (any dtype, head_dim <= 256) kernel
// and the C-ABI entry points.
//
// Math follows paged_attention_prefill_chunk_tiled
// (kernels/reference/paged_attention.py:346-434): for query i of a chunk
// starting at absolute position prefix_len, keys at positions
// p <= prefix_len + i are visible (:414-418); scores are q.k rounded to the
// input type and scaled (:411-413), softmax statistics and P@V run in FP32
// (:415-431) and the output is rounded once to the input type (:433-434).
//
// Generic kernel: one workgroup per (sequence, query head, 32-query tile);
// eight lanes share one query, each owning head_dim/8 of its dimensions, and
// the workgroup streams the keys the tile can see through LDS in tiles of
// up to 64 keys, with a per-key online-softmax update.
#include "paged_prefill.h"

namespace mlr {
namespace {

constexpr int kTpq = 8;             // lanes per query
constexpr int kBq = 256 / kTpq;     // queries per workgroup

template <typename T>
__device__ __forceinline__ float prefill_score(typename Elem<T>::acc dot,
                                               double scale) {
  if constexpr (std::is_same<T, double>::value) {
    return static_cast<float>(dot * scale);
  } else {
    const float r = Elem<T>::round_acc(dot);
    return Elem<T>::round_acc(r * static_cast<float>(scale));
  }
}

template <typename T, int DPT>
__global__ __launch_bounds__(256) void prefill_generic(PrefillParams p,
                                                       int bk) {
  using E = Elem<T>;
  using Acc = typename E::acc;
  const int seq = blockIdx.z, h = blockIdx.y, qt = blockIdx.x;
  const int kvh = h / p.group;
  const SeqRange r = seq_range(p, seq);
  const int64_t qi0 = static_cast<int64_t>(qt) * kBq;
  if (qi0 >= r.qlen) return;  // uniform over the workgroup

  const int tid = threadIdx.x, sub = tid % kTpq;
  const int64_t qi = qi0 + tid / kTpq;
  const bool qvalid = qi < r.qlen;
  const int64_t qpos = r.prefix + qi;
  // Keys this tile can see: [0, prefix + min(qlen, qi0 + kBq)).
  const int64_t kv_end = r.prefix + min<int64_t>(r.qlen, qi0 + kBq);

  const T *qp = static_cast<const T *>(p.q) + (r.q0 + (qvalid ? qi : 0)) * p.q_st +
                (int64_t)h * p.q_sh;
  Acc qreg[DPT];
  float acc[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) {
    const int e = sub + kTpq * i;
    qreg[i] = (qvalid && e < p.d) ? E::to_acc(qp[e]) : Acc(0);
    acc[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;

  extern __shared__ __align__(16) unsigned char smem[];
  Acc *k_s = reinterpret_cast<Acc *>(smem);                      // [bk][d]
  float *v_s = reinterpret_cast<float *>(k_s + (int64_t)bk * p.d);  // [bk][d]
  int64_t *row_s = reinterpret_cast<int64_t *>(v_s + (int64_t)bk * p.d);  // [bk]

  const T *kc = static_cast<const T *>(p.kc);
  const T *vc = static_cast<const T *>(p.vc);
  const int64_t *bt_row = p.bt + seq * p.bt_stride;

  for (int64_t kt = 0; kt < kv_end; kt += bk) {
    const int nk = static_cast<int>(min<int64_t>(bk, kv_end - kt));
    __syncthreads();
    for (int j = tid; j < nk; j += blockDim.x) {
      const int64_t pos = kt + j;
      const int64_t blk = bt_row[pos / p.block_size];
      row_s[j] = (blk >= 0 && blk < p.num_blocks)
                     ? ((blk * p.block_size + pos % p.block_size) * p.hkv + kvh) * p.d
                     : -1;
    }
    __syncthreads();
    for (int i = tid; i < nk * p.d; i += blockDim.x) {
      const int j = i / p.d, e = i % p.d;
      const int64_t row = row_s[j];
      k_s[i] = row >= 0 ? E::to_acc(kc[row + e]) : Acc(0);
      v_s[i] = row >= 0 ? static_cast<float>(E::to_acc(vc[row + e])) : 0.f;
    }
    __syncthreads();
    for (int j = 0; j < nk; ++j) {
      Acc part = 0;
#pragma unroll
      for (int i = 0; i < DPT; ++i) {
        const int e = sub + kTpq * i;
        if (e < p.d) part += qreg[i] * k_s[j * p.d + e];
      }
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      const bool vis = qvalid && (kt + j <= qpos) && row_s[j] >= 0;
      if (vis) {
        const float s = prefill_score<T>(part, p.scale);
        const float mn = fmaxf(m, s);
        const float alpha = (m == -INFINITY) ? 0.f : expf(m - mn);
        const float pe = expf(s - mn);
        l = l * alpha + pe;
#pragma unroll
        for (int i = 0; i < DPT; ++i) {
          const int e = sub + kTpq * i;
          if (e < p.d) acc[i] = acc[i] * alpha + pe * v_s[j * p.d + e];
        }
        m = mn;
      }
    }
  }

  if (qvalid) {
    T *op = static_cast<T *>(p.out) + (r.q0 + qi) * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
      const int e = sub + kTpq * i;
      if (e < p.d) op[e] = E::from_f32(acc[i] / l);
    }
  }
}

template <typename T>
int launch_generic(const PrefillParams &p, int64_t max_qlen,
                   hipStream_t stream) {
  using Acc = typename Elem<T>::acc;
  // Key tile: as many keys as fit 48 KiB of LDS, at most 64.
  const int64_t per_key = (int64_t)p.d * (sizeof(Acc) + sizeof(float)) + 8;
  int bk = 64;
  while (bk > 8 && bk * per_key > 48 * 1024) bk /= 2;
  const size_t lds = bk * per_key;
  dim3 grid(static_cast<unsigned>(ceil_div(max_qlen, kBq)), p.hq, p.num_seqs);
  const int dpt = static_cast<int>(ceil_div(p.d, kTpq));
  if (dpt <= 1) {
    prefill_generic<T, 1><<<grid, 256, lds, stream>>>(p, bk);
  } else if (dpt <= 2) {
    prefill_generic<T, 2><<<grid, 256, lds, stream>>>(p, bk);
  } else if (dpt <= 4) {
    prefill_generic<T, 4><<<grid, 256, lds, stream>>>(p, bk);
  } else if (dpt <= 8) {
    prefill_generic<T, 8><<<grid, 256, lds, stream>>>(p, bk);
  } else if (dpt <= 16) {
    prefill_generic<T, 16><<<grid, 256, lds, stream>>>(p, bk);
  } else {
    prefill_generic<T, 32><<<grid, 256, lds, stream>>>(p, bk);
  }
  return check_launch("mlr_paged_prefill");
}

int run_prefill(const PrefillParams &params, int dtype, int64_t max_qlen,
                hipStream_t stream) {
  if (max_qlen <= 0) return MLR_OK;
  PrefillParams p = params;
  p.bs_log2 = log2_if_pow2(p.block_size);
  if (prefill_mfma_eligible(p, dtype))
    return launch_prefill_mfma(p, dtype, max_qlen, stream);
  if (prefill_f32_eligible(p, dtype)) return launch_prefill_f32(p, max_qlen, stream);
  switch (dtype) {
    case MLR_DTYPE_F32: return launch_generic<float>(p, max_qlen, stream);
    case MLR_DTYPE_F16: return launch_generic<f16_t>(p, max_qlen, stream);
    case MLR_DTYPE_BF16: return launch_generic<bf16_t>(p, max_qlen, stream);
    case MLR_DTYPE_F64: return launch_generic<double>(p, max_qlen, stream);
    default: return set_error(MLR_ERR_INVALID, "mlr_paged_prefill: bad dtype");
  }
}

int check_common(const void *q, const void *k_cache, const void *v_cache,
                 int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                 int64_t head_dim, int64_t num_q_heads, int dtype,
                 const void *out) {
  MLR_REQUIRE(num_kv_heads > 0 && num_q_heads > 0,
              "mlr_paged_prefill: head counts must be > 0");
  MLR_REQUIRE(num_q_heads % num_kv_heads == 0,
              "mlr_paged_prefill: num_q_heads must be divisible by num_kv_heads");
  MLR_REQUIRE(head_dim > 0 && head_dim <= 256,
              "mlr_paged_prefill: head_dim must be in [1, 256]");
  MLR_REQUIRE(block_size > 0 && num_blocks > 0,
              "mlr_paged_prefill: block_size and num_blocks must be > 0");
  MLR_REQUIRE(num_q_heads <= 65535, "mlr_paged_prefill: too many query heads");
  MLR_REQUIRE(q && k_cache && v_cache && out,
              "mlr_paged_prefill: null pointer argument");
  MLR_REQUIRE(dtype_size(dtype) > 0, "mlr_paged_prefill: unknown dtype %d",
              dtype);
  return MLR_OK;
}

}  // namespace
}  // namespace mlr

using namespace mlr;

extern "C" int mlr_paged_prefill(
    const void *q, int64_t q_stride_t, int64_t q_stride_h, const void *k_cache,
    const void *v_cache, int64_t num_blocks, int64_t block_size,
    int64_t num_kv_heads, int64_t head_dim, const int64_t *block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq,
    const int64_t *query_start_loc, const int64_t *context_lens,
    int64_t num_seqs, int64_t max_query_len, int64_t num_q_heads, double scale,
    int dtype, int64_t kv_tile, void *out, int64_t out_stride_t,
    int64_t out_stride_h, void *stream) {
  clear_error();
  int rc = check_common(q, k_cache, v_cache, num_blocks, block_size,
                        num_kv_heads, head_dim, num_q_heads, dtype, out);
  if (rc != MLR_OK) return rc;
  MLR_REQUIRE(num_seqs > 0 && num_seqs <= 65535,
              "mlr_paged_prefill: num_seqs must be in [1, 65535]");
  MLR_REQUIRE(max_query_len >= 0, "mlr_paged_prefill: max_query_len < 0");
  MLR_REQUIRE(max_blocks_per_seq > 0 && block_table_stride >= max_blocks_per_seq,
              "mlr_paged_prefill: bad block table width/stride");
  MLR_REQUIRE(block_tables && query_start_loc && context_lens,
              "mlr_paged_prefill: null metadata pointer");
  PrefillParams p{};
  p.q = q;
  p.q_st = q_stride_t;
  p.q_sh = q_stride_h;
  p.kc = k_cache;
  p.vc = v_cache;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.hkv = static_cast<int>(num_kv_heads);
  p.d = static_cast<int>(head_dim);
  p.bt = block_tables;
  p.bt_stride = block_table_stride;
  p.max_blocks = max_blocks_per_seq;
  p.qsl = query_start_loc;
  p.ctx = context_lens;
  p.num_seqs = static_cast<int>(num_seqs);
  p.hq = static_cast<int>(num_q_heads);
  p.group = static_cast<int>(num_q_heads / num_kv_heads);
  p.scale = scale;
  p.kv_tile = static_cast<int>(kv_tile);
  p.out = out;
  p.o_st = out_stride_t;
  p.o_sh = out_stride_h;
  return run_prefill(p, dtype, max_query_len, static_cast<hipStream_t>(stream));
}

extern "C" int mlr_paged_prefill_chunk(
    const void *q, int64_t q_stride_t, int64_t q_stride_h, const void *k_cache,
    const void *v_cache, int64_t num_blocks, int64_t block_size,
    int64_t num_kv_heads, int64_t head_dim, const int64_t *block_table,
    int64_t block_table_len, int64_t prefix_len, int64_t context_len,
    int64_t num_q_heads, double scale, int dtype, int64_t kv_tile, void *out,
    int64_t out_stride_t, int64_t out_stride_h, void *stream) {
  clear_error();
  int rc = check_common(q, k_cache, v_cache, num_blocks, block_size,
                        num_kv_heads, head_dim, num_q_heads, dtype, out);
  if (rc != MLR_OK) return rc;
  MLR_REQUIRE(prefix_len >= 0, "mlr_paged_prefill_chunk: prefix_len < 0");
  MLR_REQUIRE(context_len > prefix_len,
              "mlr_paged_prefill_chunk: context_len must exceed prefix_len");
  MLR_REQUIRE(block_table && block_table_len > 0,
              "mlr_paged_prefill_chunk: empty block table");
  MLR_REQUIRE(ceil_div(context_len, block_size) <= block_table_len,
              "mlr_paged_prefill_chunk: block_table does not cover context_len");
  PrefillParams p{};
  p.q = q;
  p.q_st = q_stride_t;
  p.q_sh = q_stride_h;
  p.kc = k_cache;
  p.vc = v_cache;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.hkv = static_cast<int>(num_kv_heads);
  p.d = static_cast<int>(head_dim);
  p.bt = block_table;
  p.bt_stride = block_table_len;
  p.max_blocks = block_table_len;
  p.qsl = nullptr;
  p.ctx = nullptr;
  p.s_qlen = context_len - prefix_len;
  p.s_ctx = context_len;
  p.num_seqs = 1;
  p.hq = static_cast<int>(num_q_heads);
  p.group = static_cast<int>(num_q_heads / num_kv_heads);
  p.scale = scale;
  p.kv_tile = static_cast<int>(kv_tile);
  p.out = out;
  p.o_st = out_stride_t;
  p.o_sh = out_stride_h;
  return run_prefill(p, dtype, p.s_qlen, static_cast<hipStream_t>(stream));
}
