// Batched single-token paged decode, split-KV in two passes.
//
// Pass 1 (split kernel): one workgroup per (sequence, KV head, split of
// tokens_per_split tokens) computes, for every query head of the KV head's
// GQA group, the split-local softmax statistics m = max_t s_t,
// l = sum_t exp(s_t - m) and acc = sum_t exp(s_t - m) v_t, and stores them in
// the FP32 workspace. Pass 2 (combine kernel) merges the splits of one
// (sequence, query head) with the log-sum-exp rule
//   M = max_s m_s,  out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s.
//
// Math follows paged_attention_decode_batch_parallel
// (kernels/reference/paged_attention.py:178-254): scores are q.k in the input
// type (the reference's matmul rounds them to the input type), multiplied by
// scale (rounded again), then an FP32 softmax over positions t < seq_len;
// positions past seq_len and padded block-table entries never contribute.
//
// bf16, fp16 and FP32 inputs with head_dim 64 or 128, at most 16 query heads
// per KV head and block_size a multiple of 16 take the matrix-core kernel in
// paged_decode_mfma.hip (one launch, splits merged in it); everything else
// takes the generic kernels below.
#include <algorithm>
#include <atomic>

#include "mlr_common.h"
#include "paged_decode.h"

namespace mlr {
namespace {

constexpr int kGenHeads = 16;       // query heads handled per generic workgroup
constexpr int kGenMaxSplit = 512;   // tokens per split the generic kernel holds

// Score as the reference computes it: the matmul output in the element type,
// times scale in FP32 opmath, rounded to the element type, then FP32.
template <typename T>
__device__ __forceinline__ float decode_score(typename Elem<T>::acc dot,
                                              double scale) {
  if constexpr (std::is_same<T, double>::value) {
    return static_cast<float>(dot * scale);
  } else {
    const float r = Elem<T>::round_acc(dot);
    return Elem<T>::round_acc(r * static_cast<float>(scale));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void decode_split_generic(DecodeParams p) {
  using E = Elem<T>;
  using Acc = typename E::acc;
  const int split = blockIdx.x;
  const int nhc = static_cast<int>(ceil_div(p.group, kGenHeads));
  const int kvh = blockIdx.y / nhc;
  const int g0 = (blockIdx.y % nhc) * kGenHeads;
  const int ng = min(kGenHeads, p.group - g0);
  const int b = blockIdx.z;

  const int64_t cap = p.max_blocks * p.block_size;
  int64_t ctx = p.ctx[b];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int64_t t0 = static_cast<int64_t>(split) * p.ts;
  if (t0 >= ctx) return;
  const int n = static_cast<int>(min<int64_t>(p.ts, ctx - t0));

  extern __shared__ __align__(16) unsigned char smem[];
  Acc *q_s = reinterpret_cast<Acc *>(smem);                       // [16][d]
  int64_t *row_s = reinterpret_cast<int64_t *>(q_s + kGenHeads * p.d);  // [ts]
  float *s_s = reinterpret_cast<float *>(row_s + p.ts);           // [16][ts]

  const T *q = static_cast<const T *>(p.q);
  const T *kc = static_cast<const T *>(p.kc);
  const T *vc = static_cast<const T *>(p.vc);
  const int head0 = kvh * p.group + g0;

  for (int i = threadIdx.x; i < ng * p.d; i += blockDim.x) {
    const int g = i / p.d, e = i % p.d;
    q_s[i] = E::to_acc(q[b * p.q_sb + (head0 + g) * p.q_sh + e]);
  }
  // Element offset of each token's K/V row for this KV head, or -1 when the
  // block-table entry is not a valid block id.
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    const int64_t pos = t0 + t;
    const int64_t blk = p.bt[b * p.bt_stride + pos / p.block_size];
    row_s[t] = (blk >= 0 && blk < p.num_blocks)
                   ? ((blk * p.block_size + pos % p.block_size) * p.hkv + kvh) * p.d
                   : -1;
  }
  __syncthreads();

  for (int i = threadIdx.x; i < n * ng; i += blockDim.x) {
    const int t = i / ng, g = i % ng;
    const int64_t r = row_s[t];
    float s = -INFINITY;
    if (r >= 0) {
      Acc dot = 0;
      const T *kr = kc + r;
      const Acc *qg = q_s + g * p.d;
      // Unrolled so that a row's loads are in flight together.
#pragma unroll 16
      for (int e = 0; e < p.d; ++e) dot += qg[e] * E::to_acc(kr[e]);
      s = decode_score<T>(dot, p.scale);
    }
    s_s[g * p.ts + t] = s;
  }
  __syncthreads();

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  for (int g = wave; g < ng; g += nw) {
    float m = -INFINITY;
    for (int t = lane; t < n; t += kWave) m = fmaxf(m, s_s[g * p.ts + t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < n; t += kWave) {
      const float e = (m == -INFINITY) ? 0.f : expf(s_s[g * p.ts + t] - m);
      s_s[g * p.ts + t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      p.ws_ml[((int64_t)b * p.hq + head0 + g) * p.split_stride + split] =
          make_float2(m, l);
    }
  }
  __syncthreads();

  // P@V: wave w takes the group's heads w, w + nw, ... (up to kGenHeads / 4
  // of them) and lane l the dimensions l, l + 64, ...; for each token the
  // wave loads the V row once, coalesced, for all its heads. Each output is
  // summed by one lane in token order. Tokens go kTok at a time, so kTok rows
  // are in flight per lane.
  constexpr int kHpw = kGenHeads / 4;
  Acc *ws_acc = static_cast<Acc *>(p.ws_acc);
  for (int e = lane; e < p.d; e += kWave) {
    Acc a[kHpw];
#pragma unroll
    for (int j = 0; j < kHpw; ++j) a[j] = 0;
    constexpr int kTok = 8;
    int t = 0;
    for (; t + kTok <= n; t += kTok) {
      Acc v[kTok];
      int64_t r[kTok];
#pragma unroll
      for (int u = 0; u < kTok; ++u) {
        r[u] = row_s[t + u];
        v[u] = r[u] >= 0 ? E::to_acc(vc[r[u] + e]) : Acc(0);
      }
#pragma unroll
      for (int u = 0; u < kTok; ++u)
#pragma unroll
        for (int j = 0; j < kHpw; ++j) {
          const int g = wave + nw * j;
          if (g < ng && r[u] >= 0) a[j] += static_cast<Acc>(s_s[g * p.ts + t + u]) * v[u];
        }
    }
    for (; t < n; ++t) {
      const int64_t r = row_s[t];
      if (r < 0) continue;
      const Acc v = E::to_acc(vc[r + e]);
#pragma unroll
      for (int j = 0; j < kHpw; ++j) {
        const int g = wave + nw * j;
        if (g < ng) a[j] += static_cast<Acc>(s_s[g * p.ts + t]) * v;
      }
    }
#pragma unroll
    for (int j = 0; j < kHpw; ++j) {
      const int g = wave + nw * j;
      if (g < ng) ws_acc[(((int64_t)b * p.hq + head0 + g) * p.split_stride + split) * p.d + e] = a[j];
    }
  }
}

// Pass 2 of the generic path: one workgroup per (query head, sequence). Each
// thread returns the partial words it read to zero (no other thread reads
// them), so the workspace is all zero again when the call ends.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine(DecodeParams p) {
  using E = Elem<T>;
  using Acc = typename E::acc;
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t cap = p.max_blocks * p.block_size;
  int64_t ctx = p.ctx[b];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int ns = static_cast<int>(ceil_div(ctx, p.ts));
  float2 *ml = p.ws_ml + ((int64_t)b * p.hq + h) * p.split_stride;

  extern __shared__ __align__(16) unsigned char smem[];
  float *w_s = reinterpret_cast<float *>(smem);  // [max_splits]
  __shared__ float red[2];

  // Global max, then per-split weights and the total normaliser.
  float m = -INFINITY;
  for (int s = threadIdx.x; s < ns; s += blockDim.x) m = fmaxf(m, ml[s].x);
  m = wave_max(m);
  __shared__ float wmax[4];
  if (threadIdx.x % kWave == 0) wmax[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float mm = wmax[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) mm = fmaxf(mm, wmax[w]);
    red[0] = mm;
  }
  __syncthreads();
  const float M = red[0];
  float l = 0.f;
  for (int s = threadIdx.x; s < ns; s += blockDim.x) {
    const float2 v = ml[s];
    const float w = (v.x == -INFINITY) ? 0.f
                    : p.ml_base2      ? exp2f(v.x - M)
                                      : expf(v.x - M);
    w_s[s] = w;
    l += w * v.y;
    ml[s] = make_float2(0.f, 0.f);
  }
  l = wave_sum(l);
  __syncthreads();
  if (threadIdx.x % kWave == 0) wmax[threadIdx.x / kWave] = l;
  __syncthreads();
  if (threadIdx.x == 0) {
    float ll = 0.f;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) ll += wmax[w];
    red[1] = ll;
  }
  __syncthreads();
  const float L = red[1];

  Acc *acc = static_cast<Acc *>(p.ws_acc) + ((int64_t)b * p.hq + h) * p.split_stride * p.d;
  T *out = static_cast<T *>(p.out) + b * p.o_sb + h * p.o_sh;
  for (int e = threadIdx.x; e < p.d; e += blockDim.x) {
    Acc a = 0;
    for (int s = 0; s < ns; ++s) {
      a += static_cast<Acc>(w_s[s]) * acc[(int64_t)s * p.d + e];
      acc[(int64_t)s * p.d + e] = Acc(0);
    }
    out[e] = E::from_acc(a / static_cast<Acc>(L));
  }
}

template <typename T>
int launch_generic(const DecodeParams &p, hipStream_t stream) {
  using Acc = typename Elem<T>::acc;
  const int nhc = static_cast<int>(ceil_div(p.group, kGenHeads));
  dim3 grid(p.max_splits, p.hkv * nhc, p.batch);
  const size_t lds = sizeof(Acc) * kGenHeads * p.d + sizeof(int64_t) * p.ts +
                     sizeof(float) * kGenHeads * p.ts;
  decode_split_generic<T><<<grid, 256, lds, stream>>>(p);
  int rc = check_launch("mlr_paged_decode(split)");
  if (rc != MLR_OK) return rc;
  return launch_combine<T>(p, stream);
}

}  // namespace

template <typename T>
int launch_combine(const DecodeParams &p, hipStream_t stream) {
  dim3 grid(p.hq, p.batch);
  const size_t lds = sizeof(float) * p.max_splits;
  decode_combine<T><<<grid, 256, lds, stream>>>(p);
  return check_launch("mlr_paged_decode(combine)");
}

template int launch_combine<bf16_t>(const DecodeParams &, hipStream_t);

int64_t default_tokens_per_split(bool mfma, int64_t head_dim, int64_t max_context, int dtype) {
  // Generic kernel: an eighth of the longest context, as a power of two in
  // [32, 256] (its scores are held in LDS), so that short contexts still
  // spread over several workgroups per (sequence, KV head). Matrix-core
  // kernel at head_dim 64 with contexts of up to 16 x 320 tokens: 320 (four
  // tiles per wave in registers and one in LDS), so a batch of long contexts
  // fits the GPU in one generation of workgroups. Otherwise at least 256
  // tokens (16 tiles, four per wave, loaded in one batch; FP32 tiles go two
  // or one per batch), and at most 16 splits per sequence: long contexts
  // then get fewer, longer splits (measured at 8 x 32K tokens: 133 us with
  // 128 splits, 108-111 us with 8-16), and the merge takes every sequence in
  // one 16-split chunk.
  if (!mfma) {
    int64_t ts = 32;
    while (ts < 256 && ts * 8 < max_context) ts *= 2;
    return ts;
  }
  if ((dtype == MLR_DTYPE_BF16 || dtype == MLR_DTYPE_F16) && head_dim == 64 &&
      max_context <= 16 * kLdsSplit64)
    return kLdsSplit64;
  const int64_t per16 = ceil_div(max_context, 16);
  return per16 <= 256 ? 256 : ceil_div(per16, 256) * 256;
}

// bf16/fp16 matrix-core kernel when the default split gives fewer work items
// (sequence, KV head, split) than the GPU has CUs: a sixteenth of the context,
// in whole 64-token steps of at least 64 tokens, up to 512-token splits; then
// 512-token splits up to 32 of them; then 32 splits. Measured on one request,
// 32 q / 8 KV heads, head_dim 128 (graphs, every call from HBM): 512 tokens
// 7.9 us against 10.0 us with two 256-token splits, 2048 tokens 9.4 against
// 10.9 us, 16K 21.5 against 22.8 us, 32K 33.8 against 37.9 us; 28/4 heads at
// 32K 28.8 against 36.6 us; 14/2 heads, head_dim 64, at 512 tokens 6.9
// against 8.6 us (two 320-token splits). Splits of one tile per wave (64
// tokens) past 512 tokens, or more than 32 splits, were slower: the merge
// then reads more chunks than the extra waves save. At most 32 splits, and
// never more than the generic kernel's default split count rounded up to the
// 16-row padding, so mlr_paged_decode_workspace_size covers it.
static int64_t sparse_tokens_per_split(int64_t max_context) {
  const int64_t per16 = ceil_div(ceil_div(max_context, 16), 64) * 64;
  if (per16 <= 512) return per16 < 64 ? 64 : per16;
  const int64_t per32 = ceil_div(ceil_div(max_context, 32), 16) * 16;
  return per32 < 512 ? 512 : per32;
}

DecodeWorkspace decode_workspace_layout(int64_t batch, int64_t hq, int64_t d,
                                        int64_t max_splits, int dtype) {
  DecodeWorkspace w;
  w.ml_offset = kFlagBytes;
  const int64_t rows = batch * hq * (ceil_div(max_splits, kSplitRowPad) * kSplitRowPad);
  const int64_t ml_bytes = rows * static_cast<int64_t>(sizeof(float2));
  w.acc_offset = w.ml_offset + (ml_bytes + 255) / 256 * 256;
  const int64_t acc_elem = dtype == MLR_DTYPE_F64 ? 8 : 4;
  w.total = w.acc_offset + rows * d * acc_elem;
  return w;
}

}  // namespace mlr

using namespace mlr;

extern "C" size_t mlr_paged_decode_workspace_size(int64_t batch,
                                                  int64_t num_q_heads,
                                                  int64_t head_dim,
                                                  int64_t max_context,
                                                  int64_t tokens_per_split,
                                                  int dtype) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_context <= 0)
    return 0;
  // The default is sized for the generic kernel's split, the smallest either
  // kernel uses by default, so it covers whichever kernel the call takes.
  const int64_t ts = tokens_per_split > 0
                         ? tokens_per_split
                         : default_tokens_per_split(false, head_dim, max_context, dtype);
  const int64_t splits = ceil_div(max_context, ts);
  return static_cast<size_t>(
      decode_workspace_layout(batch, num_q_heads, head_dim, splits, dtype).total);
}

namespace {

// The new-token rows of mlr_paged_decode_append (and, for
// mlr_paged_decode_qkv, the inverse frequencies of the fused rotary
// embedding; inv_freq == nullptr: none).
struct AppendArgs {
  const void *new_k;
  const void *new_v;
  int64_t sb, sh;
  const int64_t *slots;
  const float *inv_freq = nullptr;
};

int run_decode(const void *q, int64_t q_stride_b, int64_t q_stride_h,
               const void *k_cache, const void *v_cache, int64_t num_blocks,
               int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
               const int64_t *block_tables, int64_t block_table_stride,
               int64_t max_blocks_per_seq, const int64_t *context_lens,
               int64_t batch, int64_t num_q_heads, double scale, int dtype,
               int64_t tokens_per_split, void *workspace,
               size_t workspace_bytes, void *out, int64_t out_stride_b,
               int64_t out_stride_h, void *stream, const AppendArgs *app) {
  MLR_REQUIRE(batch > 0, "mlr_paged_decode: batch must be > 0");
  MLR_REQUIRE(num_kv_heads > 0 && num_q_heads > 0,
              "mlr_paged_decode: head counts must be > 0");
  MLR_REQUIRE(num_q_heads % num_kv_heads == 0,
              "mlr_paged_decode: num_q_heads must be divisible by num_kv_heads");
  MLR_REQUIRE(head_dim > 0 && head_dim <= 1024,
              "mlr_paged_decode: head_dim must be in [1, 1024]");
  MLR_REQUIRE(block_size > 0 && num_blocks > 0,
              "mlr_paged_decode: block_size and num_blocks must be > 0");
  MLR_REQUIRE(max_blocks_per_seq > 0,
              "mlr_paged_decode: block tables must have at least one column");
  MLR_REQUIRE(block_table_stride >= max_blocks_per_seq,
              "mlr_paged_decode: block_table_stride < max_blocks_per_seq");
  MLR_REQUIRE(q && k_cache && v_cache && block_tables && context_lens && out,
              "mlr_paged_decode: null pointer argument");
  MLR_REQUIRE(dtype_size(dtype) > 0, "mlr_paged_decode: unknown dtype %d", dtype);
  MLR_REQUIRE(batch <= 65535 && num_kv_heads * num_q_heads <= (1 << 20),
              "mlr_paged_decode: batch or head count too large for the grid");

  const int64_t max_context = max_blocks_per_seq * block_size;
  // The MFMA kernel moves 16-byte Q and K fragments and 8/16-byte V fragments.
  const bool aligned = (reinterpret_cast<uintptr_t>(q) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(k_cache) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v_cache) & 15u) == 0 &&
                       q_stride_b % 8 == 0 && q_stride_h % 8 == 0;
  // The matrix-core kernel keeps token positions in 32 bits, and the byte
  // offsets of a GQA group's q rows (group x q_stride_h elements).
  const bool mfma =
      aligned && max_context < (int64_t(1) << 31) && q_stride_h < (int64_t(1) << 20) &&
      decode_mfma_eligible(dtype, head_dim, num_q_heads / num_kv_heads, block_size);
  int64_t ts = tokens_per_split > 0 ? tokens_per_split
                                    : default_tokens_per_split(mfma, head_dim, max_context, dtype);
  if (tokens_per_split <= 0 && mfma && (dtype == MLR_DTYPE_BF16 || dtype == MLR_DTYPE_F16)) {
    const int cus = current_device_cus();
    if (cus > 0 && batch * num_kv_heads * ceil_div(max_context, ts) < cus)
      ts = sparse_tokens_per_split(max_context);
  }
  if (!mfma) {
    MLR_REQUIRE(ts <= kGenMaxSplit,
                "mlr_paged_decode: tokens_per_split %lld exceeds %d for this "
                "dtype/shape", (long long)ts, kGenMaxSplit);
    MLR_REQUIRE(head_dim <= 512,
                "mlr_paged_decode: head_dim > 512 is not supported");
  } else {
    MLR_REQUIRE(ts % 16 == 0,
                "mlr_paged_decode: tokens_per_split must be a multiple of 16");
  }
  const int64_t max_splits = ceil_div(max_context, ts);
  MLR_REQUIRE(max_splits <= 8192,
              "mlr_paged_decode: %lld splits exceed the combine limit of 8192; "
              "raise tokens_per_split", (long long)max_splits);
  const DecodeWorkspace wl =
      decode_workspace_layout(batch, num_q_heads, head_dim, max_splits, dtype);
  if (!workspace || workspace_bytes < static_cast<size_t>(wl.total)) {
    return set_error(MLR_ERR_WORKSPACE,
                     "mlr_paged_decode: workspace of %zu bytes is smaller than "
                     "the %lld bytes required",
                     workspace_bytes, (long long)wl.total);
  }
  MLR_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
              "mlr_paged_decode: workspace must be 256-byte aligned");

  DecodeParams p{};
  p.q = q;
  p.q_sb = q_stride_b;
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
  p.ctx = context_lens;
  p.batch = static_cast<int>(batch);
  p.hq = static_cast<int>(num_q_heads);
  p.group = static_cast<int>(num_q_heads / num_kv_heads);
  p.scale = scale;
  p.ts = static_cast<int>(ts);
  p.max_splits = static_cast<int>(max_splits);
  p.split_stride = static_cast<int>(ceil_div(max_splits, kSplitRowPad) * kSplitRowPad);
  p.ws_flag = static_cast<uint32_t *>(workspace);
  p.ws_ml = reinterpret_cast<float2 *>(static_cast<unsigned char *>(workspace) + wl.ml_offset);
  p.ws_acc = static_cast<unsigned char *>(workspace) + wl.acc_offset;
  p.ml_base2 = mfma ? 1 : 0;
  p.dtype = dtype;
  p.out = out;
  p.o_sb = out_stride_b;
  p.o_sh = out_stride_h;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (app != nullptr) {
    MLR_REQUIRE(app->new_k && app->new_v && app->slots,
                "mlr_paged_decode_append: null new_k, new_v or slot_mapping");
    // The MFMA kernel moves 16-byte K and 8/16-byte V fragments of the rows.
    const bool rows_aligned = (reinterpret_cast<uintptr_t>(app->new_k) & 15u) == 0 &&
                              (reinterpret_cast<uintptr_t>(app->new_v) & 15u) == 0 &&
                              app->sb % 8 == 0 && app->sh % 8 == 0;
    if (app->inv_freq != nullptr) {
      // The fused rotary embedding exists on the matrix-core kernel only.
      MLR_REQUIRE(mfma && (dtype == MLR_DTYPE_BF16 || dtype == MLR_DTYPE_F16) && rows_aligned,
                  "mlr_paged_decode_qkv: needs bf16 or fp16, head_dim 64 or 128, at most 16 query "
                  "heads per KV head, block_size a multiple of 16 and 16-byte aligned rows");
      p.inv_freq = app->inv_freq;
    }
    if (mfma && rows_aligned) {
      p.new_k = app->new_k;
      p.new_v = app->new_v;
      p.new_sb = app->sb;
      p.new_sh = app->sh;
      p.new_slots = app->slots;
      p.kc_w = const_cast<void *>(k_cache);
      p.vc_w = const_cast<void *>(v_cache);
    } else {
      const int rc = mlr_kv_write(app->new_k, app->new_v, dtype, batch, app->sb,
                                  app->sh, 1, app->sb, app->sh, 1, app->slots,
                                  MLR_INDEX_I64, const_cast<void *>(k_cache),
                                  const_cast<void *>(v_cache), dtype,
                                  num_blocks * block_size, num_kv_heads, head_dim,
                                  stream);
      if (rc != MLR_OK) return rc;
    }
  }
  if (mfma) return launch_decode_mfma(p, s);
  switch (dtype) {
    case MLR_DTYPE_F32: return launch_generic<float>(p, s);
    case MLR_DTYPE_F16: return launch_generic<f16_t>(p, s);
    case MLR_DTYPE_BF16: return launch_generic<bf16_t>(p, s);
    case MLR_DTYPE_F64: return launch_generic<double>(p, s);
    default: return set_error(MLR_ERR_INVALID, "mlr_paged_decode: bad dtype");
  }
}

}  // namespace

extern "C" int mlr_paged_decode(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k_cache,
    const void *v_cache, int64_t num_blocks, int64_t block_size,
    int64_t num_kv_heads, int64_t head_dim, const int64_t *block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq,
    const int64_t *context_lens, int64_t batch, int64_t num_q_heads,
    double scale, int dtype, int64_t tokens_per_split, void *workspace,
    size_t workspace_bytes, void *out, int64_t out_stride_b,
    int64_t out_stride_h, void *stream) {
  clear_error();
  return run_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                    block_size, num_kv_heads, head_dim, block_tables,
                    block_table_stride, max_blocks_per_seq, context_lens, batch,
                    num_q_heads, scale, dtype, tokens_per_split, workspace,
                    workspace_bytes, out, out_stride_b, out_stride_h, stream,
                    nullptr);
}

extern "C" int mlr_paged_decode_append(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, void *k_cache,
    void *v_cache, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
    int64_t head_dim, const int64_t *block_tables, int64_t block_table_stride,
    int64_t max_blocks_per_seq, const int64_t *context_lens, int64_t batch,
    int64_t num_q_heads, double scale, int dtype, int64_t tokens_per_split,
    void *workspace, size_t workspace_bytes, const void *new_k,
    const void *new_v, int64_t new_stride_b, int64_t new_stride_h,
    const int64_t *slot_mapping, void *out, int64_t out_stride_b,
    int64_t out_stride_h, void *stream) {
  clear_error();
  const AppendArgs app{new_k, new_v, new_stride_b, new_stride_h, slot_mapping};
  return run_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                    block_size, num_kv_heads, head_dim, block_tables,
                    block_table_stride, max_blocks_per_seq, context_lens, batch,
                    num_q_heads, scale, dtype, tokens_per_split, workspace,
                    workspace_bytes, out, out_stride_b, out_stride_h, stream,
                    &app);
}

extern "C" int mlr_paged_decode_qkv(
    const void *qkv, int64_t qkv_stride_b, const float *inv_freq,
    void *k_cache, void *v_cache, int64_t num_blocks, int64_t block_size,
    int64_t num_kv_heads, int64_t head_dim, const int64_t *block_tables,
    int64_t block_table_stride, int64_t max_blocks_per_seq, const int64_t *context_lens,
    const int64_t *slot_mapping, int64_t batch, int64_t num_q_heads, double scale,
    int dtype, int64_t tokens_per_split, void *workspace, size_t workspace_bytes, void *out,
    int64_t out_stride_b, int64_t out_stride_h, void *stream) {
  clear_error();
  MLR_REQUIRE(qkv && inv_freq, "mlr_paged_decode_qkv: null qkv or inv_freq");
  MLR_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0,
              "mlr_paged_decode_qkv: head counts and head_dim must be > 0");
  MLR_REQUIRE(qkv_stride_b >= (num_q_heads + 2 * num_kv_heads) * head_dim,
              "mlr_paged_decode_qkv: qkv row stride smaller than its row");
  const size_t esz = static_cast<size_t>(dtype_size(dtype));
  MLR_REQUIRE(esz > 0, "mlr_paged_decode_qkv: unknown dtype %d", dtype);
  const unsigned char *base = static_cast<const unsigned char *>(qkv);
  AppendArgs app{base + esz * static_cast<size_t>(num_q_heads * head_dim),
                 base + esz * static_cast<size_t>((num_q_heads + num_kv_heads) * head_dim),
                 qkv_stride_b, head_dim, slot_mapping};
  app.inv_freq = inv_freq;
  return run_decode(qkv, qkv_stride_b, head_dim, k_cache, v_cache, num_blocks, block_size,
                    num_kv_heads, head_dim, block_tables, block_table_stride,
                    max_blocks_per_seq, context_lens, batch, num_q_heads, scale, dtype,
                    tokens_per_split, workspace, workspace_bytes, out, out_stride_b,
                    out_stride_h, stream, &app);
}

// ---------------------------------------------------------------------------
// mlr_paged_decode_append_static: the decode step with the library's own
// scratch instead of a caller workspace, for callers that cannot allocate.
// ---------------------------------------------------------------------------
namespace {

// Decode scratch of the library on every GPU it runs on: the flag region and
// the split partials of one call (8 MiB covers, for instance, 64 sequences x
// 14 query heads x 16 splits at head_dim 64). Each device holds its own copy
// until the process ends. Static device memory starts zeroed, as a decode
// workspace must; every call leaves it zero again.
constexpr size_t kStaticScratchBytes = size_t(8) << 20;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxScratchDevices];

// The device address of `scratch` on the current device, looked up once per
// device with that device current. In host code the array's name is only a
// stand-in for the symbol; kernels must be given this address.
int scratch_address(void **out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return set_error(MLR_ERR_HIP, "mlr_paged_decode_append_static: hipGetDevice failed: %s",
                     hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(MLR_ERR_UNSUPPORTED,
                     "mlr_paged_decode_append_static: device %d is past the %d devices "
                     "the library keeps scratch addresses for", dev, kMaxScratchDevices);
  void *ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return set_error(MLR_ERR_HIP,
                       "mlr_paged_decode_append_static: hipGetSymbolAddress(scratch) "
                       "failed on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);  // same value from any thread
  }
  *out = ptr;
  return MLR_OK;
}

}  // namespace

extern "C" int mlr_paged_decode_append_static(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, void *k_cache,
    void *v_cache, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
    int64_t head_dim, const int64_t *block_tables, int64_t block_table_stride,
    int64_t max_blocks_per_seq, const int64_t *context_lens, int64_t batch,
    int64_t num_q_heads, double scale, int dtype, int64_t tokens_per_split,
    const void *new_k, const void *new_v, int64_t new_stride_b, int64_t new_stride_h,
    const int64_t *slot_mapping, void *out, int64_t out_stride_b,
    int64_t out_stride_h, void *stream) {
  clear_error();
  void *ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc != MLR_OK) return rc;
  const AppendArgs app{new_k, new_v, new_stride_b, new_stride_h, slot_mapping};
  rc = run_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks, block_size,
                  num_kv_heads, head_dim, block_tables, block_table_stride,
                  max_blocks_per_seq, context_lens, batch, num_q_heads, scale, dtype,
                  tokens_per_split, ws, kStaticScratchBytes, out, out_stride_b,
                  out_stride_h, stream, &app);
  if (rc == MLR_ERR_WORKSPACE) {
    char why[384];
    snprintf(why, sizeof(why), "%s", mlr_last_error());
    return set_error(MLR_ERR_WORKSPACE,
                     "mlr_paged_decode_append_static: these sizes need more decode scratch "
                     "than the library's %zu-byte array (%s); call mlr_paged_decode_append "
                     "with a workspace instead", kStaticScratchBytes, why);
  }
  return rc;
}

// ---------------------------------------------------------------------------
// Merge-failure check and recovery of a decode workspace (or of the static
// scratch): read the flag word; when it is set, zero the whole workspace.
// ---------------------------------------------------------------------------
namespace {

// Zeroes `bytes` bytes at p (16-byte aligned): 16-byte stores, then the tail.
__global__ __launch_bounds__(256) void zero_bytes(unsigned char *p, size_t bytes) {
  const size_t n16 = bytes / 16;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    reinterpret_cast<uint4 *>(p)[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && threadIdx.x < bytes % 16) p[16 * n16 + threadIdx.x] = 0;
}

int check_and_clear(void *ws, size_t bytes, hipStream_t s, const char *what) {
  MLR_REQUIRE(ws != nullptr && bytes >= static_cast<size_t>(kFlagBytes),
              "%s: the workspace must hold at least its %lld-byte flag region", what,
              (long long)kFlagBytes);
  MLR_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 255u) == 0,
              "%s: workspace must be 256-byte aligned", what);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing(s, &cap);
  if (err != hipSuccess)
    return set_error(MLR_ERR_HIP, "%s: hipStreamIsCapturing failed: %s", what,
                     hipGetErrorString(err));
  MLR_REQUIRE(cap == hipStreamCaptureStatusNone,
              "%s: the stream is being captured; the check synchronises and must run "
              "outside capture", what);
  uint32_t flag = 0;
  err = hipMemcpyAsync(&flag, ws, sizeof(flag), hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  if (err != hipSuccess)
    return set_error(MLR_ERR_HIP, "%s: reading the flag word failed: %s", what,
                     hipGetErrorString(err));
  if (flag == 0u) return MLR_OK;
  const size_t blocks = std::min<size_t>(1024, (bytes / 16 + 255) / 256 + 1);
  zero_bytes<<<dim3(static_cast<unsigned>(blocks)), 256, 0, s>>>(static_cast<unsigned char *>(ws),
                                                                   bytes);
  int rc = check_launch(what);
  if (rc != MLR_OK) return rc;
  err = hipStreamSynchronize(s);
  if (err != hipSuccess)
    return set_error(MLR_ERR_HIP, "%s: clearing the workspace failed: %s", what,
                     hipGetErrorString(err));
  return set_error(MLR_ERR_MERGE,
                   "%s: a single-launch split merge gave up waiting for its partial results; "
                   "the multi-split decode outputs computed on this workspace since then are "
                   "NaN. The workspace has been cleared and can be used again.", what);
}

}  // namespace

extern "C" int mlr_paged_decode_workspace_check(void *workspace, size_t workspace_bytes,
                                                void *stream) {
  clear_error();
  return check_and_clear(workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                         "mlr_paged_decode_workspace_check");
}

extern "C" int mlr_paged_decode_static_check(void *stream) {
  clear_error();
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != MLR_OK) return rc;
  return check_and_clear(ws, kStaticScratchBytes, static_cast<hipStream_t>(stream),
                         "mlr_paged_decode_static_check");
}
