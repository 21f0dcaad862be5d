// bf16 paged chunk prefill on gfx950 matrix cores.
//
// One workgroup = 64 queries of one query head (four waves x 16 queries).
// Keys stream in tiles of kBN positions through two LDS stages: while a tile
// is being used, the next tile's rows are already in flight from HBM into
// registers, and the block ids of the tile after that are in flight too.
//
// Per tile and wave (16 queries x kBN keys), with v_mfma_f32_16x16x32_bf16:
//   S^T[16 keys x 16 queries] = K[16 keys x D] . Q^T[D x 16 queries]
//       A = K rows from LDS (row-major, rows padded by 16 bytes so the 16 row
//       reads of one instruction fall in distinct banks); B = Q^T fragments
//       held in registers for the whole kernel.
//   base-2 online softmax in FP32: lane l owns query l%16 and keys
//       4(l/16)..+3 of each 16-key block; the row max is two cross-row
//       shuffles. The running max moves only when a tile raises it by more
//       than kLazy (base-2 units): until then the accumulators keep their
//       scale and probabilities may reach 2^kLazy (exact either way, since
//       numerator and denominator share the reference point).
//   O^T[D x 16 queries] += V^T[D x 32 keys] . P^T[32 keys x 16 queries]
//       B = P^T straight from the S^T registers of two 16-key blocks (k slot
//       8g+i <-> key 16*(2kp + i/4) + 4g + i%4), rounded to bf16; A = V^T,
//       read from the row-major V tile with ds_read_b64_tr_b16 (two per
//       MFMA), which transposes 16-bit elements across 16 lanes.
// Causal masking (key position <= query position, both absolute) is applied
// only on tiles that reach the workgroup's first query position; keys past
// the last position any of its queries can see are neither loaded nor used.
//
// Numerics follow paged_attention_prefill_chunk_tiled
// (kernels/reference/paged_attention.py:346-434): FP32 softmax statistics
// and FP32 accumulation of P@V, one rounding of the output. P is rounded to
// bf16 as the MFMA operand, and the scores are not rounded to bf16 first
// (the reference rounds q.k to bf16 at :411-413); both stay far inside the
// 2e-2 tolerance the reference's own bf16 tests use.
#include "paged_prefill.h"

namespace mlr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_t;    // LDS bytes
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;
constexpr int kBM = 64;  // queries per workgroup

template <int D, int BN>
struct PrefillCfg {
  static constexpr int kKRow = D * 2 + 16;    // bytes per K row in LDS
  static constexpr int kVRow = D * 2 + 16;    // bytes per V row in LDS
  static constexpr int kKBytes = BN * kKRow;
  static constexpr int kVBytes = BN * kVRow;
  static constexpr int kStage = kKBytes + kVBytes;
  static constexpr int kTpk = 256 / BN;          // loader threads per key
  static constexpr int kDpt = D / kTpk;          // dims per loader thread
  static constexpr int kChunks = kDpt / 8;       // 16-byte chunks per thread
  static_assert(kChunks >= 1, "tile too large for this head_dim");
};

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16 (round to nearest even): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

template <int D, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void prefill_mfma(PrefillParams p) {
  using C = PrefillCfg<D, BN>;
  constexpr int QS = D / 32;   // k-steps of S^T
  constexpr int NB = D / 16;   // 16-dim blocks of O^T
  constexpr int KB = BN / 16;  // 16-key blocks per tile
  constexpr int KP = BN / 32;  // 32-key steps of P@V
  extern __shared__ __align__(16) unsigned char smem[];

  // Grid (query head, sequence, query tile), query tiles last-first: the
  // tiles with the most keys start first.
  const int h = blockIdx.x, seq = blockIdx.y;
  const int qt = static_cast<int>(gridDim.z) - 1 - static_cast<int>(blockIdx.z);
  const int kvh = h / p.group;
  const SeqRange r = seq_range(p, seq);
  const int64_t q0 = static_cast<int64_t>(qt) * kBM;
  if (q0 >= r.qlen) return;  // uniform

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m16 = lane & 15, g = lane >> 4;

  const int64_t kv_end = r.prefix + min<int64_t>(r.qlen, q0 + kBM);  // keys used
  const int ntiles = static_cast<int>(ceil_div(kv_end, BN));
  // Tiles below nfull end before the first query position: no mask needed.
  const int nfull = static_cast<int>((r.prefix + q0) / BN);

  // Q^T fragments: lane l holds Q[query 16w + l%16][32s + 8g .. +8).
  const int64_t qi = q0 + 16 * w + m16;
  const bool q_ok = qi < r.qlen;
  const int64_t qpos = r.prefix + qi;
  const int qpos32 = static_cast<int>(qpos);
  const uint16_t *qrow = static_cast<const uint16_t *>(p.q) +
                         (r.q0 + (q_ok ? qi : 0)) * p.q_st + (int64_t)h * p.q_sh;
  bf16x8_t qf[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) {
    const uint4 raw = q_ok ? *reinterpret_cast<const uint4 *>(qrow + 32 * s + 8 * g)
                           : make_uint4(0, 0, 0, 0);
    qf[s] = __builtin_bit_cast(bf16x8_t, raw);
  }

  // Loader role: key kk of a tile, dims [dc, dc + kDpt).
  const int kk = tid / C::kTpk;
  const int dc = (tid % C::kTpk) * C::kDpt;
  const uint16_t *kc = static_cast<const uint16_t *>(p.kc);
  const uint16_t *vc = static_cast<const uint16_t *>(p.vc);
  const int64_t *bt_row = p.bt + seq * p.bt_stride;
  // Positions fit 32 bits; block_size is a power of two on this path.
  const int bs_log2 = p.bs_log2;
  const int bs_mask = (1 << bs_log2) - 1;
  const int kv_end32 = static_cast<int>(kv_end);
  auto block_of = [&](int t) -> int64_t {
    const int pos = t * BN + kk;
    if (pos >= kv_end32) return -1;
    const int64_t blk = bt_row[pos >> bs_log2];
    return (blk >= 0 && blk < p.num_blocks) ? blk : -1;
  };
  uint4 kreg[C::kChunks], vreg[C::kChunks];
  auto load_rows = [&](int t, int64_t blk) {
    const int pos = t * BN + kk;
    const int64_t off =
        (((blk << bs_log2) + (pos & bs_mask)) * p.hkv + kvh) * int64_t(D) + dc;
#pragma unroll
    for (int c = 0; c < C::kChunks; ++c) {
      // Absent keys load zeros: masked keys must not carry NaN into P@V.
      kreg[c] = blk >= 0 ? *reinterpret_cast<const uint4 *>(kc + off + 8 * c)
                         : make_uint4(0, 0, 0, 0);
      vreg[c] = blk >= 0 ? *reinterpret_cast<const uint4 *>(vc + off + 8 * c)
                         : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_rows = [&](int stage) {
    unsigned char *base = smem + stage * C::kStage;
#pragma unroll
    for (int c = 0; c < C::kChunks; ++c) {
      *reinterpret_cast<uint4 *>(base + kk * C::kKRow + (dc + 8 * c) * 2) = kreg[c];
      *reinterpret_cast<uint4 *>(base + C::kKBytes + kk * C::kVRow + (dc + 8 * c) * 2) =
          vreg[c];
    }
  };

  const float c2 = static_cast<float>(p.scale) * kLog2e;  // score -> base-2
  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int t, int stage) {
    const unsigned char *base = smem + stage * C::kStage;
    const int tile0 = t * BN;
    f32x4_t s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      s[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(
            base + (16 * kb + m16) * C::kKRow + (32 * st + 8 * g) * 2);
        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[st], s[kb], 0, 0, 0);
      }
    }
    if (t >= nfull) {  // diagonal tile: key position <= query position
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tile0 + 16 * kb + 4 * g + i > qpos32) s[kb][i] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      mx = fmaxf(fmaxf(mx, fmaxf(s[kb][0], s[kb][1])), fmaxf(s[kb][2], s[kb][3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_tile = mx * c2;
    // Move the reference point only when the tile exceeds it by > kLazy.
    const bool move = m_tile > m_run + kLazy;
    if (__any(move)) {
      const float m_new = move ? m_tile : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 1 if kept
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < NB; ++n) acc[n] *= alpha;
      m_run = m_new;
    }
    float pr[KB][4];
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[kb][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], c2, -m_run));
        psum += pr[kb][i];
      }
    l_run += psum;
#pragma unroll
    for (int kp = 0; kp < KP; ++kp) {
      const bf16x8_t pb = __builtin_bit_cast(
          bf16x8_t,
          make_uint4(bf16_pack2(pr[2 * kp][0], pr[2 * kp][1]),
                     bf16_pack2(pr[2 * kp][2], pr[2 * kp][3]),
                     bf16_pack2(pr[2 * kp + 1][0], pr[2 * kp + 1][1]),
                     bf16_pack2(pr[2 * kp + 1][2], pr[2 * kp + 1][3])));
      // A = V^T from the row-major V tile with ds_read_b64_tr_b16: in each
      // 16-lane group, lane r points at V[kbase + r/4][dim0 + 4(r%4) .. +4)
      // and lane i receives V[kbase + 0..3][dim0 + i] (kbase = 32kp + 4g,
      // then +16 for slots 4..7; dim0 = 16n).
      lds_t *vrow0 = (lds_t *)(base + C::kKBytes +
                               (32 * kp + 4 * g + (m16 >> 2)) * C::kVRow + (m16 & 3) * 8);
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const s16x4_t lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vrow0 + 32 * n));
        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_t *)(vrow0 + 32 * n + 16 * C::kVRow));
        const bf16x8_t a = __builtin_bit_cast(
            bf16x8_t, make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                 __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y));
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, acc[n], 0, 0, 0);
      }
    }
  };

  // Pipeline: block ids two tiles ahead, rows one tile ahead, LDS stage t % 2.
  int64_t blk_next = ntiles > 1 ? block_of(1) : -1;
  load_rows(0, block_of(0));
  store_rows(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int64_t blk_after = t + 2 < ntiles ? block_of(t + 2) : -1;
    if (t + 1 < ntiles) load_rows(t + 1, blk_next);
    compute(t, t & 1);
    if (t + 1 < ntiles) store_rows((t + 1) & 1);
    __syncthreads();
    blk_next = blk_after;
  }

  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (q_ok) {
    const float inv = 1.f / l_run;
    uint16_t *orow = static_cast<uint16_t *>(p.out) + (r.q0 + qi) * p.o_st +
                     (int64_t)h * p.o_sh;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      // Lane l holds O[query][dims 16n + 4g + i].
      const uint2 v = make_uint2(
          (uint32_t)float_to_bf16_bits(acc[n][0] * inv) |
              ((uint32_t)float_to_bf16_bits(acc[n][1] * inv) << 16),
          (uint32_t)float_to_bf16_bits(acc[n][2] * inv) |
              ((uint32_t)float_to_bf16_bits(acc[n][3] * inv) << 16));
      *reinterpret_cast<uint2 *>(orow + 16 * n + 4 * g) = v;
    }
  }
}

template <int D, int BN>
int launch(const PrefillParams &p, int64_t max_query_len, hipStream_t stream) {
  using C = PrefillCfg<D, BN>;
  const size_t lds = 2 * C::kStage;
  dim3 grid(p.hq, p.num_seqs, static_cast<unsigned>(ceil_div(max_query_len, kBM)));
  prefill_mfma<D, BN><<<grid, 256, lds, stream>>>(p);
  return check_launch("mlr_paged_prefill(mfma)");
}

}  // namespace

bool prefill_mfma_eligible(int dtype, int64_t head_dim, int64_t block_size) {
  (void)block_size;
  return dtype == MLR_DTYPE_BF16 && (head_dim == 64 || head_dim == 128);
}

int launch_prefill_mfma(const PrefillParams &p, int64_t max_query_len,
                        hipStream_t stream) {
  if (max_query_len > int64_t(65535) * kBM)
    return set_error(MLR_ERR_UNSUPPORTED, "mlr_paged_prefill: chunk too long");
  // The reference's tile_size only orders the FP32 accumulation; the kernel's
  // key tile is fixed per head_dim by its LDS budget.
  if (p.d == 64) return launch<64, 64>(p, max_query_len, stream);
  return launch<128, 32>(p, max_query_len, stream);
}

}  // namespace mlr
