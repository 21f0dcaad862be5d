// FP32 paged chunk prefill on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// One workgroup = 64 queries of one query head as four waves of 16 queries.
// The waves share no LDS and no barrier: each runs its own key range, the
// keys up to its last query's position. Per wave and block of 16 keys:
//   S^T[16 keys x 16 queries] = K[16 keys x D] . Q^T[D x 16 queries] in D/4
//     MFMAs. Step (j, e) takes dims 16j + 4g + e from lane group g = l/16:
//     lane l holds key l%16's row chunk j (one 16-byte load per j) and query
//     l%16's matching Q chunk, loaded once and pre-multiplied by
//     scale*log2(e), so the scores come out in base-2 units.
//   Lane l then holds S^T[keys 4g..4g+3][query l%16]. A query's 16 scores
//     sit in the four lanes l%16 + 16g', so its row max is two lane swaps;
//     its row sum is kept per lane and added across those lanes once, at the
//     end.
//   O^T += V^T . P^T in D/4 MFMAs: step i takes keys 4g + i, whose
//     probabilities are the lane's four values; dim block c takes dims
//     VC*m + c of row m (VC = D/16), so lane l loads VC consecutive floats of
//     each of its four V rows with vector loads, and accumulator c holds
//     O^T[dim VC*(4g + i) + c][query l%16]: VC consecutive dims per lane and
//     i, one vector store per i at the end.
// Each wave issues the next block's K and V loads before the current
// block's MFMAs, so one block's loads are in flight while the matrix cores
// work (8 x 512-token chunks in FP32: 665 us per call against 717 us without).
// Keys past the last one the wave needs, and keys of an out-of-range block
// id, load as zeros and are masked; so are keys past a query's position
// (causal by absolute position). Rows the wave does not need are never
// read, so unwritten rows of the pool (whatever they hold) never reach a
// product.
//
// Numerics: FP32 products and sums throughout (the reference's FP32 path,
// kernels/reference/paged_attention.py:346-434), online softmax in base 2;
// the scale is folded into q (one FP32 rounding). The reference's tile_size
// only orders its FP32 accumulation, as here the 16-key blocks do.
//
// Work: items are (sequence, 64-query tile) pairs, each run once per query
// head. Workgroup b goes to XCD b mod 8 (the dispatcher deals workgroups to
// the XCDs in turn), and the query heads of one item get workgroups of one
// residue mod 8, so the K/V rows a GQA group re-reads come from one L2.
// Items start last query tile first: later tiles see more keys.
#include "paged_prefill.h"

namespace mlr {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2eF32 = 1.4426950408889634f;
constexpr int kQW = 16;      // queries per wave
constexpr int kBMF = 64;     // queries per workgroup (four waves)

__device__ __forceinline__ float swap_max(float x, int lanes) {
  return fmaxf(x, __shfl_xor(x, lanes, 64));
}

template <int D>
__global__ __launch_bounds__(256) void prefill_f32_mfma(PrefillParams p) {
  constexpr int QK = D / 16;  // 16-dim chunks of a row (S^T k-steps: 4 each)
  constexpr int VC = D / 16;  // dims per lane and V row (O^T dim blocks)
  const int nqt = p.n_qtiles;
  const int nitems = p.num_seqs * nqt;
  const int b = static_cast<int>(blockIdx.x);
  const int t = b >> 3;
  const int h = t % p.hq;
  const int rank = (t / p.hq) * 8 + (b & 7);
  if (rank >= nitems) return;  // uniform: the grid is padded to whole groups of 8
  const int seq = rank % p.num_seqs;
  const int qt = nqt - 1 - rank / p.num_seqs;
  SeqRange rg = seq_range(p, seq);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wq = qt * kBMF + kQW * wv;  // the wave's first query (chunk index)
  const int qlen = static_cast<int>(rg.qlen);
  if (wq >= qlen) return;  // uniform per wave; no barrier follows
  const int prefix = static_cast<int>(rg.prefix);
  const int kvh = h / p.group;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, m = lane & 15;

  // Q^T fragments of query wq + m (zeros past the chunk).
  const int qi = wq + m;
  const bool q_ok = qi < qlen;
  const float c2 = static_cast<float>(p.scale) * kLog2eF32;
  f32x4_t qf[QK];
  {
    const float *qrow = static_cast<const float *>(p.q) +
                        (rg.q0 + (q_ok ? qi : wq)) * p.q_st + static_cast<int64_t>(h) * p.q_sh;
#pragma unroll
    for (int j = 0; j < QK; ++j) {
      const f32x4_t v = *reinterpret_cast<const f32x4_t *>(qrow + 16 * j + 4 * g);
      qf[j] = q_ok ? v * c2 : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Keys this wave needs: up to its last query's position.
  const int kv_end = prefix + min(qlen, wq + kQW);
  const int nkb = (kv_end + 15) >> 4;
  // Lane l's query position for the causal mask (the S^T column).
  const int qpos = prefix + wq + m;
  const int first_masked = prefix + wq;  // blocks ending at or before it see no mask
  const int bs_log2 = p.bs_log2;
  const int bs_mask = (1 << bs_log2) - 1;
  const int64_t row_elems = static_cast<int64_t>(p.hkv) * D;
  const float *kc = static_cast<const float *>(p.kc) + static_cast<int64_t>(kvh) * D;
  const float *vc = static_cast<const float *>(p.vc) + static_cast<int64_t>(kvh) * D;
  const int64_t *bt_row = p.bt + static_cast<int64_t>(seq) * p.bt_stride;

  f32x4_t acc[VC];
#pragma unroll
  for (int c = 0; c < VC; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_lane = 0.f;

  // Block kb's K fragments and V rows into kf / vf; returns whether its
  // block id is in range.
  auto load_block = [&](int kb, f32x4_t (&kf)[QK], f32x4_t (&vf)[4][VC / 4]) -> bool {
    const int key0 = kb * 16;
    // 16 keys never straddle a cache block (block_size a power of two >= 16).
    const int64_t raw = bt_row[key0 >> bs_log2];
    const int64_t blk = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(raw))) |
                        (static_cast<int64_t>(__builtin_amdgcn_readfirstlane(
                             static_cast<uint32_t>(static_cast<uint64_t>(raw) >> 32))) << 32);
    const bool blk_ok = blk >= 0 && blk < p.num_blocks;
    const int64_t slot0 = (blk_ok ? blk : 0) * p.block_size + (key0 & bs_mask);
    // K rows: lane l reads key key0 + m (zeros past kv_end or for a bad block).
    {
      const bool ok = blk_ok && key0 + m < kv_end;
      const float *krow = kc + (slot0 + (ok ? m : 0)) * row_elems;
#pragma unroll
      for (int j = 0; j < QK; ++j)
        kf[j] = ok ? *reinterpret_cast<const f32x4_t *>(krow + 16 * j + 4 * g)
                   : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // V rows of keys key0 + 4g + i: VC consecutive dims each.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = 4 * g + i;
      const bool ok = blk_ok && key0 + k < kv_end;
      const float *vrow = vc + (slot0 + (ok ? k : 0)) * row_elems + VC * m;
#pragma unroll
      for (int u = 0; u < VC / 4; ++u)
        vf[i][u] = ok ? *reinterpret_cast<const f32x4_t *>(vrow + 4 * u)
                      : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    return blk_ok;
  };
  f32x4_t kf[QK], vf[4][VC / 4];
  bool blk_ok = load_block(0, kf, vf);
  for (int kb = 0; kb < nkb; ++kb) {
    const int key0 = kb * 16;
    f32x4_t nkf[QK], nvf[4][VC / 4];
    bool nok = false;
    if (kb + 1 < nkb) nok = load_block(kb + 1, nkf, nvf);
    // S^T of the block.
    f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QK; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j][e], qf[j][e], s, 0, 0, 0);
    // Mask: keys past the query's position, and all keys of a bad block.
    if (!blk_ok || key0 + 15 > first_masked) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!blk_ok || key0 + 4 * g + i > qpos) s[i] = -INFINITY;
    }
    // Online softmax (base 2). The reference point stays 0 until the query
    // has seen a key, so masked scores give exactly zero probabilities.
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mx = swap_max(mx, 16);
    mx = swap_max(mx, 32);
    const float m_new = fmaxf(m_run, mx);
    const float ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - ref);  // 0 while m_run is -inf
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(s[i] - ref);
    l_lane = l_lane * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    m_run = m_new;
#pragma unroll
    for (int c = 0; c < VC; ++c) acc[c] *= alpha;
    // O^T += V^T P^T.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < VC; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[i][c >> 2][c & 3], pr[i], acc[c], 0, 0, 0);
    if (kb + 1 < nkb) {
#pragma unroll
      for (int j = 0; j < QK; ++j) kf[j] = nkf[j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int u = 0; u < VC / 4; ++u) vf[i][u] = nvf[i][u];
      blk_ok = nok;
    }
  }

  // Row sum across the query's four lanes, then the output rows.
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot = l_tot + __shfl_xor(l_tot, 32, 64);
  if (q_ok) {
    const float inv = 1.f / l_tot;
    float *orow = static_cast<float *>(p.out) + (rg.q0 + qi) * p.o_st +
                  static_cast<int64_t>(h) * p.o_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // acc[c][i] = O[query qi][dim VC*(4g + i) + c].
#pragma unroll
      for (int u = 0; u < VC / 4; ++u) {
        f32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[4 * u + e][i] * inv;
        *reinterpret_cast<f32x4_t *>(orow + VC * (4 * g + i) + 4 * u) = o;
      }
    }
  }
}

template <int D>
int launch_f32(const PrefillParams &p, int64_t max_query_len, hipStream_t stream) {
  PrefillParams q = p;
  q.n_qtiles = static_cast<int>(ceil_div(max_query_len, kBMF));
  const int64_t items = static_cast<int64_t>(q.num_seqs) * q.n_qtiles;
  const int64_t blocks = ceil_div(items, 8) * 8 * q.hq;
  if (blocks > INT32_MAX)
    return set_error(MLR_ERR_UNSUPPORTED, "mlr_paged_prefill: too many work items");
  prefill_f32_mfma<D><<<dim3(static_cast<unsigned>(blocks)), 256, 0, stream>>>(q);
  return check_launch("mlr_paged_prefill(fp32 mfma)");
}

}  // namespace

bool prefill_f32_eligible(const PrefillParams &p, int dtype) {
  const bool aligned = (reinterpret_cast<uintptr_t>(p.q) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.kc) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.vc) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0 &&
                       p.q_st % 4 == 0 && p.q_sh % 4 == 0 && p.o_st % 4 == 0 &&
                       p.o_sh % 4 == 0;
  // Positions are 32-bit inside the kernel.
  constexpr int64_t k2g = int64_t(1) << 31;
  return dtype == MLR_DTYPE_F32 && (p.d == 64 || p.d == 128) && aligned && p.bs_log2 >= 4 &&
         p.max_blocks * p.block_size < k2g && p.scale > 0.0 && p.scale < 1e30;
}

int launch_prefill_f32(const PrefillParams &p, int64_t max_query_len, hipStream_t stream) {
  if (p.d == 64) return launch_f32<64>(p, max_query_len, stream);
  return launch_f32<128>(p, max_query_len, stream);
}

}  // namespace mlr
