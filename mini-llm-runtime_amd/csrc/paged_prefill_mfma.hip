// bf16 and fp16 paged chunk prefill on gfx950 matrix cores
// (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x16_f16).
//
// One workgroup = 128 queries of one query head and eight waves: two splits
// of the key range (waves 0-3 and 4-7, merged through LDS at the end), each
// with four waves of 32 queries. Waves w and w + 4 share a SIMD, and the two
// splits run a ping-pong schedule on it (see the main loop): while one
// split's waves work the matrix cores, the other's run the softmax on the
// VALU.
// Keys stream through LDS in tiles of BN = 64 positions (both head sizes;
// the launcher fixes it), two K and two V stages per split, copied from HBM
// straight into LDS with buffer_load_dwordx4 ... lds (no register staging),
// two phases ahead of their use. Each wave copies 16 consecutive key rows of
// K and of V per tile. With block_size a power of two >= 16 those rows sit in
// one cache block, so their source address is scalar (a buffer resource at
// the slot base) plus a lane-constant offset. Rows past the last key the
// workgroup needs, and out-of-range blocks, fall outside the buffer resource
// and read as zeros; keys of an out-of-range block are also masked.
//
// LDS rows are unpadded (2*D bytes). The 16-byte chunk c of tile row r is
// stored at chunk c ^ swz(r), which keeps both the K reads of S^T and the
// transposing V reads of P@V free of bank conflicts.
//
// Per tile and wave (32 queries x BN keys):
//   S^T[32 keys x 32 queries] = K[32 keys x D] . Q^T[D x 32 queries] for each
//       32-key block of the tile, D/16 MFMAs each; A = K rows (ds_read_b128),
//       B = Q^T fragments held in registers throughout.
//   Lane l owns query l%32 and keys 8(i/4) + 4(l/32) + i%4 (i < 16) of each
//   32-key block; lanes l and l^32 share a query, so the row max is one
//   permlane32 swap. Base-2 online softmax in FP32 with no per-score scaling:
//   Q is pre-multiplied by scale*log2(e) and the S^T accumulator is seeded
//   with -m, so the matrix cores return scores in base-2 units relative to the
//   running reference point m and P = exp2(S^T) directly. The reference point
//   moves only when a tile raises the row max by more than kLazy, so
//   probabilities stay below 2^kLazy and numerator and denominator share it.
//   O^T[32 dims x 32 queries] += V^T[32 dims x 16 keys] . P^T[16 keys x 32 q]
//       B = P^T packed to the 16-bit type straight from the S^T registers (k slot
//       8(l/32)+e <-> key 16kb + 8(e/4) + 4(l/32) + e%4), A = V^T from two
//       ds_read_b64_tr_b16 per MFMA.
//   The row sums add the FP32 probabilities, as the reference does.
// Causal masking (key position <= query position, both absolute) runs only
// on tiles that reach the wave's first query position; a wave skips the
// tiles past its last query position.
//
// Numerics follow paged_attention_prefill_chunk_tiled
// (kernels/reference/paged_attention.py:346-434): FP32 softmax statistics,
// FP32 accumulation of P@V and one rounding of the output. Three roundings
// differ from the reference and stay far inside the 2e-2 tolerance of its
// bf16 tests: q*scale*log2(e) is rounded to bf16 (relative 2^-9 per element,
// the size of the reference's own bf16 rounding of q.k at :411-413, which is
// not done here), and P is rounded to bf16 as the MFMA operand. fp16 runs the
// same kernel with fp16 operands (the same two roundings, to fp16: relative
// 2^-12), round-to-nearest-even throughout.
#include "paged_prefill.h"

#include <atomic>

namespace mlr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;
constexpr float kFloor = -1.0e30f;  // initial reference point (base 2)
constexpr int kBM = 128;      // queries per workgroup (4 waves x 32)
constexpr int kSpanRows = 16; // key rows per copy span
constexpr int kRankMax = 512; // most work items ranked in the prologue

template <int D, int BN>
struct Cfg {
  static constexpr int kRowB = 2 * D;                        // LDS bytes per key row
  static constexpr int kTileB = BN * kRowB;                  // one K (or V) tile
  static constexpr int kChunks = D / 8;                      // 16-byte chunks per row
  static constexpr int kCopies = kSpanRows * kRowB / 1024;   // 1 KB copies per span
  static constexpr int kBlocks = BN / 32;                    // 32-key blocks per tile
  static_assert(BN / 4 == kSpanRows, "each wave copies one 16-row span per tile");
};

// Chunk swizzle (depends on the low four row bits only, so it repeats every
// 16 rows): physical chunk = logical chunk ^ swz(row).
template <int D>
__device__ __forceinline__ int swz(int r) {
  if (D == 64) return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
  return ((r & 1) << 1) | (((r >> 1) & 3) << 2) | ((r >> 3) & 1);
}

// Two floats to packed bf16 (round to nearest even): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// The 16-bit operand type of the MFMAs: bf16 or fp16 fragments, the 32x32x16
// MFMA of that type, two floats packed to it (round to nearest even), and the
// two halves of a 32-bit word of it widened to FP32.
template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  using v8 = bf16x8_t;
  __device__ static f32x16_t mfma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) { return bf16_pack2(lo, hi); }
  __device__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static uint32_t bits(float x) { return float_to_bf16_bits(x); }
};
template <> struct Mma<f16_t> {
  using v8 = f16x8_t;
  __device__ static f32x16_t mfma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) {
    const f16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t);
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static float lo(uint32_t w) { return f16_bits_to_float(static_cast<uint16_t>(w)); }
  __device__ static float hi(uint32_t w) { return f16_bits_to_float(static_cast<uint16_t>(w >> 16)); }
  __device__ static uint32_t bits(float x) { return float_to_f16_bits(x); }
};

// max(a, b, c) as one v_maximum3_f32 (NaN-propagating, no canonicalisation).
__device__ __forceinline__ float max3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Lanes l and l ^ 32 exchange x (one v_permlane32_swap): the two halves of
// the result hold x of the lower and of the upper half-wave.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Rank (0 = most keys) of the work taken by workgroup b of nwg; see the
// kernel's prologue.
__device__ __forceinline__ int workgroup_rank(int b, int nwg, int ncu, int pair_cu) {
  if (!pair_cu || nwg <= ncu || b >= 2 * ncu) return b;
  const int paired = min(nwg, 2 * ncu) - ncu;  // CUs that host two workgroups
  const int single = ncu - paired;             // CUs that host one
  if (b >= ncu) return single + 2 * paired - 1 - (b - ncu);  // light half, reversed
  return b < paired ? single + b : b - paired;
}

template <typename T, int D, int BN, int KS>
__global__ __launch_bounds__(256 * KS) __attribute__((amdgpu_waves_per_eu(D == 64 ? 4 : 2)))
void prefill_mfma(PrefillParams p) {
  using C = Cfg<D, BN>;
  using M = Mma<T>;
  using v8 = typename M::v8;
  constexpr int QS = D / 16;         // 16-dim k-steps of S^T
  constexpr int NB = D / 32;         // 32-dim blocks of O^T
  constexpr int KB = C::kBlocks;     // 32-key blocks per tile
  static_assert(KS == 2, "the ping-pong schedule pairs two splits");
  // Per split: two stages of K and of V, each a separate LDS object, so that
  // reads of one stage need not wait for copies into another. Byte w of
  // badkS[k] is set when wave w's 16 rows of split k's K tile in stage S lie
  // in an out-of-range block (bytes 4l + w hold the same flag, one per lane).
  __shared__ __align__(1024) unsigned char ks0[KS][C::kTileB];
  __shared__ __align__(1024) unsigned char ks1[KS][C::kTileB];
  __shared__ __align__(1024) unsigned char vs0[KS][C::kTileB];
  __shared__ __align__(1024) unsigned char vs1[KS][C::kTileB];
  __shared__ __align__(16) unsigned char badk0[KS][256];
  __shared__ __align__(16) unsigned char badk1[KS][256];

  // Work items are (sequence, query tile) pairs, each run once per query head;
  // a workgroup's rank wr = rank * hq + head, where rank orders the items by
  // the keys they need, longest first, ties by item index. With more than
  // kRankMax items the ranking is skipped and items go sequence by sequence,
  // last query tile first.
  // Workgroups start in order of blockIdx.x and the hardware hands a freed CU
  // the next one. When two fit per CU, the first 2*ncu start at once, and
  // workgroups b and b + ncu share a CU (the dispatcher deals each XCD's CUs
  // in the same order on every pass). Those pairs get a heavy and a light
  // rank, and CUs left with one workgroup get the heaviest; later workgroups
  // follow in rank order (list scheduling).
  const int nqt = p.n_qtiles;
  const int nitems = p.num_seqs * nqt;
  const int wr = workgroup_rank(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x),
                                p.ncu, p.pair_cu);
  // Heads of one item on one XCD. The dispatcher deals workgroups to the 8
  // XCDs in turn (blockIdx mod 8), and within each segment of
  // workgroup_rank, wr mod 8 fixes blockIdx mod 8. For the ranks in whole
  // groups of 8, wr = 8 (g hq + h) + x is rank 8g + x, head h: all heads of
  // a rank share an XCD and its L2, so the K/V tiles of a GQA group come from
  // HBM once rather than once per query head. Rank order (heaviest first)
  // holds to within a group of 8. Ranks past the last whole group keep
  // rank = wr / hq.
  const int nranks = static_cast<int>(gridDim.x) / p.hq;
  const int grouped = (nranks / 8) * 8 * p.hq;
  int rank, h;
  if (wr < grouped) {
    const int t = wr >> 3;
    rank = (t / p.hq) * 8 + (wr & 7);
    h = t % p.hq;
  } else {
    rank = wr / p.hq;
    h = wr % p.hq;
  }
  int item;
  if (nitems <= kRankMax) {
    __shared__ int item_len[kRankMax];
    __shared__ int ranked_item;
    auto keys_of = [&](int i) __attribute__((always_inline)) -> int {
      const SeqRange r = seq_range(p, i / nqt);
      const int64_t lo = static_cast<int64_t>(i % nqt) * kBM;
      return lo < r.qlen ? static_cast<int>(r.prefix + min<int64_t>(r.qlen, lo + kBM)) : 0;
    };
    for (int i = threadIdx.x; i < nitems; i += blockDim.x) item_len[i] = keys_of(i);
    __syncthreads();
    for (int i = threadIdx.x; i < nitems; i += blockDim.x) {
      const int li = item_len[i];
      int r = 0;
      for (int j = 0; j < nitems; ++j) {
        const int lj = item_len[j];
        r += (lj > li || (lj == li && j < i)) ? 1 : 0;
      }
      if (r == rank) ranked_item = i;
    }
    __syncthreads();
    item = __builtin_amdgcn_readfirstlane(ranked_item);
  } else {
    item = (rank / nqt) * nqt + (nqt - 1 - rank % nqt);
  }
  const int seq = item / nqt, qt = item % nqt;
  SeqRange rg = seq_range(p, seq);
  // Workgroup-uniform: kept in scalar registers.
  rg.q0 = uniform64(rg.q0);
  rg.qlen = uniform64(rg.qlen);
  rg.prefix = uniform64(rg.prefix);
  const int q0 = qt * kBM;
  if (q0 >= rg.qlen) return;  // uniform
  const int kvh = h / p.group;
  const int qlen = static_cast<int>(rg.qlen), prefix = static_cast<int>(rg.prefix);

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = wv & 3, split = wv >> 2;  // query group, key-range split
  const int m32 = lane & 31, hh = lane >> 5;

  // Keys the workgroup needs: up to its last query position; split k takes
  // tiles [t_lo, t_hi).
  const int kv_end = prefix + min(qlen, q0 + kBM);
  const int ntiles = (kv_end + BN - 1) / BN;
  const int chunk = (ntiles + KS - 1) / KS;
  const int t_lo = split * chunk, t_hi = min(ntiles, t_lo + chunk);
  // This wave's queries [wq, wq_end); tiles it reads; tiles it sees whole.
  const int wq = q0 + 32 * w;
  const int wq_end = min(qlen, wq + 32);
  const int wave_tiles = wq < wq_end ? min(t_hi, (prefix + wq_end - 1) / BN + 1) : 0;
  const int wave_nfull = (prefix + wq + 1) / BN;

  // Q^T fragments: lane l holds Q[query wq + l%32][16s + 8(l/32) .. +8).
  const int qi = wq + m32;
  const bool q_ok = qi < qlen;
  const int qpos = prefix + qi;
  const uint16_t *qrow = static_cast<const uint16_t *>(p.q) +
                         (rg.q0 + (q_ok ? qi : 0)) * p.q_st + static_cast<int64_t>(h) * p.q_sh;
  // Issued here and turned into fragments after the prologue's copies have
  // been issued and waited for: the row address is clamped, so the loads
  // are unconditional (a load under a branch made the compiler wait for it
  // before issuing the block-id loads and the first copies).
  uint4 qraw[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) qraw[s] = *reinterpret_cast<const uint4 *>(qrow + 16 * s + 8 * hh);
  v8 qf[QS];

  // Copy role: copy i of a span moves chunk positions [64i, 64i + 64) of its 16
  // rows; lane l fills position 64i + l (row rr, physical chunk pc) with
  // logical chunk pc ^ swz(rr) of source row rr.
  const uint32_t row_bytes = static_cast<uint32_t>(p.hkv) * D * 2;  // slot stride
  uint32_t src_off[C::kCopies];
#pragma unroll
  for (int i = 0; i < C::kCopies; ++i) {
    const int pos = 64 * i + lane;
    const int rr = pos / C::kChunks, pc = pos % C::kChunks;
    src_off[i] = rr * row_bytes + ((pc ^ swz<D>(rr)) << 4);
  }
  // The block table is read-only for the whole launch: read it through the
  // constant address space, so the wave-uniform lookups are scalar loads.
  typedef __attribute__((address_space(4))) const int64_t const_i64;
  const const_i64 *bt_row = (const const_i64 *)p.bt + static_cast<int64_t>(seq) * p.bt_stride;
  const int bs_log2 = p.bs_log2;
  const int bs_mask = (1 << bs_log2) - 1;
  // The four waves' out-of-range flags of a K stage (bytes 0..3).
  auto read_bad = [&](const unsigned char *bad) __attribute__((always_inline)) -> uint32_t {
    return __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t *>(bad));
  };

  // Lane-constant LDS offsets. K read of step st: row m32 (+32 per key block),
  // logical chunk 2st + hh. V^T read (two per MFMA, rows +8 apart): in each
  // 16-lane group G, lane li points at row 4(G/2) + li/4 (+ 16kb) and byte
  // 64n + 32(G%2) + 8(li%4). Only the step-0 and (half 0, n 0) offsets are
  // kept: the swizzle is an XOR of the chunk index, whose parts 2st, 4n lie
  // in bits of their own, and 8 rows further it flips chunk bit 0, so
  //   koff(st) = koff0 ^ (st << 5),
  //   voff(half, n) = (voff0 ^ (half << 4) ^ (n << 6)) + half * 8 rows.
  const int koff0 = m32 * C::kRowB + ((hh ^ swz<D>(m32)) << 4);
  const int G = lane >> 4, li = lane & 15;
  const int vrow0 = 4 * (G >> 1) + (li >> 2);
  const int vbyte0 = 32 * (G & 1) + 8 * (li & 3);
  const int voff0 =
      vrow0 * C::kRowB + ((((vbyte0 >> 4) ^ swz<D>(vrow0)) << 4) | (vbyte0 & 15));
  // The derived offsets are recomputed where they are used (a few XORs)
  // rather than held in registers across the loop.
  auto koffs = [&](int (&ko)[QS]) __attribute__((always_inline)) {
    int k0 = koff0;
    asm volatile("" : "+v"(k0));
#pragma unroll
    for (int st = 0; st < QS; ++st) ko[st] = k0 ^ (st << 5);
  };
  auto voffs = [&](int (&vo)[2][NB]) __attribute__((always_inline)) {
    int v0 = voff0;
    asm volatile("" : "+v"(v0));
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int n = 0; n < NB; ++n) vo[half][n] = (v0 ^ (half << 4) ^ (n << 6)) + half * 8 * C::kRowB;
  };

  // Reference point m of the running softmax (base 2). It stays at the
  // finite floor kFloor (never -inf: a query can see no key at all in one
  // split's tiles, and exp2(-inf - (-inf)) would be NaN) until the row sees a
  // key. negm seeds S^T: -m, or 0 while m is unset. A tile needs the rescale
  // when its relative max exceeds thr: kLazy once m is set, any visible key
  // before. Masked scores stay -inf, so their probabilities are exactly 0.
  float m_run = kFloor, l_run = 0.f, thr = -__FLT_MAX__;
  f32x16_t negm;
#pragma unroll
  for (int i = 0; i < 16; ++i) negm[i] = 0.f;
  f32x16_t acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[n][i] = 0.f;

  // S^T of one tile from its K stage.
  auto scores = [&](const unsigned char *kst, f32x16_t (&s)[KB]) __attribute__((always_inline)) {
    int koff[QS];
    koffs(koff);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        const v8 a = *reinterpret_cast<const v8 *>(kst + 32 * j * C::kRowB + koff[st]);
        s[j] = M::mfma(a, qf[st], st == 0 ? negm : s[j]);
      }
    }
    // At most two K reads ahead of the MFMAs (four VGPRs each): hoisting all
    // of them would hold 8 * 4 more registers at the peak of the phase.
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int g = 0; g < KB * QS - 2; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  };
  // Causal mask (key position <= query position) and out-of-range spans.
  // Element i of block j holds key 32j + 8(i/4) + 4hh + i%4, compared here
  // as the constant 32j + 8(i/4) + i%4 against lim - 4hh; its 16-row span is
  // 2j + i/8 in every lane.
  auto mask = [&](int t, uint32_t badw, f32x16_t (&s)[KB]) __attribute__((always_inline)) {
    const int lim = qpos - t * BN - 4 * hh;  // last visible key of the lane's query
#pragma unroll
    for (int j = 0; j < KB; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool bad = (badw >> (8 * (2 * j + (i >> 3)))) & 1;
        if (bad || 32 * j + 8 * (i >> 2) + (i & 3) > lim) s[j][i] = -INFINITY;
      }
  };
  // Row max of a tile relative to m (base 2): chains of eight, then the lane pair.
  auto tile_max = [&](const f32x16_t (&s)[KB]) __attribute__((always_inline)) -> float {
    float mc[2 * KB];
#pragma unroll
    for (int c = 0; c < 2 * KB; ++c) {
      const int j = c >> 1, b = 8 * (c & 1);
      mc[c] = max3(s[j][b], s[j][b + 1], s[j][b + 2]);
      mc[c] = max3(mc[c], s[j][b + 3], s[j][b + 4]);
      mc[c] = max3(mc[c], s[j][b + 5], s[j][b + 6]);
      mc[c] = __builtin_elementwise_maximum(mc[c], s[j][b + 7]);
    }
#pragma unroll
    for (int width = KB; width >= 1; width >>= 1)
#pragma unroll
      for (int c = 0; c < width; ++c) mc[c] = __builtin_elementwise_maximum(mc[c], mc[c + width]);
    return pair_max(mc[0]);
  };
  // Moves the reference point to the tile max where that passed thr, rescales
  // the accumulators and shifts the tile's scores to the new point.
  auto rescale = [&](float m_rel, f32x16_t (&s)[KB]) __attribute__((always_inline)) {
    if (__any(m_rel > thr)) {
      const bool unset = m_run == kFloor;
      const bool move = m_rel > thr;
      const float m_new = move ? (unset ? 0.f : m_run) + m_rel : m_run;
      const float shift = move ? m_rel : 0.f;
      const float alpha = unset ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);  // 1 where kept
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < NB; ++n) acc[n] *= alpha;
      m_run = m_new;
      thr = m_new == kFloor ? -__FLT_MAX__ : kLazy;
      const float seed = m_new == kFloor ? 0.f : -m_new;
#pragma unroll
      for (int i = 0; i < 16; ++i) negm[i] = seed;
#pragma unroll
      for (int j = 0; j < KB; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[j][i] -= shift;
    }
  };
  constexpr int kBatchCopies = 2 * C::kCopies;
  // s_waitcnt vmcnt(kBatchCopies) lgkmcnt(0), and lgkmcnt(0) alone (gfx9
  // encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
  constexpr int kWaitBatch = (kBatchCopies & 15) | ((kBatchCopies >> 4) << 14) | 0x70;
  constexpr int kWaitLds = 0xC07F;
  const int nw = max(0, min(t_hi, wave_tiles) - t_lo);  // tiles this wave computes
  // Launches with num_blocks < 2^31 and blocks < 2^31 bytes only.
  const uint32_t nb32 = static_cast<uint32_t>(p.num_blocks);
  const uint32_t block_bytes = row_bytes << bs_log2;
  const uint32_t kv_bytes = static_cast<uint32_t>(kvh) * (2 * D);

  // The wave's span of tile t: the byte offset and record count of a buffer
  // resource covering the rows the workgroup needs (rows past them, and a
  // block id out of range, read as zeros) and whether its block id is out
  // of range. Scalar code, run in the M phase ahead of the V phase that
  // issues the copies.
  struct Span {
    uint32_t off_lo, off_hi, nrec, bad;
  };
  // In-block byte offset of the wave's rows: (64t + 16w) & bs_mask is
  // ((64t) & bs_mask) + ((16w) & bs_mask), as 64t has no bits below 64 and
  // 16w < 64; the second part (and the KV head's offset) is per wave.
  const uint32_t inblk_w = static_cast<uint32_t>((kSpanRows * w) & bs_mask) * row_bytes + kv_bytes;
  auto span_of = [&](int t, int64_t id) __attribute__((always_inline)) -> Span {
    const int pos0 = t * BN + (BN / 4) * w;
    const bool live = pos0 < kv_end && t < t_hi;
    const uint32_t lo = static_cast<uint32_t>(id);
    const uint32_t hi = static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32);
    const bool ok = live && hi == 0u && lo < nb32;
    const uint32_t nrows = static_cast<uint32_t>(min(kv_end - pos0, kSpanRows));
    Span sp;
    sp.nrec = ok ? (nrows - 1) * row_bytes + 2 * D : 0u;
    const uint64_t byte0 = static_cast<uint64_t>(ok ? lo : 0u) * block_bytes +
                           (static_cast<uint32_t>((t * BN) & bs_mask) * row_bytes + inblk_w);
    sp.off_lo = static_cast<uint32_t>(byte0);
    sp.off_hi = static_cast<uint32_t>(byte0 >> 32);
    sp.bad = (live && !ok) ? 1u : 0u;
    // Keeps the arithmetic here rather than sunk into the V phase.
    asm volatile("" : "+s"(sp.off_lo), "+s"(sp.off_hi), "+s"(sp.nrec));
    return sp;
  };
  auto id_of = [&](int t) __attribute__((always_inline)) -> int64_t {
    return bt_row[min(t * BN + (BN / 4) * w, kv_end - 1) >> bs_log2];
  };
  // Copies the wave's 16 rows; with `bad`, records the span's flag there
  // (lane l writes byte 4l + w, so bytes 0..3 hold the four waves' flags).
  auto issue_span = [&](const Span &sp, const void *cache, unsigned char *dst,
                        unsigned char *bad) __attribute__((always_inline)) {
    const uint64_t byte0 = (static_cast<uint64_t>(sp.off_hi) << 32) | sp.off_lo;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char *>(static_cast<const unsigned char *>(cache) + byte0), 0,
        sp.nrec, 0x00020000);
    unsigned char *sdst = dst + (BN / 4) * w * C::kRowB;
#pragma unroll
    for (int i = 0; i < C::kCopies; ++i) {
      // A local copy: an element of the captured array as the builtin's
      // argument makes the host pass drop the kernel's launch stub.
      const uint32_t off = src_off[i];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)(sdst + 1024 * i), 16, off, 0,
                                               0, 0);
    }
    if (bad != nullptr) bad[4 * lane + w] = static_cast<unsigned char>(sp.bad);
  };
  // exp2 of a tile's S^T packed to the 16-bit type (the P@V operand), with the FP32
  // probabilities added to the row sum (four chains).
  auto probs = [&](const f32x16_t (&sc)[KB], uint32_t (&pk)[KB][8]) __attribute__((always_inline)) {
    float lsum[4];
#pragma unroll
    for (int j = 0; j < KB; ++j)
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const float p0 = __builtin_amdgcn_exp2f(sc[j][2 * x]);
        const float p1 = __builtin_amdgcn_exp2f(sc[j][2 * x + 1]);
        pk[j][x] = M::pack2(p0, p1);
        if (j == 0 && x < 2) {
          lsum[2 * x] = p0;
          lsum[2 * x + 1] = p1;
        } else {
          lsum[(2 * x) & 3] += p0;
          lsum[(2 * x + 1) & 3] += p1;
        }
      }
    l_run += (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
  };
  // O^T += V^T P^T from packed P.
  auto pv = [&](const uint32_t (&pk)[KB][8], const unsigned char *vst) __attribute__((always_inline)) {
    int voff[2][NB];
    voffs(voff);
#pragma unroll
    for (int j = 0; j < KB; ++j)
#pragma unroll
      for (int h16 = 0; h16 < 2; ++h16) {
        const int kb = 2 * j + h16;  // 16-key block
        const v8 pb = __builtin_bit_cast(
            v8, make_uint4(pk[j][4 * h16], pk[j][4 * h16 + 1], pk[j][4 * h16 + 2],
                           pk[j][4 * h16 + 3]));
#pragma unroll
        for (int n = 0; n < NB; ++n) {
          const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t *)(vst + 16 * kb * C::kRowB + voff[0][n]));
          const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t *)(vst + 16 * kb * C::kRowB + voff[1][n]));
          const uint2 ulo = __builtin_bit_cast(uint2, lo), uhi = __builtin_bit_cast(uint2, hi);
          const v8 a = __builtin_bit_cast(v8, make_uint4(ulo.x, ulo.y, uhi.x, uhi.y));
          acc[n] = M::mfma(a, pb, acc[n]);
        }
      }
    // Two MFMAs' V^T reads (two each) ahead of the MFMAs.
    constexpr int kMfma = 2 * KB * NB;
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int g = 0; g < kMfma - 2; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  };

  // Main loop: a ping-pong schedule of the two key-range splits (waves w and
  // w + 4 share a SIMD). Per split-local tile i a wave runs an MFMA phase M_i and a
  // softmax phase V_i, with a workgroup barrier after each phase:
  //   M_i: O^T += V^T P^T of tile i - 1, S^T of tile i, and the scalar
  //        set-up of the copies V_i will issue;
  //   V_i: issue those copies, then mask, row max, rescale, exp2 and 16-bit
  //        packing of tile i, with the FP32 row sums.
  // Split 1 passes one extra barrier first, so it runs a phase behind split
  // 0 and on every SIMD one wave's matrix-core work overlaps the other's
  // VALU work:
  //   phase      0   1   2   3   4  ...
  //   split 0    M0  V0  M1  V1  M2 ...
  //   split 1    -   M0  V0  M1  V1 ...
  // Copies run two phases ahead: V_i copies K(i+2) into K stage i%2 (free
  // since M_i) and V(i+1) into V stage (i+1)%2 (free since P@V(i-1) in M_i);
  // M_i needs K(i) and V(i-1), copied in V_{i-2}. Each V phase issues the
  // same number of copies (tiles past the split read zeros), so before the
  // barrier ahead of an M phase a wave waits for all but its newest batch.
  //
  // dk: the span of the newest K copy issued (tile i + 1 when M_i starts);
  // the V copy of the same tile, one phase later, reads the same rows of the
  // V cache. id_b: the block id of tile i + 2 when M_i starts.
  Span dk, dv;
  int64_t id_b;
  {
    const int64_t id0 = id_of(t_lo);
    const int64_t id1 = id_of(t_lo + 1);
    id_b = id_of(t_lo + 2);
    const Span s0 = span_of(t_lo, id0);
    issue_span(s0, p.kc, ks0[split], badk0[split]);
    issue_span(s0, p.vc, vs0[split], nullptr);
    dk = span_of(t_lo + 1, id1);
    issue_span(dk, p.kc, ks1[split], badk1[split]);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's prologue copies and flags, and q
  __builtin_amdgcn_s_barrier();
  // Q pre-multiplied by scale*log2(e) (the scores come out in base-2 units);
  // rows past the chunk are zero.
  const float c2 = static_cast<float>(p.scale) * kLog2e;
#pragma unroll
  for (int s = 0; s < QS; ++s) {
    const uint4 raw = q_ok ? qraw[s] : make_uint4(0, 0, 0, 0);
    const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t o4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o4[e] = M::pack2(M::lo(w4[e]) * c2, M::hi(w4[e]) * c2);
    qf[s] = __builtin_bit_cast(v8, make_uint4(o4[0], o4[1], o4[2], o4[3]));
  }
  if (split == 1) __builtin_amdgcn_s_barrier();
  // S^T (M to V) and packed P (V to M) are defined in every phase, idle
  // ones included, so neither is live across the phase that does not use it.
  f32x16_t s[KB];
  uint32_t pk[KB][8];
  uint32_t badw = 0;
  // M_i: K stage kst holds K(i) and its out-of-range flags kbad (read here:
  // V_i overwrites them), V stage vst holds V(i-1).
  auto m_phase = [&](int i, const unsigned char *kst, const unsigned char *kbad,
                     const unsigned char *vst) __attribute__((always_inline)) {
    const int64_t id_c = id_of(t_lo + i + 3);  // scalar load, used by M_{i+1}
    // Raised wave priority for the matrix work: the other split's softmax
    // phase on this SIMD takes the issue slots the MFMAs leave.
    __builtin_amdgcn_s_setprio(3);
    if (i >= 1 && i - 1 < nw) pv(pk, vst);
    // P dies with the last P@V MFMA before S^T is allocated.
    __builtin_amdgcn_sched_barrier(0);
    if (i < nw) {
      scores(kst, s);
      badw = read_bad(kbad);
    } else {
#pragma unroll
      for (int j = 0; j < KB; ++j) s[j] = f32x16_t{};
    }
    __builtin_amdgcn_s_setprio(0);
    dv = dk;  // V(i+1) reads the rows K(i+1) read
    dk = span_of(t_lo + i + 2, id_b);
    id_b = id_c;
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    __builtin_amdgcn_s_barrier();
  };
  // V_i: copies K(i+2) -> kdst (flags kbad) and V(i+1) -> vdst, then the
  // softmax of tile i.
  auto v_phase = [&](int i, unsigned char *kdst, unsigned char *kbad, unsigned char *vdst)
      __attribute__((always_inline)) {
    issue_span(dk, p.kc, kdst, kbad);
    issue_span(dv, p.vc, vdst, nullptr);
    if (i < nw) {
      const int t = t_lo + i;
      if (t >= wave_nfull || badw != 0) mask(t, badw, s);
      rescale(tile_max(s), s);
      probs(s, pk);
    } else {
#pragma unroll
      for (int j = 0; j < KB; ++j)
#pragma unroll
        for (int x = 0; x < 8; ++x) pk[j][x] = 0;
    }
    __builtin_amdgcn_s_waitcnt(kWaitBatch);
    __builtin_amdgcn_s_barrier();
  };
  // Unrolled by two so every stage is a fixed LDS object.
  for (int i = 0; i < chunk; i += 2) {
    m_phase(i, ks0[split], badk0[split], vs1[split]);
    v_phase(i, ks0[split], badk0[split], vs1[split]);
    m_phase(i + 1, ks1[split], badk1[split], vs0[split]);
    v_phase(i + 1, ks1[split], badk1[split], vs0[split]);
  }
  // P@V of the last tile when chunk is even (odd chunks ran it above).
  if ((chunk & 1) == 0) m_phase(chunk, ks0[split], badk0[split], vs1[split]);
  if (split == 0) __builtin_amdgcn_s_barrier();
  // Outstanding copies (all of absent tiles) would land on the merge
  // buffers laid over the stage objects.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();

  if constexpr (KS > 1) {
    // Splits 1.. hand (m, l, O^T) to split 0 through LDS, in a lane-major
    // layout: word a of lane l of query group w at ((k-1)*4 + w)*A + a)*64 + l,
    // laid over the stage objects in turn.
    constexpr int A = 16 * NB + 2;
    constexpr int kPer = static_cast<int>(sizeof(ks0) / sizeof(float));
    static_assert(4 * sizeof(ks0) >= (KS - 1) * 4 * A * 64 * sizeof(float), "merge buffer");
    auto xw = [&](int k, int a) __attribute__((always_inline)) -> float * {
      const int idx = (((k - 1) * 4 + w) * A + a) * 64 + lane;
      float *base = idx < kPer       ? reinterpret_cast<float *>(&ks0[0][0])
                    : idx < 2 * kPer ? reinterpret_cast<float *>(&ks1[0][0])
                    : idx < 3 * kPer ? reinterpret_cast<float *>(&vs0[0][0])
                                     : reinterpret_cast<float *>(&vs1[0][0]);
      return base + idx % kPer;
    };
    if (split > 0) {
#pragma unroll
      for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) *xw(split, 16 * n + i) = acc[n][i];
      *xw(split, 16 * NB) = m_run;
      *xw(split, 16 * NB + 1) = l_run;
    }
    __syncthreads();
    if (split > 0) return;
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const float m_o = *xw(k, 16 * NB), l_o = *xw(k, 16 * NB + 1);
      const float m_new = __builtin_elementwise_maximum(m_run, m_o);
      const float a_s = __builtin_amdgcn_exp2f(m_run - m_new);
      const float a_o = __builtin_amdgcn_exp2f(m_o - m_new);
      l_run = l_run * a_s + l_o * a_o;
#pragma unroll
      for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[n][i] = acc[n][i] * a_s + *xw(k, 16 * n + i) * a_o;
      m_run = m_new;
    }
  }

  const float l_tot = pair_sum(l_run);
  // The lane's query and half are recomputed from the lane id here rather
  // than kept in registers across the main loop (which spilled them).
  int lane_e = __lane_id();
  asm volatile("" : "+v"(lane_e));
  const int qi_e = wq + (lane_e & 31), hh_e = lane_e >> 5;
  if (qi_e < qlen) {
    const float inv = 1.f / l_tot;
    uint16_t *orow = static_cast<uint16_t *>(p.out) + (rg.q0 + qi_e) * p.o_st +
                     static_cast<int64_t>(h) * p.o_sh;
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        // acc[n][4g4 + e] = O[query][32n + 8g4 + 4hh + e].
        const f32x16_t &a = acc[n];
        const uint2 v = make_uint2(
            M::bits(a[4 * g4] * inv) | (M::bits(a[4 * g4 + 1] * inv) << 16),
            M::bits(a[4 * g4 + 2] * inv) | (M::bits(a[4 * g4 + 3] * inv) << 16));
        *reinterpret_cast<uint2 *>(orow + 32 * n + 8 * g4 + 4 * hh_e) = v;
      }
  }
}

template <typename T, int D, int BN, int KS>
int launch(const PrefillParams &p, int64_t max_query_len, hipStream_t stream) {
  PrefillParams q = p;
  q.n_qtiles = static_cast<int>(ceil_div(max_query_len, kBM));
  const int64_t blocks = static_cast<int64_t>(q.num_seqs) * q.n_qtiles * q.hq;
  if (blocks > INT32_MAX)
    return set_error(MLR_ERR_UNSUPPORTED, "mlr_paged_prefill: too many work items");
  // CU count and workgroups per CU of this kernel, queried once per device
  // (threads that race here store the same values).
  constexpr int kMaxDevices = 64;
  static std::atomic<int> ncu_of[kMaxDevices], per_cu_of[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(MLR_ERR_HIP, "mlr_paged_prefill: no current device");
  if (ncu_of[dev].load(std::memory_order_acquire) == 0) {
    int ncu = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(prefill_mfma<T, D, BN, KS>), 256 * KS, 0) !=
            hipSuccess)
      return set_error(MLR_ERR_HIP, "mlr_paged_prefill: device query failed");
    per_cu_of[dev].store(per_cu, std::memory_order_relaxed);
    ncu_of[dev].store(ncu, std::memory_order_release);
  }
  q.ncu = ncu_of[dev].load(std::memory_order_acquire);
  q.pair_cu = per_cu_of[dev].load(std::memory_order_relaxed) == 2 ? 1 : 0;
  prefill_mfma<T, D, BN, KS><<<dim3(static_cast<unsigned>(blocks)), 256 * KS, 0, stream>>>(q);
  return check_launch("mlr_paged_prefill(mfma)");
}

}  // namespace

bool prefill_mfma_eligible(const PrefillParams &p, int dtype) {
  const bool aligned = (reinterpret_cast<uintptr_t>(p.q) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.kc) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.vc) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 7u) == 0 &&
                       p.q_st % 8 == 0 && p.q_sh % 8 == 0 && p.o_st % 4 == 0 &&
                       p.o_sh % 4 == 0;
  // Positions, block ids and in-block byte offsets are 32-bit inside the
  // kernel; a 16-row span must fit a block.
  constexpr int64_t k2g = int64_t(1) << 31;
  return (dtype == MLR_DTYPE_BF16 || dtype == MLR_DTYPE_F16) && (p.d == 64 || p.d == 128) &&
         aligned &&
         p.bs_log2 >= 4 && p.max_blocks * p.block_size < k2g && p.num_blocks < k2g &&
         p.block_size * p.hkv * p.d * 2 < k2g && p.scale > 0.0 && p.scale < 1e30;
}

int launch_prefill_mfma(const PrefillParams &p, int dtype, int64_t max_query_len,
                        hipStream_t stream) {
  // The reference's tile_size only orders the FP32 accumulation; the kernel's
  // key tile is fixed per head_dim by its LDS budget.
  if (dtype == MLR_DTYPE_F16) {
    if (p.d == 64) return launch<f16_t, 64, 64, 2>(p, max_query_len, stream);
    return launch<f16_t, 128, 64, 2>(p, max_query_len, stream);
  }
  if (p.d == 64) return launch<bf16_t, 64, 64, 2>(p, max_query_len, stream);
  return launch<bf16_t, 128, 64, 2>(p, max_query_len, stream);
}

}  // namespace mlr
