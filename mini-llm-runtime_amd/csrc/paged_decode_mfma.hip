// bf16, fp16 and FP32 split-KV paged decode on gfx950 matrix cores, in one launch.
//
// One workgroup of four wavefronts per (live split, KV head), or of eight per
// (live split, pair of KV heads), four for each head (FP32 grids that leave
// most CUs idle: eight wavefronts per KV head). A split is
// tokens_per_split tokens of one sequence; the live splits of all sequences
// are numbered sequence by sequence and every workgroup finds its own from a
// prefix sum of the context lengths, so no workgroup is spent on a split past
// a sequence's end (only the grid's tail, sized for the widest table, exits
// at once). The split's
// 16-token tiles are dealt round-robin to a head's waves; each wave keeps the
// online-softmax state of all (<= 16) query heads of the KV head's GQA group,
// so every K/V byte is read from HBM exactly once for the whole group.
//
// Per 16-token tile, in one wave:
//   S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//       v_mfma_f32_16x16x32_bf16, D/32 steps. Lane l holds token l%16's K
//       row slice [32j + 8(l/16), +8): the A operand comes straight from a
//       16-byte global load, no LDS.
//   online softmax (FP32, base-2): lane l owns head l%16 and tokens
//       4(l/16)..+3 of the tile; the head's max is two lane swaps
//       (v_permlane16_swap, v_permlane32_swap).
//   O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//       v_mfma_f32_16x16x16bf16_1k, D/16 tiles. P^T is the S^T accumulator
//       layout itself (rows 4(l/16)+i, column l%16), rounded to bf16. V is
//       loaded as 4 rows x (D/16) dims per lane, so one global_load of 16
//       lanes covers a whole 128/256-byte row, and a 4x4 transpose of 16-bit
//       halves inside the lane builds the A operand: tile n, row m <-> dim
//       (D/16)*m + n.
// Memory-level parallelism: a wave issues the loads of a whole batch of
// kBatch tiles at once and the next batch's loads before computing the
// current one (two register buffers), so 8-16 KiB per wave are in flight.
//
// A KV head's waves merge through LDS. A sequence that fits one split writes its
// output directly; otherwise every split but the last stores its (m, l, acc)
// to the workspace with device-coherent stores, each word encoded so that
// zero means "not stored yet", and the workgroup of the last split (the
// group's highest index, dispatched after the others) reads the rows until
// every word has arrived and merges them with its own split:
//   M = max_s m_s,  out = sum_s 2^{m_s - M} acc_s / sum_s 2^{m_s - M} l_s,
// returning the rows to zero for the next call. That saves the second launch
// of a separate combine kernel (about 1.9 us of launch gap plus a memory
// round trip per step), and, against a merge by the last split to finish
// (stores, wait for them, bump a counter, read), two of the three dependent
// memory round trips at the end of the step. The partials go through memory,
// not an XCD's L2, so the merge holds wherever the hardware places the
// workgroups.
//
// Scores are rounded like the reference's bf16 matmul (to bf16, times scale,
// to bf16 again: kernels/reference/paged_attention.py:246-247) before the
// FP32 softmax (:251).
//
// fp16 inputs take the bf16 layout with v_mfma_f32_16x16x32_f16 and
// v_mfma_f32_16x16x16_f16, and round scores and probabilities to fp16 where
// the bf16 tile rounds to bf16 (the reference's fp16 matmul, scale and
// probs.to(v.dtype)).
//
// FP32 inputs take the same kernel with v_mfma_f32_16x16x4_f32 in place of
// the bf16 instructions (compute_tile for Tile<float, D>): its 16x16
// accumulator has the bf16 tiles' layout, so the softmax, the merges, the
// work items and the fused KV write are shared. Scores, probabilities and
// P@V stay FP32, as in the reference's FP32 path.
#include "paged_decode.h"

namespace mlr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // waves per KV head, unless a launch picks another count
constexpr float kLog2e = 1.4426950408889634f;

template <int D> struct VRow;
template <> struct VRow<64> { using type = uint2; };   // 4 bf16 per lane
template <> struct VRow<128> { using type = uint4; };  // 8 bf16 per lane
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));

// What one lane holds of a 16-token tile, by element type (bf16_t or float):
// K as kKChunks 16-byte chunks of token l%16's row (8 bf16 or 4 floats each:
// the elements 4 kE j + kE g .. + kE of chunk j, kE = 16 / element size,
// g = l/16), and V as rows 4g .. 4g + 3, D/16 elements each (VT).
template <typename T, int D> struct TileTraits;
template <int D> struct TileTraits<bf16_t, D> {
  static constexpr int kKChunks = D / 32;
  using VT = typename VRow<D>::type;
  using S = uint16_t;  // storage element
};
template <int D> struct TileTraits<f16_t, D> : TileTraits<bf16_t, D> {};
template <> struct TileTraits<float, 64> {
  static constexpr int kKChunks = 4;
  using VT = uint4;
  using S = float;
};
template <> struct TileTraits<float, 128> {
  static constexpr int kKChunks = 8;
  using VT = u32x8_t;
  using S = float;
};

// a and b rounded to bf16 (nearest even) and back to FP32, with one
// v_cvt_pk_bf16_f32 for the pair.
__device__ __forceinline__ void bf16_round2(float &a, float &b) {
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{a, b}, bf16x2_v));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  const __bf16 a = static_cast<__bf16>(lo);
  const __bf16 b = static_cast<__bf16>(hi);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

__device__ __forceinline__ float bf16_elem(const uint4 &v, int e) {
  const uint32_t w = e < 2 ? v.x : (e < 4 ? v.y : (e < 6 ? v.z : v.w));
  return bf16_bits_to_float((e & 1) ? (w >> 16) : (w & 0xffffu));
}

__device__ __forceinline__ float f16_elem(const uint4 &v, int e) {
  const uint32_t w = e < 2 ? v.x : (e < 4 ? v.y : (e < 6 ? v.z : v.w));
  return f16_bits_to_float(static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu)));
}

// a and b rounded to fp16 (nearest even) and back to FP32.
__device__ __forceinline__ void f16_round2(float &a, float &b) {
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
  const f16x2_v h = __builtin_convertvector(f32x2_v{a, b}, f16x2_v);
  a = static_cast<float>(h[0]);
  b = static_cast<float>(h[1]);
}

__device__ __forceinline__ uint32_t f16_pack2(float lo, float hi) {
  const _Float16 a = static_cast<_Float16>(lo);
  const _Float16 b = static_cast<_Float16>(hi);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// The 16-bit element types on the matrix cores: the reference computes q.k,
// the scale and the probabilities in the input dtype, so the tile rounds
// them to that dtype (nearest even), and the MFMAs take that dtype's
// operands with FP32 accumulation.
template <typename T> struct Half16;
template <> struct Half16<bf16_t> {
  using v8 = bf16x8_t;
  __device__ static void round2(float &a, float &b) { bf16_round2(a, b); }
  __device__ static uint32_t pack2(float lo, float hi) { return bf16_pack2(lo, hi); }
  __device__ static float elem(const uint4 &v, int e) { return bf16_elem(v, e); }
  __device__ static f32x4_t qk(uint4 k, v8 q, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, k), q, c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(s16x4_t v, s16x4_t p, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v, p, c, 0, 0, 0);
  }
  __device__ static uint16_t store(float x) { return float_to_bf16_bits(x); }
};
template <> struct Half16<f16_t> {
  using v8 = f16x8_t;
  __device__ static void round2(float &a, float &b) { f16_round2(a, b); }
  __device__ static uint32_t pack2(float lo, float hi) { return f16_pack2(lo, hi); }
  __device__ static float elem(const uint4 &v, int e) { return f16_elem(v, e); }
  __device__ static f32x4_t qk(uint4 k, v8 q, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, k), q, c, 0, 0, 0);
  }
  __device__ static f32x4_t pv(s16x4_t v, s16x4_t p, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, v),
                                                 __builtin_bit_cast(f16x4_t, p), c, 0, 0, 0);
  }
  __device__ static uint16_t store(float x) { return float_to_f16_bits(x); }
};

// Rotary embedding of one (x[i], x[i + d/2]) pair in bf16 or fp16 as the
// reference's apply_rotary_pos_emb computes it (model/qwen2.py:125-209),
// operation by operation: each product and the sum rounded to the 16-bit type
// (nearest even), no fused multiply-add. The products are rounded here, two
// at a time (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32); the sums come back
// unrounded, and Half16<T>::pack2 rounds them as it packs two outputs into one
// word. (For fp16, rounding an FP32 sum or product of two fp16 values to fp16
// equals rounding the exact result once: FP32 carries more than 2 x 11 + 2
// bits.)
template <typename T>
__device__ __forceinline__ void rope_pair(float x_lo, float x_hi, float c, float s,
                                          float &sum_lo, float &sum_hi) {
#pragma clang fp contract(off)
  float a = x_lo * c, b = -x_hi * s;
  float e = x_hi * c, f = x_lo * s;
  Half16<T>::round2(a, b);
  Half16<T>::round2(e, f);
  sum_lo = a + b;
  sum_hi = e + f;
}

// Butterfly steps across lanes l ^ 16 and l ^ 32 as VALU lane swaps
// (v_permlane16_swap / v_permlane32_swap), not LDS permutes: after the swap
// of x with itself, the two halves of the result hold x of both partners, in
// every lane. max and + are commutative, so the results equal those of a
// __shfl_xor butterfly bit for bit.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Reductions over each 16-lane row of a wave (lanes 16r .. 16r + 15) with DPP
// moves inside the row (quad xor 1, quad xor 2, half-row mirror, row mirror):
// afterwards every lane of the row holds its row's result. VALU only, no LDS
// permutes; every lane of the row must be active.
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp_move<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = fmaxf(x, dpp_move<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = fmaxf(x, dpp_move<0x141>(x));  // row_half_mirror
  return fmaxf(x, dpp_move<0x140>(x));  // row_mirror
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_move<0xB1>(x);
  x += dpp_move<0x4E>(x);
  x += dpp_move<0x141>(x);
  return x + dpp_move<0x140>(x);
}

template <int D>
__device__ __forceinline__ uint32_t vword(const typename VRow<D>::type &v, int c) {
  if constexpr (D == 64) {
    return c == 0 ? v.x : v.y;
  } else {
    return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
  }
}

// c ? a : b for the HIP vector structs, as a select of native vectors (a
// ternary on the structs themselves goes through stack copies).
template <typename T>
__device__ __forceinline__ T select_vec(bool c, const T &a, const T &b) {
  typedef uint32_t words_t __attribute__((ext_vector_type(sizeof(T) / 4)));
  const words_t wa = __builtin_bit_cast(words_t, a), wb = __builtin_bit_cast(words_t, b);
  const words_t m = c ? ~words_t(0) : words_t(0);
  return __builtin_bit_cast(T, (wa & m) | (wb & ~m));
}

// Registers of one loaded tile. blk and rel are wave-uniform.
template <typename T, int D>
struct Tile {
  uint4 k[TileTraits<T, D>::kKChunks];
  typename TileTraits<T, D>::VT v[4];
  int blk;  // physical block id, -1 when the tile is absent or invalid
  int rel;  // position of the tile's first token relative to the split start
  int sub;  // row (0..15) whose K/V the appended token replaces, or -1
};

template <int D>
struct DecodeState {
  f32x4_t acc[D / 16];
  float m, l;
};

// Per-lane byte offsets inside a 16-token tile, fixed for the whole kernel.
struct LaneOffsets {
  int k;       // K row of token m16, chunk 0 of lane group g: ((m16 * hkv + kvh) * D) * size + 16g
  int v;       // V row of token 4g, dims VC*m16..: ((4g * hkv + kvh) * D + VC*m16) * size
  int v_step;  // bytes between consecutive token rows (hkv * D * size)
};

// Raw buffer resource over one physical block (gfx9 descriptor word 3). The
// base is wave-uniform, so the loads use a scalar descriptor plus 32-bit lane
// offsets, and the hardware drops any access outside the block.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const void *base,
                                                             uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

template <typename T, int D>
__device__ __forceinline__ void load_tile(Tile<T, D> &t, const typename TileTraits<T, D>::S *kc,
                                          const typename TileTraits<T, D>::S *vc,
                                          int64_t block_elems, int tile_off_bytes, int blk,
                                          int rel, const LaneOffsets &o) {
  constexpr int QK = TileTraits<T, D>::kKChunks;
  using VT = typename TileTraits<T, D>::VT;
  constexpr int kSize = static_cast<int>(sizeof(T));
  t.blk = blk;
  t.rel = rel;
  t.sub = -1;
  // The loads are issued for absent tiles too, through an empty resource
  // (they return zeros and touch no memory): loads under a branch would make
  // the compiler's wait counts assume the fewest loads on any path, so the
  // first tile would wait for nearly every load of the batch.
  const bool ok = blk >= 0;
  const uint32_t bytes = ok ? static_cast<uint32_t>(block_elems * kSize) : 0u;
  const int64_t base = ok ? (int64_t)blk * block_elems : 0;
  const __amdgpu_buffer_rsrc_t rk = block_rsrc(kc + base, bytes);
  const __amdgpu_buffer_rsrc_t rv = block_rsrc(vc + base, bytes);
#pragma unroll
  for (int j = 0; j < QK; ++j)
    t.k[j] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, o.k + 64 * j, tile_off_bytes, 0));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (sizeof(VT) == 8) {
      t.v[i] = __builtin_bit_cast(
          VT, __builtin_amdgcn_raw_buffer_load_b64(rv, o.v + i * o.v_step, tile_off_bytes, 0));
    } else if constexpr (sizeof(VT) == 16) {
      t.v[i] = __builtin_bit_cast(
          VT, __builtin_amdgcn_raw_buffer_load_b128(rv, o.v + i * o.v_step, tile_off_bytes, 0));
    } else {  // 32 bytes: two loads
      const uint4 lo = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, o.v + i * o.v_step, tile_off_bytes, 0));
      const uint4 hi = __builtin_bit_cast(
          uint4,
          __builtin_amdgcn_raw_buffer_load_b128(rv, o.v + i * o.v_step + 16, tile_off_bytes, 0));
      t.v[i] = VT{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// A tile landed in LDS instead of registers (head_dim 64): 16 rows of one KV
// head, K (2 KB) then V (2 KB), copied straight from memory by
// buffer_load_dwordx4 ... lds (lane l of copy i writes LDS bytes
// 1024 i + 16 l). Row r's 16-byte chunk c lands at chunk c ^ (r & 7), which
// keeps the fragment reads below free of bank conflicts: the eight lanes of a
// K read (rows 0..7, one logical chunk) and the sixteen of a V read (one row,
// consecutive 8-byte pieces) each cover 128 distinct bytes of banks.
constexpr int kLdsTileBytes = 4096;

__device__ __forceinline__ void copy_tile_to_lds(unsigned char *dst, const uint16_t *kc,
                                                 const uint16_t *vc, int64_t block_elems,
                                                 int tile_off_bytes, int blk, int kvh,
                                                 int row_bytes, int lane) {
  const bool ok = blk >= 0;
  const uint32_t bytes = ok ? static_cast<uint32_t>(block_elems * 2) : 0u;
  const int64_t base = ok ? (int64_t)blk * block_elems : 0;
  const __amdgpu_buffer_rsrc_t rk = block_rsrc(kc + base, bytes);
  const __amdgpu_buffer_rsrc_t rv = block_rsrc(vc + base, bytes);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * i + (lane >> 3);
    const int src_chunk = (lane & 7) ^ (row & 7);
    const uint32_t off = static_cast<uint32_t>(row * row_bytes + kvh * 128 + 16 * src_chunk);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void_t *)(dst + 1024 * i), 16, off,
                                             tile_off_bytes, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void_t *)(dst + 2048 + 1024 * i), 16, off,
                                             tile_off_bytes, 0, 0);
  }
}

// The register fragments of a tile landed by copy_tile_to_lds, in the layout
// load_tile gives them (head_dim 64).
template <typename T>
__device__ __forceinline__ void read_tile_from_lds(Tile<T, 64> &t, const unsigned char *src,
                                                   int blk, int rel, int m16, int g) {
  t.blk = blk;
  t.rel = rel;
  t.sub = -1;
#pragma unroll
  for (int j = 0; j < 2; ++j)  // K row m16, elements 32j + 8g .. +8
    t.k[j] = *reinterpret_cast<const uint4 *>(src + m16 * 128 + 16 * ((4 * j + g) ^ (m16 & 7)));
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // V row 4g + i, elements 4 m16 .. +4
    const int row = 4 * g + i;
    t.v[i] = *reinterpret_cast<const uint2 *>(src + 2048 + row * 128 +
                                              16 * ((m16 >> 1) ^ (row & 7)) + 8 * (m16 & 1));
  }
}

// The online-softmax update of one tile: x[i] are the base-2 scores of the
// lane's tokens 4g + i for head l%16 (-inf where masked; every tile has a
// live token). Updates (m, l), rescales acc when m moved, and returns the
// probabilities.
template <int D>
__device__ __forceinline__ void softmax_update(DecodeState<D> &st, const float (&x)[4],
                                               float (&pr)[4]) {
  float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  mx = max_xor32(max_xor16(mx));
  const float m_new = fmaxf(st.m, mx);  // finite: every tile has a live token
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
#pragma unroll
  for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
  st.l = st.l * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
  st.m = m_new;
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int n = 0; n < D / 16; ++n) st.acc[n] *= alpha;
  }
}

// With kAppend, row t.sub of the tile (if any) takes the appended token's K
// and V rows, staged in LDS (new_row: K row then V row), in place of what was
// read from the cache; the substitution is a per-lane select at compute time,
// so it never waits on the tile's loads and holds no registers before.
// bf16 and fp16 (Half16 gives the dtype's rounding and MFMAs).
template <int D, bool kAppend, typename T>
__device__ __forceinline__ void compute_tile(DecodeState<D> &st, Tile<T, D> &t,
                                             const typename Half16<T>::v8 *qf, float scale,
                                             int live, int g, int m16,
                                             const uint16_t *new_row) {
  using H = Half16<T>;
  constexpr int QK = D / 32, VC = D / 16;
  using VT = typename VRow<D>::type;
  if (t.blk < 0) return;  // absent tile or invalid block id: no keys (uniform)
  const int lim = live - t.rel;  // tokens of this tile inside the context
  if constexpr (kAppend) {
    if (t.sub >= 0) {  // uniform
      const bool k_row = m16 == t.sub;
#pragma unroll
      for (int j = 0; j < QK; ++j)
        t.k[j] = select_vec(k_row, *reinterpret_cast<const uint4 *>(new_row + 32 * j + 8 * g),
                            t.k[j]);
      const VT vrow = *reinterpret_cast<const VT *>(new_row + D + VC * m16);
#pragma unroll
      for (int i = 0; i < 4; ++i) t.v[i] = select_vec(4 * g + i == t.sub, vrow, t.v[i]);
    }
  }

  f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < QK; ++j) s = H::qk(t.k[j], qf[j], s);
  float r[4] = {s[0], s[1], s[2], s[3]};
  H::round2(r[0], r[1]);
  H::round2(r[2], r[3]);
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] *= scale;
  H::round2(r[0], r[1]);
  H::round2(r[2], r[3]);
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = (4 * g + i < lim) ? r[i] * kLog2e : -INFINITY;
  float pr[4];
  softmax_update(st, x, pr);
  // Tokens past the context may hold anything (even NaN): zero their V.
  if (lim < 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i >= lim) t.v[i] = VT{};
  }
  const s16x4_t pb = __builtin_bit_cast(
      s16x4_t, make_uint2(H::pack2(pr[0], pr[1]), H::pack2(pr[2], pr[3])));
#pragma unroll
  for (int n = 0; n < VC; ++n) {
    const int c = n >> 1, h = n & 1;
    // Half h of the words of rows 0/1 (and 2/3), one v_perm_b32 each.
    const uint32_t sel = h ? 0x07060302u : 0x05040100u;
    const uint32_t lo = __builtin_amdgcn_perm(vword<D>(t.v[1], c), vword<D>(t.v[0], c), sel);
    const uint32_t hi = __builtin_amdgcn_perm(vword<D>(t.v[3], c), vword<D>(t.v[2], c), sel);
    const s16x4_t va = __builtin_bit_cast(s16x4_t, make_uint2(lo, hi));
    st.acc[n] = H::pv(va, pb, st.acc[n]);
  }
}

// The FP32 tile, on v_mfma_f32_16x16x4_f32 (FP32 products, FP32 sums) with
// the accumulator layouts of the bf16 tile, so the softmax and the merges are
// shared. S^T: step (j, e) takes dims 16j + 4g + e of lane group g from K
// chunk j (its 16-byte load) and the matching q chunk. O^T: step i takes
// tokens 4g + i, whose probability is the lane's pr[i]; dim block c takes
// dims VC*m + c of the V rows (VC = D/16 floats per lane and row), so
// accumulator c holds O[dim VC*(4g + i) + c][head l%16], as in the bf16
// tile. Scores are q.k times scale in FP32, as the reference's FP32 matmul
// and scale give them (kernels/reference/paged_attention.py:246-247).
template <int D, bool kAppend>
__device__ __forceinline__ void compute_tile(DecodeState<D> &st, Tile<float, D> &t,
                                             const f32x4_t *qf, float scale, int live, int g,
                                             int m16, const float *new_row) {
  constexpr int QK = D / 16, VC = D / 16;
  using VT = typename TileTraits<float, D>::VT;
  typedef float vf_t __attribute__((ext_vector_type(VC)));
  if (t.blk < 0) return;  // absent tile or invalid block id: no keys (uniform)
  const int lim = live - t.rel;  // tokens of this tile inside the context
  if constexpr (kAppend) {
    if (t.sub >= 0) {  // uniform
      const bool k_row = m16 == t.sub;
#pragma unroll
      for (int j = 0; j < QK; ++j)
        t.k[j] = select_vec(k_row, *reinterpret_cast<const uint4 *>(new_row + 16 * j + 4 * g),
                            t.k[j]);
      const VT vrow = *reinterpret_cast<const VT *>(new_row + D + VC * m16);
#pragma unroll
      for (int i = 0; i < 4; ++i) t.v[i] = select_vec(4 * g + i == t.sub, vrow, t.v[i]);
    }
  }
  f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < QK; ++j) {
    const f32x4_t k = __builtin_bit_cast(f32x4_t, t.k[j]);
#pragma unroll
    for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_16x16x4f32(k[e], qf[j][e], s, 0, 0, 0);
  }
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = (4 * g + i < lim) ? (s[i] * scale) * kLog2e : -INFINITY;
  float pr[4];
  softmax_update(st, x, pr);
  // Tokens past the context may hold anything (even NaN): zero their V.
  if (lim < 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i >= lim) t.v[i] = VT{};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const vf_t v = __builtin_bit_cast(vf_t, t.v[i]);
#pragma unroll
    for (int c = 0; c < VC; ++c)
      st.acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[c], pr[i], st.acc[c], 0, 0, 0);
  }
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Where one work item lies: sequence b, split, and the sequence's clamped
// context length and split count.
struct WorkItem {
  int b;  // -1: past the last live item
  int split;
  int ctx;
  int ns;
};

// Work items are the live (sequence, split) pairs, sequence b having
// ns_b = ceil(ctx_b / ts) splits, in three runs:
//   1. every split but the last of each sequence with two or more splits,
//      sequence by sequence in split order (the producers of the merge);
//   2. the last splits of those sequences, which merge their sequence's
//      splits: dispatched after every split they wait for, and, with their
//      own tokens streamed after the producers', they usually find the
//      partials already published;
//   3. the sequences that fit one split (nothing to merge).
// Every wave derives the same answer from the context lengths (64 per round
// trip), so no workgroup is spent on a split past its sequence's end, and no
// host-side prefix is needed.
__device__ __forceinline__ WorkItem find_item(const DecodeParams &p, int j, int64_t cap) {
  const int lane = threadIdx.x & 63;
  WorkItem it{-1, 0, 0, 0};
  auto splits_of = [&](int c0, int &ctx) -> int {
    const int idx = c0 + lane;
    int64_t c = idx < p.batch ? p.ctx[idx] : 0;  // lanes past the batch: no splits
    c = c < 0 ? 0 : (c > cap ? cap : c);
    ctx = static_cast<int>(c);  // < 2^31 on this path
    return (ctx + p.ts - 1) / p.ts;
  };
  // Run 1, and the number of sequences with two or more splits.
  int carry = 0, nmerge = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) {
    int ctx;
    const int ns = splits_of(c0, ctx);
    const int np = ns > 1 ? ns - 1 : 0;
    const int incl = carry + wave_inclusive_scan(np);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (it.b < 0 && j >= carry && j < total) {  // uniform: the item lies in this chunk
      // Sequences wholly before item j are the lanes whose prefix is <= j
      // (the prefix is non-decreasing; lanes past the batch carry the total).
      const int bl = __popcll(__ballot(incl <= j));
      it.b = c0 + bl;
      it.ns = __builtin_amdgcn_readlane(ns, bl);
      it.split = j - (__builtin_amdgcn_readlane(incl, bl) - __builtin_amdgcn_readlane(np, bl));
      it.ctx = __builtin_amdgcn_readlane(ctx, bl);
    }
    carry = total;
    nmerge += __popcll(__ballot(ns > 1));
  }
  if (it.b >= 0) return it;
  // Runs 2 and 3: the k-th sequence with two or more splits (its last
  // split), else the k-th sequence with one split.
  int k = j - carry;
  const bool merging = k < nmerge;
  if (!merging) k -= nmerge;
  int before = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) {
    int ctx;
    const int ns = splits_of(c0, ctx);
    const uint64_t sel = __ballot(merging ? ns > 1 : ns == 1);
    const int cnt = __popcll(sel);
    if (k < before + cnt) {  // uniform
      // The selected lane with k - before selected lanes below it.
      const int upto = __popcll(sel & ((2ull << lane) - 1));  // selected lanes <= this one
      const int bl = __popcll(__ballot(upto <= k - before));
      it.b = c0 + bl;
      it.ns = __builtin_amdgcn_readlane(ns, bl);
      it.split = merging ? it.ns - 1 : 0;
      it.ctx = __builtin_amdgcn_readlane(ctx, bl);
      break;
    }
    before += cnt;
  }
  return it;
}

// Device-coherent stores and loads of the split partials (the sc1 cache
// policy, bit 4 of the buffer intrinsics' aux operand on gfx950): stores are
// written through to memory and loads are not served from a possibly stale
// L2 line, so a workgroup on any XCD reads what another wrote once the
// store has reached memory, and a read issued earlier returns the old word.
// Plain buffer loads, not atomic ones: relaxed atomic loads whose addresses
// might alias are issued one at a time, these are issued back to back.
constexpr int kCoherent = 16;

// A partial word in the workspace is the value's bits with the sign bit
// flipped, after NaNs become the canonical quiet NaN and -0 becomes +0: no
// value is stored as zero, so a word is zero exactly when its producer has
// not stored it yet, and a zero word reads back as -0 (a finite value that a
// zero weight cancels). Aligned 32-bit stores and loads are single-copy
// atomic, so a word is read whole or not at all.
__device__ __forceinline__ void publish(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  uint32_t u = v != v ? 0x7FC00000u : __float_as_uint(v);
  u = u == 0x80000000u ? 0u : u;
  __builtin_amdgcn_raw_buffer_store_b32(u ^ 0x80000000u, r, off, 0, kCoherent);
}
__device__ __forceinline__ float unpublish(uint32_t w) { return __uint_as_float(w ^ 0x80000000u); }

// One work item (a split of one sequence, one KV head) for the workgroup.
// kH KV heads per workgroup (1 or 2), kW waves each: waves
// hs * kW .. + kW - 1 serve KV head kvh_base + hs over the same
// tiles, so with kH = 2 both halves of every slot row are requested by one
// workgroup at the same time.
template <typename T, int D, int kBatch, bool kDouble, bool kAppend, bool kLds, int kH,
          bool kRope, int kW>
__device__ __forceinline__ void decode_item(const DecodeParams &p, const WorkItem &it,
                                            int kvh_base) {
  constexpr bool kF32 = std::is_same<T, float>::value;
  constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
  static_assert(kF32 || kBf16 || std::is_same<T, f16_t>::value, "bf16, fp16 or FP32 elements");
  static_assert(!kF32 || !kLds, "the LDS tile is for 16-bit elements");
  static_assert(!kRope || !kF32, "the rotary embedding is bf16 or fp16");
  using S = typename TileTraits<T, D>::S;  // storage element
  constexpr int QK = TileTraits<T, D>::kKChunks;
  constexpr int kSize = static_cast<int>(sizeof(T));
  constexpr int kE = 16 / kSize;          // elements per 16-byte chunk
  constexpr int kRowChunks = D / kE;      // 16-byte chunks per K (or V) row of one head
  constexpr int VC = D / 16;
  constexpr int kThreads = 64 * kW * kH;
  const int lane = threadIdx.x & 63;
  // The wave index is uniform within a wave; saying so keeps every value
  // derived from it (tile counts, block ids, descriptors) in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = wave % kW;   // the wave's place among its KV head's waves
  const int hs = wave / kW;  // which of the workgroup's KV heads it serves
  const int kvh = kvh_base + hs;
  const int m16 = lane & 15, g = lane >> 4;
  const int b = it.b, split = it.split, nsplits = it.ns;
  const int64_t ctx = it.ctx;
  const int64_t t0 = static_cast<int64_t>(split) * p.ts;
  const int64_t *bt_row = p.bt + b * p.bt_stride;

  // Prologue: the Q fragments and the first 64 block ids of this wave do not
  // depend on one another, so both loads are issued before either is used.
  // Block ids are read for every tile position the split could hold, within
  // the table's width.
  // The GQA group's q rows lie under one buffer resource; lanes past the
  // group read beyond its range and get zeros. No branch and no select, so
  // nothing makes the compiler wait for these loads before it issues the
  // block-id and tile loads (a conditional load here did, on the rotary
  // variant: one more memory round trip ahead of the tile loads).
  const bool head_ok = m16 < p.group;
  const uint32_t q_bytes =
      static_cast<uint32_t>(((int64_t)(p.group - 1) * p.q_sh + D) * kSize);
  const __amdgpu_buffer_rsrc_t q_r = block_rsrc(
      static_cast<const S *>(p.q) + b * p.q_sb + (int64_t)(kvh * p.group) * p.q_sh, q_bytes);
  const uint32_t q_off = head_ok ? static_cast<uint32_t>(m16 * p.q_sh * kSize) : q_bytes;
  uint4 qraw[QK];
#pragma unroll
  for (int j = 0; j < QK; ++j)
    qraw[j] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(q_r, q_off + (4 * kE * j + kE * g) * kSize, 0, 0));
  // Token positions fit in 32 bits here (max_blocks * block_size < 2^31;
  // speculative tile positions stay below 2^32): block index and offset by
  // shift and mask when block_size is a power of two, else 32-bit division.
  const uint32_t bs32 = static_cast<uint32_t>(p.block_size);
  const bool bs_pow2 = (bs32 & (bs32 - 1)) == 0;
  const uint32_t bs_shift = static_cast<uint32_t>(__builtin_ctz(bs32));
  auto block_of = [&](uint32_t pos) -> uint32_t {
    return bs_pow2 ? (pos >> bs_shift) : pos / bs32;
  };
  auto in_block = [&](uint32_t pos) -> uint32_t {
    return bs_pow2 ? (pos & (bs32 - 1)) : pos % bs32;
  };
  auto raw_block_id = [&](int k) -> int64_t {
    const int64_t idx = block_of(static_cast<uint32_t>(t0) + 16u * (w + kW * k));
    return idx < p.max_blocks ? bt_row[idx] : int64_t(-1);
  };
  int64_t blk_raw = raw_block_id(lane);
  const int64_t t1 = min<int64_t>(ctx, t0 + p.ts);
  // Fused KV write: the new token (position ctx - 1) lives in the last tile of
  // the last split, and the wave that owns that tile (tiles are dealt
  // round-robin) takes the new K/V rows: their slot and rows (16 bytes per
  // lane) come with the prologue, so staging them (LDS and cache) waits for no
  // tile load, and as the same wave reads them back no barrier is needed.
  const int64_t last_pos = ctx - 1;
  const bool append_here = kAppend && last_pos >= t0 && last_pos < t1;
  const int last_rel = static_cast<int>(last_pos - t0) & ~15;  // tile of ctx - 1
  const int last_tok = static_cast<int>(last_pos - t0) & 15;   // its row
  const bool new_owner = append_here && w == (last_rel >> 4) % kW;  // uniform
  __shared__ __align__(16) S new_row_s[kH][2 * D];
  const int64_t new_slot = kAppend ? p.new_slots[b] : -1;
  const bool new_is_v = lane >= kRowChunks;
  const int new_off = kE * (new_is_v ? lane - kRowChunks : lane);
  uint4 new_chunk = make_uint4(0, 0, 0, 0);
  if (new_owner && lane < 2 * kRowChunks)
    new_chunk = *reinterpret_cast<const uint4 *>(
        static_cast<const S *>(new_is_v ? p.new_v : p.new_k) + b * p.new_sb +
        (int64_t)kvh * p.new_sh + new_off);
  // Fused rotary embedding (p.inv_freq set; fused write only): every wave
  // puts cos and sin of the decode position ctx - 1 for the d/2 frequencies,
  // rounded to the 16-bit type, in its own LDS row and rotates q and the new K row with
  // them, as the fused pre-attention kernel does (qkv_rope.hip), once the
  // tile loads are in flight. The frequency is loaded here, before the tile
  // loads: memory loads complete in order, so a load issued after them
  // could only be used once they had all landed.
  static_assert(kAppend || !kRope, "the rotary embedding rides on the fused write");
  constexpr bool rope = kRope;
  __shared__ float rope_s[kW * kH][D];  // cos at [i], sin at [d/2 + i]
  float rope_freq = 0.f;
  // Every lane loads (lanes past d/2 a duplicate, never used): no branch.
  if (rope) rope_freq = p.inv_freq[lane & (D / 2 - 1)];

  const int ntiles = static_cast<int>(ceil_div(t1 - t0, 16));

  // Q^T as the B operand: lane l holds Q[head l%16][4kE j + kE g .. +kE)
  // (bf16: 32j + 8g; FP32: 16j + 4g), the dims of its K chunks.
  using QF = typename std::conditional<kF32, f32x4_t,
                                       typename std::conditional<kBf16, bf16x8_t, f16x8_t>::type>::type;
  QF qf[QK];
#pragma unroll
  for (int j = 0; j < QK; ++j) qf[j] = __builtin_bit_cast(QF, qraw[j]);
  // Rotates the lane's q fragments: fragment j < QK/2 holds dims
  // 32j + 8g + e (e < 8) and fragment j + QK/2 their partners d/2 further, so
  // each pair is in one lane. LDS operations of one wave complete in order,
  // so the wave reads back the cos/sin it has just written; the wave barrier
  // (no instruction) keeps the compiler from moving the other lanes' reads
  // above those writes.
  auto rotate_q = [&]() {
    if constexpr (kRope) {
    using H = Half16<T>;
    if (lane < D / 2) {
      // sincosf shares one argument reduction between the two; its results
      // are those of cosf and sinf.
      float sn, cs;
      sincosf(static_cast<float>(ctx - 1) * rope_freq, &sn, &cs);
      H::round2(cs, sn);
      rope_s[wave][lane] = cs;
      rope_s[wave][D / 2 + lane] = sn;
    }
    __builtin_amdgcn_wave_barrier();
    if (!head_ok) return;  // columns past the group stay zero
#pragma unroll
    for (int j = 0; j < QK / 2; ++j) {
      const int i0 = 32 * j + 8 * g;
      float lo[8], hi[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        rope_pair<T>(H::elem(qraw[j], e), H::elem(qraw[j + QK / 2], e), rope_s[wave][i0 + e],
                     rope_s[wave][D / 2 + i0 + e], lo[e], hi[e]);
      qf[j] = __builtin_bit_cast(QF, make_uint4(H::pack2(lo[0], lo[1]), H::pack2(lo[2], lo[3]),
                                                H::pack2(lo[4], lo[5]), H::pack2(lo[6], lo[7])));
      qf[j + QK / 2] =
          __builtin_bit_cast(QF, make_uint4(H::pack2(hi[0], hi[1]), H::pack2(hi[2], hi[3]),
                                            H::pack2(hi[4], hi[5]), H::pack2(hi[6], hi[7])));
    }
    }
  };

  const S *kc = static_cast<const S *>(p.kc);
  const S *vc = static_cast<const S *>(p.vc);
  const float scale = static_cast<float>(p.scale);

  DecodeState<D> st;
#pragma unroll
  for (int n = 0; n < VC; ++n) st.acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  // This wave's tiles: w, w + kW, w + 2 kW, ...; block id of the wave's k-th
  // tile lives in lane (k % 64) of blk_reg (-1: no tile or invalid id).
  const int nk = ntiles > w ? (ntiles - w + kW - 1) / kW : 0;
  auto valid_id = [&](int k, int64_t raw) -> int {
    return (k < nk && raw >= 0 && raw < p.num_blocks) ? static_cast<int>(raw) : -1;
  };
  int blk_reg = valid_id(lane, blk_raw);
  auto load_block_ids = [&](int kbase) {
    if (kbase == 0) return;  // the prologue loaded the first 64
    const int k = kbase + lane;
    blk_reg = valid_id(k, k < nk ? raw_block_id(k) : int64_t(-1));
  };
  const int row_elems = p.hkv * D;  // elements of one slot (token row)
  const int64_t block_elems = p.block_size * row_elems;
  LaneOffsets lo;
  lo.k = (m16 * p.hkv + kvh) * D * kSize + 16 * g;
  lo.v = ((4 * g * p.hkv + kvh) * D + VC * m16) * kSize;
  lo.v_step = row_elems * kSize;
  const int live = static_cast<int>(t1 - t0);
  // The owning wave stores the new K/V rows to slot new_slots[b] and to LDS,
  // and, when that slot is the one position ctx - 1 maps to, uses them in
  // place of what it read from the cache for that row. Called once, after
  // the wave's first batch of tile loads is issued. LDS operations of one
  // wave complete in order, so the wave's later reads of new_row_s see these
  // writes.
  // With the fused rotary embedding each K lane takes the chunk of its
  // rotary partner (K chunks of lanes l and l ^ d/16 hold dims i and
  // i + d/2) and rotates its own, so the slot and LDS receive the finished
  // rows.
  auto stage_new_row = [&]() {
    if (!new_owner) return;  // uniform
    uint4 v = new_chunk;
    if constexpr (kRope) {
      using H = Half16<T>;
      uint4 xp;
      xp.x = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v.x), D / 16, 64));
      xp.y = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v.y), D / 16, 64));
      xp.z = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v.z), D / 16, 64));
      xp.w = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v.w), D / 16, 64));
      if (!new_is_v) {
        const bool low = new_off < D / 2;
        const int i0 = low ? new_off : new_off - D / 2;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = H::elem(v, e), xo = H::elem(xp, e);
          float ol, oh;
          rope_pair<T>(low ? x : xo, low ? xo : x, rope_s[wave][i0 + e],
                       rope_s[wave][D / 2 + i0 + e], ol, oh);
          o[e] = low ? ol : oh;
        }
        v = make_uint4(H::pack2(o[0], o[1]), H::pack2(o[2], o[3]), H::pack2(o[4], o[5]),
                       H::pack2(o[6], o[7]));
      }
    }
    if (lane < 2 * kRowChunks) {
      *reinterpret_cast<uint4 *>(new_row_s[hs] + (new_is_v ? D : 0) + new_off) = v;
      const int64_t num_slots = p.num_blocks * p.block_size;
      if (new_slot >= 0 && new_slot < num_slots) {
        S *dst = static_cast<S *>(new_is_v ? p.vc_w : p.kc_w) +
                 (new_slot * p.hkv + kvh) * D + new_off;
        *reinterpret_cast<uint4 *>(dst) = v;
      }
    }
    // Every lane of this wave reads the staged rows at compute time.
    __builtin_amdgcn_wave_barrier();
  };
  // Marks row last_tok of the new token's tile for substitution when the
  // new slot is the one position ctx - 1 maps to.
  auto mark_new_row = [&](Tile<T, D> &t) {
    const bool same_slot =
        t.blk >= 0 &&
        new_slot == (int64_t)t.blk * p.block_size + in_block(static_cast<uint32_t>(last_pos));
    if (same_slot) t.sub = last_tok;
  };

  auto issue = [&](Tile<T, D>(&buf)[kBatch], int kb) {
    if ((kb & 63) == 0) load_block_ids(kb);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = kb + u;
      const int blk = k < nk ? __builtin_amdgcn_readlane(blk_reg, k & 63) : -1;
      const int rel = 16 * (w + kW * k);
      // Byte offset of the tile's first token inside its block.
      const int tile_off =
          static_cast<int>(in_block(static_cast<uint32_t>(t0) + rel)) * row_elems * kSize;
      load_tile<T, D>(buf[u], kc, vc, block_elems, tile_off, blk, rel, lo);
    }
    if (append_here) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int k = kb + u;
        if (k < nk && 16 * (w + kW * k) == last_rel) mark_new_row(buf[u]);
      }
    }
  };
  auto compute = [&](Tile<T, D>(&buf)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      compute_tile<D, kAppend>(st, buf[u], qf, scale, live, g, m16, new_row_s[hs]);
  };

  // The wave holding the new token stages its rows once, after its first
  // batch of loads is in flight.
  if constexpr (kDouble) {
    // Next batch in flight while the current one computes.
    // Batches are issued whether or not they hold tiles (absent tiles read
    // zeros), so the wait before each compute counts only its own batch.
    Tile<T, D> bufA[kBatch], bufB[kBatch];
    issue(bufA, 0);
    if (rope) rotate_q();
    if (append_here) stage_new_row();
    for (int kb = 0; kb < nk; kb += 2 * kBatch) {
      issue(bufB, kb + kBatch);
      compute(bufA);
      if (kb + kBatch >= nk) break;
      issue(bufA, kb + 2 * kBatch);
      compute(bufB);
    }
  } else if constexpr (kLds) {
    // Five tiles per wave (320-token splits): four in registers and the
    // fifth in this wave's LDS slot, all issued up front, so that one
    // workgroup keeps 80 KB in flight and the splits of a batch like 64
    // sequences of up to 4K tokens fit the GPU in one generation.
    static_assert(D == 64 && kBatch == 4 && !kF32,
                  "LDS landing is laid out for 16-bit elements at head_dim 64");
    __shared__ __align__(16) unsigned char lds_tiles[kW * kH][kLdsTileBytes];
    Tile<T, D> buf[kBatch];
    issue(buf, 0);
    const int rel4 = 16 * (w + kW * kBatch);
    const int blk4 = kBatch < nk ? __builtin_amdgcn_readlane(blk_reg, kBatch) : -1;
    copy_tile_to_lds(lds_tiles[wave], kc, vc, block_elems,
                     static_cast<int>(in_block(static_cast<uint32_t>(t0) + rel4)) * row_elems * 2,
                     blk4, kvh, row_elems * 2, lane);
    if (rope) rotate_q();
    if (append_here) stage_new_row();
    compute(buf);
    if (kBatch < nk) {  // uniform
      read_tile_from_lds(buf[0], lds_tiles[wave], blk4, rel4, m16, g);
      if (append_here && rel4 == last_rel) mark_new_row(buf[0]);
      compute_tile<D, kAppend>(st, buf[0], qf, scale, live, g, m16, new_row_s[hs]);
    }
  } else {
    // Issued whatever nk is (absent tiles read zeros), so that every path
    // reaching the computes has the same loads in flight.
    Tile<T, D> buf[kBatch];
    issue(buf, 0);
    if (rope) rotate_q();
    if (append_here) stage_new_row();
    for (int kb = 0; kb < nk; kb += kBatch) {
      if (kb > 0) issue(buf, kb);
      compute(buf);
    }
  }

  // Per-head l: sum the four lanes that share the head.
  st.l = sum_xor32(sum_xor16(st.l));

  __shared__ float o_s[kW * kH][16][D + 4];
  __shared__ float m_s[kW * kH][16];
  __shared__ float l_s[kW * kH][16];
  if (g == 0) {
    m_s[wave][m16] = st.m;
    l_s[wave][m16] = st.l;
  }
  // Lane l holds O[head l%16][dims VC*(4g+i) + n].
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int n = 0; n < VC; ++n) o_s[wave][m16][VC * (4 * g + i) + n] = st.acc[n][i];
  }
  __syncthreads();

  // Merge the waves of each KV head. A sequence that fits one split is
  // finished here. Otherwise splits 0 .. nsplits - 2 publish their (m, l,
  // acc) rows to the workspace (m as a base-2 exponent) and the sequence's
  // last split merges them with its own, which it keeps. The workgroup's
  // query heads are the kH GQA groups of its KV heads, ngh in all; thread t
  // holds the outputs t + kThreads r (head (t + kThreads r) / D, dim
  // (t + kThreads r) % D).
  const int ngh = kH * p.group;
  const int head0 = kvh_base * p.group;
  S *out = static_cast<S *>(p.out);
  auto store_out = [&](float x) -> S {
    if constexpr (kF32) return x;
    else return Half16<T>::store(x);
  };
  // The workgroup's partial rows: (m, l) pairs and acc rows for its heads h
  // and splits s at row h * split_stride + s, under buffer resources of their
  // span (at most 16 heads x 8192 splits x 128 dims of FP32: 32-bit offsets).
  const int64_t row_b = (int64_t)b * p.hq + head0;
  const int rows_g = ngh * p.split_stride;
  const __amdgpu_buffer_rsrc_t acc_r = __builtin_amdgcn_make_buffer_rsrc(
      static_cast<float *>(p.ws_acc) + row_b * p.split_stride * D, 0,
      static_cast<uint32_t>(rows_g) * D * 4u, 0x00020000);
  const __amdgpu_buffer_rsrc_t ml_r = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<float *>(p.ws_ml) + row_b * p.split_stride * 2, 0,
      static_cast<uint32_t>(rows_g) * 8u, 0x00020000);
  const bool merger = nsplits > 1 && split == nsplits - 1;
  // Outputs per thread, at most (at least the merge's kPre per pass).
  constexpr int kMaxOut = (16 * D + kThreads - 1) / kThreads < 2 ? 2
                                                                  : (16 * D + kThreads - 1) / kThreads;
  const int nout = ngh * D;
  float own[kMaxOut];
  __shared__ float own_m_s[16], own_l_s[16];
#pragma unroll
  for (int r = 0; r < kMaxOut; ++r) {
    const int idx = threadIdx.x + kThreads * r;
    own[r] = 0.f;
    if (idx < nout) {
      const int h = idx / D, d = idx % D;
      // Waves w0 .. w0 + kW - 1 hold head h (head hg of their group).
      const int w0 = kH == 1 ? 0 : (h / p.group) * kW;
      const int hg = kH == 1 ? h : h % p.group;
      float M = m_s[w0][hg];
#pragma unroll
      for (int ww = 1; ww < kW; ++ww) M = fmaxf(M, m_s[w0 + ww][hg]);
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int ww = 0; ww < kW; ++ww) {
        const float f = __builtin_amdgcn_exp2f(m_s[w0 + ww][hg] - M);
        num += f * o_s[w0 + ww][hg][d];
        den += f * l_s[w0 + ww][hg];
      }
      if (nsplits == 1) {
        out[b * p.o_sb + (int64_t)(head0 + h) * p.o_sh + d] = store_out(num / den);
      } else if (merger) {
        own[r] = num;
        if (d == 0) {
          own_m_s[h] = M;
          own_l_s[h] = den;
        }
      } else {
        const uint32_t row = static_cast<uint32_t>(h * p.split_stride + split);
        publish(acc_r, (row * D + d) * 4u, num);
        if (d == 0) {
          publish(ml_r, row * 8u, M);
          publish(ml_r, row * 8u + 4u, den);
        }
      }
    }
  }
  if (!merger) return;

  // The group merge, in split order: splits 0 .. nsplits - 2 from the
  // workspace, kChunk per round trip, and this workgroup's own split folded
  // in with the last chunk:
  //   M = max_s m_s,  out = sum_s 2^{m_s - M} acc_s / sum_s 2^{m_s - M} l_s
  // (the numerators add in split order; a chunk's part of the denominator is
  // a reduction over its 16 splits).
  // A chunk is read again until every word of it has arrived (none is zero).
  // Its producers are workgroups of lower index, dispatched before this one:
  // they hold or held a slot and finish without waiting on anything, so the
  // wait ends; a wait past kMaxPolls reads means that assumption failed, and
  // the merge then records the failure in the workspace's flag word and
  // writes NaN (as it does when the flag word was already set). Words that
  // were read are returned to zero.
  constexpr int kChunk = 16;
  constexpr int kMaxPolls = 1 << 17;
  static_assert(kSplitRowPad % kChunk == 0, "a chunk's rows stay inside one head's rows");
  __shared__ float f_s[kChunk + 1][16];  // 2^{m_s - M_new}: the chunk's splits, then own
  __shared__ float rescale_s[16];      // 2^{M_old - M_new} per head
  __shared__ float den_s[16];
  __shared__ float mrun_s[16];
  if (threadIdx.x < 16) {
    den_s[threadIdx.x] = 0.f;
    mrun_s[threadIdx.x] = -INFINITY;
  }
  // Outputs per thread whose partial rows are in flight together: two cover
  // up to 2 * kThreads outputs (ngh * head_dim) in one pass.
  constexpr int kPre = 2;
  const int nprev = nsplits - 1;
  // Thread t reads the (m, l) pair of head t / kChunk, split s0 + t % kChunk
  // (threads past the group read head 0's: neither checked nor used).
  const int mh = threadIdx.x / kChunk, ms = threadIdx.x % kChunk;
  const bool ml_real = mh < ngh;
  // The workspace's flag word: set by an earlier merge that gave up, it
  // means the workspace may hold stale rows, so nothing read from it can be
  // trusted. Read with the first chunk, in the same round trip.
  const __amdgpu_buffer_rsrc_t flag_r =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_flag, 0, 4u, 0x00020000);
  __shared__ uint32_t flag_s;
  bool failed = false;
  float num[kMaxOut];
#pragma unroll
  for (int r = 0; r < kMaxOut; ++r) num[r] = 0.f;
  for (int s0 = 0; s0 < nprev && !failed; s0 += kChunk) {
    const int cnt = min(kChunk, nprev - s0);
    const bool last = s0 + kChunk >= nprev;  // own split folds in here
    const uint32_t live = (1u << cnt) - 1u;  // the chunk's splits, as bits
    const uint32_t mloff =
        static_cast<uint32_t>((ml_real ? mh : 0) * p.split_stride + s0 + ms) * 8u;
#pragma unroll
    for (int pass = 0; pass < kMaxOut / kPre; ++pass) {
      if (pass * kPre * kThreads >= nout) break;  // uniform
      // Per thread one byte offset per output at split s0; split s0 + s is
      // s * D * 4 bytes further (an immediate offset). All kChunk rows are
      // read: they lie inside the head's rows (split_stride is a multiple of
      // kChunk), and those past cnt are neither checked nor used (they hold
      // zero, which reads as -0, and their weight is 0).
      // (Signed offsets: their sums cannot wrap, so the constant part can go
      // to the instruction's immediate offset field.)
      int abase[kPre];
#pragma unroll
      for (int r = 0; r < kPre; ++r) {
        const int idx = threadIdx.x + kThreads * (pass * kPre + r);
        const int h = idx < nout ? idx / D : 0, d = idx % D;
        abase[r] = ((h * p.split_stride + s0) * D + d) * 4;
      }
      uint32_t a[kPre][kChunk], mw = 0, lw = 0;
      for (int tries = 0;; ++tries) {
        // Opaque to the optimiser, so that the split offsets are added inside
        // the loop and land in the loads' immediate fields instead of being
        // hoisted into one register per load.
#pragma unroll
        for (int r = 0; r < kPre; ++r) asm volatile("" : "+v"(abase[r]));
#pragma unroll
        for (int s = 0; s < kChunk; ++s) {
#pragma unroll
          for (int r = 0; r < kPre; ++r)
            a[r][s] = __builtin_amdgcn_raw_buffer_load_b32(acc_r, abase[r] + s * D * 4, 0,
                                                           kCoherent);
        }
        if (pass == 0) {
          mw = __builtin_amdgcn_raw_buffer_load_b32(ml_r, mloff, 0, kCoherent);
          lw = __builtin_amdgcn_raw_buffer_load_b32(ml_r, mloff + 4u, 0, kCoherent);
        }
        // A zero word among the chunk's splits that exist. Head_dim 64: the
        // unsigned minimum over them is zero; head_dim 128: a bit mask of the
        // zero words, tested against the splits that exist. (Measured, A/B on
        // one box: the minimum took the 64 x 4K-context step from 21.51-21.55
        // to 21.40-21.43 us, but the 8 x 32K decode at head_dim 128 from
        // 100.0-100.6 to 100.7-101.5 us.)
        bool missing = false;
#pragma unroll
        for (int r = 0; r < kPre; ++r) {
          bool zero;
          if constexpr (D == 64) {
            uint32_t mn = ~0u;
#pragma unroll
            for (int s = 0; s < kChunk; ++s) mn = min(mn, s < cnt ? a[r][s] : ~0u);
            zero = mn == 0u;
          } else {
            uint32_t z = 0;
#pragma unroll
            for (int s = 0; s < kChunk; ++s) z |= (a[r][s] == 0u ? 1u : 0u) << s;
            zero = (z & live) != 0u;
          }
          missing |= threadIdx.x + kThreads * (pass * kPre + r) < nout && zero;
        }
        if (pass == 0) missing |= ml_real && ms < cnt && (mw == 0u || lw == 0u);
        const bool first = s0 == 0 && pass == 0 && tries == 0;  // uniform
        if (first && threadIdx.x == 0)
          flag_s = __builtin_amdgcn_raw_buffer_load_b32(flag_r, 0u, 0, kCoherent);
        const bool any_missing = __syncthreads_or(missing);  // uniform
        if (first && flag_s != 0u) {  // uniform: read by all after the barrier
          failed = true;
          break;
        }
        if (!any_missing) break;
        if (tries == kMaxPolls) {
          failed = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (failed) break;  // uniform
      // Every word of the pass has arrived: return them to zero. (Threads
      // past the group's outputs point at head 0's words of the chunk, which
      // were read too: storing zero there again needs no per-lane test.)
#pragma unroll
      for (int r = 0; r < kPre; ++r) asm volatile("" : "+v"(abase[r]));
#pragma unroll
      for (int s = 0; s < kChunk; ++s) {
        if (s < cnt) {  // uniform
#pragma unroll
          for (int r = 0; r < kPre; ++r)
            __builtin_amdgcn_raw_buffer_store_b32(0u, acc_r, abase[r] + s * D * 4, 0, kCoherent);
        }
      }
      if (pass == 0) {
        if (ml_real && ms < cnt) {
          __builtin_amdgcn_raw_buffer_store_b32(0u, ml_r, mloff, 0, kCoherent);
          __builtin_amdgcn_raw_buffer_store_b32(0u, ml_r, mloff + 4u, 0, kCoherent);
        }
        // The chunk's weights, one (head mh, split s0 + ms) per thread: the
        // 16 threads of a head are one 16-lane row of a wave, so the head's
        // new reference point and its part of the denominator are DPP
        // reductions inside the row. Rows past cnt weigh 0 (their l word is
        // zero, read as -0).
        if (mh < 16) {
          const int h = mh;
          const float m_old = mrun_s[h];
          const float mc = ms < cnt ? unpublish(mw) : -INFINITY;
          float m_new = row_max16(fmaxf(m_old, mc));
          if (last) m_new = fmaxf(m_new, own_m_s[h]);
          const float f = ms < cnt ? __builtin_amdgcn_exp2f(mc - m_new) : 0.f;
          const float part = row_sum16(f * unpublish(lw));
          f_s[ms][h] = f;
          if (ms == 0) {
            const float rs = __builtin_amdgcn_exp2f(m_old - m_new);  // 0 on the first chunk
            const float f_own = last ? __builtin_amdgcn_exp2f(own_m_s[h] - m_new) : 0.f;
            f_s[kChunk][h] = f_own;
            rescale_s[h] = rs;
            den_s[h] = den_s[h] * rs + part + f_own * own_l_s[h];
            mrun_s[h] = m_new;
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int r = 0; r < kPre; ++r) {
        const int idx = threadIdx.x + kThreads * (pass * kPre + r);
        if (idx < nout) {
          const int h = idx / D;
          float acc = num[pass * kPre + r] * rescale_s[h];
#pragma unroll
          for (int s = 0; s < kChunk; ++s)
            acc += f_s[s][h] * unpublish(a[r][s]);  // rows past cnt: f = 0, word 0 (-0)
          acc += f_s[kChunk][h] * own[pass * kPre + r];  // 0 before the last chunk
          num[pass * kPre + r] = acc;
        }
      }
    }
  }
  if (failed) {
    if (threadIdx.x == 0) __builtin_amdgcn_raw_buffer_store_b32(1u, flag_r, 0u, 0, kCoherent);
#pragma unroll
    for (int r = 0; r < kMaxOut; ++r) {
      const int idx = threadIdx.x + kThreads * r;
      if (idx < nout)
        out[b * p.o_sb + (int64_t)(head0 + idx / D) * p.o_sh + idx % D] = store_out(__builtin_nanf(""));
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < kMaxOut; ++r) {
    const int idx = threadIdx.x + kThreads * r;
    if (idx < nout) {
      const int h = idx / D, d = idx % D;
      out[b * p.o_sb + (int64_t)(head0 + h) * p.o_sh + d] = store_out(num[r] / den_s[h]);
    }
  }
}

// One workgroup per (live item, kH KV heads). The KV-head groups of one
// (sequence, split) are adjacent workgroups; the grid is sized for the widest
// table and the workgroups past the live items exit after the context
// lengths.
template <typename T, int D, int kBatch, bool kDouble, bool kAppend, bool kLds, int kH,
          bool kRope, int kW>
__global__ __launch_bounds__(64 * kW * kH) void decode_mfma(DecodeParams p) {
  const int64_t cap = p.max_blocks * p.block_size;
  const int nhg = p.hkv / kH;  // KV-head groups per item
  const WorkItem it = find_item(p, blockIdx.x / nhg, cap);
  if (it.b < 0) return;  // uniform
  decode_item<T, D, kBatch, kDouble, kAppend, kLds, kH, kRope, kW>(p, it,
                                                                  (blockIdx.x % nhg) * kH);
}

}  // namespace

bool decode_mfma_eligible(int dtype, int64_t head_dim, int64_t group,
                          int64_t block_size) {
  return (dtype == MLR_DTYPE_BF16 || dtype == MLR_DTYPE_F16 || dtype == MLR_DTYPE_F32) &&
         (head_dim == 64 || head_dim == 128) && group >= 1 && group <= 16 &&
         block_size % 16 == 0;
}

template <typename T, int D, int B, bool DB, bool A, bool L, int H, bool R, int W>
int launch_one(const DecodeParams &p, hipStream_t stream) {
  // Every (sequence, split) item that can exist, times the KV-head groups.
  const int64_t items = (int64_t)p.batch * p.max_splits * (p.hkv / H);
  if (items > 0x7fffffff)
    return set_error(MLR_ERR_UNSUPPORTED, "mlr_paged_decode: %lld work items exceed the grid",
                     (long long)items);
  decode_mfma<T, D, B, DB, A, L, H, R, W><<<dim3(static_cast<unsigned>(items)), 64 * W * H,
                                            0, stream>>>(p);
  return check_launch("mlr_paged_decode(mfma)");
}

// The three variants of one layout: decode only, with the fused KV write,
// and with the fused write and rotary embedding (their own instantiations,
// so the rotary code costs the other two nothing; bf16 and fp16).
template <typename T, int D, int B, bool DB, bool L, int H = 1, int W = kWaves>
int launch_variant(const DecodeParams &p, hipStream_t stream) {
  if (p.new_k == nullptr) return launch_one<T, D, B, DB, false, L, H, false, W>(p, stream);
  if constexpr (!std::is_same<T, float>::value) {
    if (p.inv_freq != nullptr) return launch_one<T, D, B, DB, true, L, H, true, W>(p, stream);
  }
  return launch_one<T, D, B, DB, true, L, H, false, W>(p, stream);
}

// bf16 and fp16 instantiations: head_dim x (one load batch | + LDS tile |
// double-buffered) x KV heads per workgroup x variant (with or without the
// rotary embedding).
template <typename T>
int launch_16bit(const DecodeParams &p, int tiles_per_wave, bool pairs, hipStream_t stream) {
  if (p.d == 64) {
    if (tiles_per_wave <= 4) return launch_variant<T, 64, 4, false, false>(p, stream);
    if (p.ts == kLdsSplit64) {
      if (pairs) return launch_variant<T, 64, 4, false, true, 2>(p, stream);
      return launch_variant<T, 64, 4, false, true>(p, stream);
    }
    return launch_variant<T, 64, 4, true, false>(p, stream);
  }
  if (pairs) {
    if (tiles_per_wave <= 2) return launch_variant<T, 128, 2, false, false, 2>(p, stream);
    return launch_variant<T, 128, 2, true, false, 2>(p, stream);
  }
  if (tiles_per_wave <= 2) return launch_variant<T, 128, 2, false, false>(p, stream);
  return launch_variant<T, 128, 2, true, false>(p, stream);
}

int launch_decode_mfma(const DecodeParams &p, hipStream_t stream) {
  // Tiles per wave: ceil(ts / 16 / 4). A split whose tiles fit one load batch
  // needs no second register buffer (fewer VGPRs, more waves per SIMD); at
  // head_dim 64 a 320-token split lands its fifth tile per wave in LDS.
  const int tiles_per_wave = static_cast<int>(ceil_div(ceil_div(p.ts, 16), kWaves));
  // Both KV heads of a pair go to one eight-wave workgroup when their GQA
  // groups fit the merge's 16 query-head rows and the paired grid still has a
  // workgroup for every CU. Measured: batch 64 x 14/2 heads, head_dim 64,
  // 320-token splits: 21.8 us per step against 22.2 us (fused write), 21.9
  // against 22.2 (decode only); 8 x 32K tokens, 28/4 heads, head_dim 128:
  // 100.7 us against 107.8 us at 16 splits, 109.7 against 113.5 at 32, but
  // 119.7 against 104.2 at 8 splits (128 paired workgroups for 256 CUs).
  const int cus = current_device_cus();
  const bool pairs = p.hkv % 2 == 0 && 2 * p.group <= 16 && cus > 0 &&
                     (int64_t)p.batch * p.max_splits * (p.hkv / 2) >= cus;
  // FP32: a tile takes twice the registers of a bf16 one. At head_dim 64 up to
  // four tiles per wave go in one batch (batch 4 x {17, 64, 130, 255} tokens,
  // 14/2 heads: 8.42 us per step against 8.57 us in two double-buffered
  // batches of two), longer splits in double-buffered batches of two; at
  // head_dim 128 one tile per batch. One KV head per workgroup.
  if (p.dtype == MLR_DTYPE_F32) {
    // A grid that leaves most CUs idle (work items for under a quarter of
    // them) spreads each split of up to 16 tiles over eight waves, two tiles
    // each: the split's matrix-core work runs on twice as many SIMDs. At
    // fp32_decode_b4 (8 work items): 7.04 us per step against 8.32 us with
    // four waves and 7.66 us with 16 waves of one tile (10-call graphs,
    // alternating libraries on one box).
    const int64_t items = (int64_t)p.batch * p.max_splits * p.hkv;
    const bool spread = cus > 0 && 4 * items <= cus && ceil_div(p.ts, 16) <= 16;
    if (p.d == 64) {
      if (spread) return launch_variant<float, 64, 2, false, false, 1, 8>(p, stream);
      if (tiles_per_wave <= 4) return launch_variant<float, 64, 4, false, false>(p, stream);
      return launch_variant<float, 64, 2, true, false>(p, stream);
    }
    if (tiles_per_wave <= 1) return launch_variant<float, 128, 1, false, false>(p, stream);
    return launch_variant<float, 128, 1, true, false>(p, stream);
  }
  if (p.dtype == MLR_DTYPE_F16) return launch_16bit<f16_t>(p, tiles_per_wave, pairs, stream);
  return launch_16bit<bf16_t>(p, tiles_per_wave, pairs, stream);
}

}  // namespace mlr

