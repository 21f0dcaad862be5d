// bf16 split-KV paged decode on gfx950 matrix cores (pass 1).
//
// One workgroup of four wavefronts per (sequence, KV head, split). The split's
// 16-token tiles are dealt round-robin to the four waves; each wave keeps the
// online-softmax state of all (<= 16) query heads of the KV head's GQA group,
// so every K/V byte is read from HBM exactly once for the whole group.
//
// Per 16-token tile, in one wave:
//   S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//       v_mfma_f32_16x16x32_bf16, D/32 steps. Lane l holds token l%16's K
//       row slice [32j + 8(l/16), +8): the A operand comes straight from a
//       16-byte global load, no LDS.
//   online softmax (FP32, base-2): lane l owns head l%16 and tokens
//       4(l/16)..+3 of the tile; the head's max is two cross-row shuffles.
//   O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//       v_mfma_f32_16x16x16bf16_1k, D/16 tiles. P^T is the S^T accumulator
//       layout itself (rows 4(l/16)+i, column l%16), rounded to bf16. V is
//       loaded as 4 rows x (D/16) dims per lane, so one global_load of 16
//       lanes covers a whole 128/256-byte row, and a 4x4 transpose of 16-bit
//       halves inside the lane builds the A operand: tile n, row m <-> dim
//       (D/16)*m + n.
// The four waves then merge through LDS and write (m, l, acc) for the split,
// which the combine kernel (paged_decode.hip) folds into the output.
//
// Scores are rounded like the reference's bf16 matmul (to bf16, times scale,
// to bf16 again: kernels/reference/paged_attention.py:246-247) before the
// FP32 softmax (:251).
#include "paged_decode.h"

namespace mlr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <int D> struct VRow;
template <> struct VRow<64> { using type = uint2; };   // 4 bf16 per lane
template <> struct VRow<128> { using type = uint4; };  // 8 bf16 per lane

__device__ __forceinline__ float bf16_round(float x) {
  // v_cvt_pk_bf16_f32 rounds to nearest even.
  const __bf16 h = static_cast<__bf16>(x);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
  const __bf16 a = static_cast<__bf16>(lo);
  const __bf16 b = static_cast<__bf16>(hi);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// 16-bit half `h` (0 = low, 1 = high) of word w.
__device__ __forceinline__ uint32_t half16(uint32_t w, int h) {
  return h ? (w >> 16) : (w & 0xffffu);
}

template <int D>
__device__ __forceinline__ uint32_t vword(const typename VRow<D>::type &v, int c) {
  if constexpr (D == 64) {
    return c == 0 ? v.x : v.y;
  } else {
    return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
  }
}

template <int D>
__global__ __launch_bounds__(256) void decode_split_mfma(DecodeParams p) {
  constexpr int QK = D / 32;  // 16x16x32 steps for S^T
  constexpr int VC = D / 16;  // PV tiles = dims per lane per V row
  using VT = typename VRow<D>::type;

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m16 = lane & 15, g = lane >> 4;

  const int64_t cap = p.max_blocks * p.block_size;
  int64_t ctx = p.ctx[b];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int64_t t0 = static_cast<int64_t>(split) * p.ts;
  if (t0 >= ctx) return;  // uniform over the workgroup
  const int64_t t1 = min<int64_t>(ctx, t0 + p.ts);
  const int ntiles = static_cast<int>(ceil_div(t1 - t0, 16));

  // Q^T as the B operand: lane l holds Q[head l%16][32j + 8g .. +8).
  const bool head_ok = m16 < p.group;
  const uint16_t *qrow = static_cast<const uint16_t *>(p.q) + b * p.q_sb +
                         (int64_t)(kvh * p.group + (head_ok ? m16 : 0)) * p.q_sh;
  bf16x8_t qf[QK];
#pragma unroll
  for (int j = 0; j < QK; ++j) {
    uint4 raw = head_ok ? *reinterpret_cast<const uint4 *>(qrow + 32 * j + 8 * g)
                        : make_uint4(0, 0, 0, 0);
    qf[j] = __builtin_bit_cast(bf16x8_t, raw);
  }

  const uint16_t *kc = static_cast<const uint16_t *>(p.kc);
  const uint16_t *vc = static_cast<const uint16_t *>(p.vc);
  const int64_t row_stride = (int64_t)p.hkv * D;  // elements between slots
  const int64_t *bt_row = p.bt + b * p.bt_stride;
  const float scale = static_cast<float>(p.scale);

  f32x4_t acc[VC];
#pragma unroll
  for (int n = 0; n < VC; ++n) acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // This wave's tiles: w, w + 4, w + 8, ...
  const int nk = ntiles > w ? (ntiles - w + kWaves - 1) / kWaves : 0;

  // Block id of the wave's k-th tile lives in lane (k % 64) of blk_reg.
  int blk_reg = -1;
  auto load_block_ids = [&](int kbase) {
    const int k = kbase + lane;
    int id = -1;
    if (k < nk) {
      const int64_t pos = t0 + 16LL * (w + kWaves * k);
      const int64_t blk = bt_row[pos / p.block_size];
      id = (blk >= 0 && blk < p.num_blocks) ? static_cast<int>(blk) : -1;
    }
    blk_reg = id;
  };

  uint4 kcur[QK], knext[QK];
  VT vcur[4], vnext[4];
  auto load_tile = [&](int k, uint4 *kr, VT *vr) {
    const int blk = __builtin_amdgcn_readlane(blk_reg, k & 63);
    const int64_t pos = t0 + 16LL * (w + kWaves * k);
    if (blk >= 0) {
      const int64_t slot0 = (int64_t)blk * p.block_size + pos % p.block_size;
      const uint16_t *kb = kc + (slot0 + m16) * row_stride + (int64_t)kvh * D;
#pragma unroll
      for (int j = 0; j < QK; ++j)
        kr[j] = *reinterpret_cast<const uint4 *>(kb + 32 * j + 8 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t *vb =
            vc + (slot0 + 4 * g + i) * row_stride + (int64_t)kvh * D + VC * m16;
        vr[i] = *reinterpret_cast<const VT *>(vb);
      }
    } else {
#pragma unroll
      for (int j = 0; j < QK; ++j) kr[j] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) vr[i] = VT{};
    }
  };

  if (nk > 0) {
    load_block_ids(0);
    load_tile(0, kcur, vcur);
  }
  for (int k = 0; k < nk; ++k) {
    // Read this tile's block id before the next chunk of ids replaces it.
    const int blk = __builtin_amdgcn_readlane(blk_reg, k & 63);
    const int64_t base = t0 + 16LL * (w + kWaves * k);
    if (k + 1 < nk) {
      if (((k + 1) & 63) == 0) load_block_ids(k + 1);
      load_tile(k + 1, knext, vnext);
    }

    // S^T = K . Q^T
    f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QK; ++j)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8_t, kcur[j]), qf[j], s, 0, 0, 0);

    // Reference rounding, masking past the context, base-2 scaling.
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float r = bf16_round(bf16_round(s[i]) * scale);
      const bool live = blk >= 0 && base + 4 * g + i < t1;
      x[i] = live ? r * kLog2e : -INFINITY;
    }
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const bool any = m_new != -INFINITY;
    const float alpha = any ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pr[i] = any ? __builtin_amdgcn_exp2f(x[i] - m_new) : 0.f;
    l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    m_run = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int n = 0; n < VC; ++n) acc[n] *= alpha;
    }

    // Tokens past the context may hold anything (even NaN): zero their V.
    if (base + 16 > t1) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (base + 4 * g + i >= t1) vcur[i] = VT{};
    }

    s16x4_t pb;
    {
      const uint32_t lo = bf16_pack2(pr[0], pr[1]);
      const uint32_t hi = bf16_pack2(pr[2], pr[3]);
      pb = __builtin_bit_cast(s16x4_t, make_uint2(lo, hi));
    }
#pragma unroll
    for (int n = 0; n < VC; ++n) {
      const int c = n >> 1, h = n & 1;
      const uint32_t lo = half16(vword<D>(vcur[0], c), h) |
                          (half16(vword<D>(vcur[1], c), h) << 16);
      const uint32_t hi = half16(vword<D>(vcur[2], c), h) |
                          (half16(vword<D>(vcur[3], c), h) << 16);
      const s16x4_t va = __builtin_bit_cast(s16x4_t, make_uint2(lo, hi));
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[n], 0, 0, 0);
    }

    if (k + 1 < nk) {
#pragma unroll
      for (int j = 0; j < QK; ++j) kcur[j] = knext[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) vcur[i] = vnext[i];
    }
  }

  // Per-head l: sum the four lanes that share the head.
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);

  __shared__ float o_s[kWaves][16][D + 4];
  __shared__ float m_s[kWaves][16];
  __shared__ float l_s[kWaves][16];
  if (g == 0) {
    m_s[w][m16] = m_run;
    l_s[w][m16] = l_run;
  }
  // Lane l holds O[head l%16][dims VC*(4g+i) + n] = a contiguous 4*VC run.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int n = 0; n < VC; ++n) o_s[w][m16][VC * (4 * g + i) + n] = acc[n][i];
  }
  __syncthreads();

  float *ws_acc = static_cast<float *>(p.ws_acc);
  const int head0 = kvh * p.group;
  for (int idx = threadIdx.x; idx < p.group * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    float M = m_s[0][h];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) M = fmaxf(M, m_s[ww][h]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float f = __builtin_amdgcn_exp2f(m_s[ww][h] - M);
        num += f * o_s[ww][h][d];
        den += f * l_s[ww][h];
      }
    }
    const int64_t row = ((int64_t)b * p.hq + head0 + h) * p.max_splits + split;
    ws_acc[row * D + d] = num;
    if (d == 0) p.ws_ml[row] = make_float2(M == -INFINITY ? M : M * kLn2, den);
  }
}

}  // namespace

bool decode_mfma_eligible(int dtype, int64_t head_dim, int64_t group,
                          int64_t block_size) {
  return dtype == MLR_DTYPE_BF16 && (head_dim == 64 || head_dim == 128) &&
         group >= 1 && group <= 16 && block_size % 16 == 0;
}

int launch_decode_mfma(const DecodeParams &p, hipStream_t stream) {
  dim3 grid(p.max_splits, p.hkv, p.batch);
  if (p.d == 64) {
    decode_split_mfma<64><<<grid, 256, 0, stream>>>(p);
  } else {
    decode_split_mfma<128><<<grid, 256, 0, stream>>>(p);
  }
  int rc = check_launch("mlr_paged_decode(split, mfma)");
  if (rc != MLR_OK) return rc;
  return launch_combine<bf16_t>(p, stream);
}

}  // namespace mlr
