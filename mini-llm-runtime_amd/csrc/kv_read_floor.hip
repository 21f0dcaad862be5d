// Read-only pass over a decode step's K/V rows: the memory floor of a paged
// decode step, measured on the same block list.
//
// For every sequence b and every context token t < context_lens[b], the
// kernel reads the whole slot row (all KV heads) of K and of V through the
// block table and folds every 32-bit word of it into an XOR checksum, one per
// workgroup. Nothing is computed on the data: what it costs is the read of
// the step's K/V bytes in their paged placement, with the one dependent
// metadata load a decode kernel also has (context length and block ids
// before the first row load).
//
// One workgroup of 256 lanes per (sequence, item of tokens_per_item tokens);
// workgroups past a sequence's context write 0 and exit. The item's block
// ids go to LDS first; then each lane reads 16-byte chunks, chunk c of the
// item being token c / (row_bytes / 16) and byte 16 * (c % (row_bytes / 16))
// of its row, so the lanes of a wave read consecutive bytes of a block.
// kUnroll chunks of K and of V per lane are in flight at once: all of them
// for items of up to 160 tokens of 256-byte rows.
#include "mlr_common.h"

namespace mlr {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 10;
constexpr int kMaxItemBlocks = 512;  // block ids of one item held in LDS

// kPow2: chunks_per_row is 1 << cpr_log2 (32-bit shifts, no division).
template <bool kPow2>
__global__ __launch_bounds__(kThreads) void kv_read_floor_kernel(
    const uint4 *__restrict__ kc, const uint4 *__restrict__ vc, int64_t num_blocks,
    int bs_log2, int chunks_per_row, int cpr_log2, const int64_t *__restrict__ bt,
    int64_t bt_stride, int64_t max_blocks, const int64_t *__restrict__ ctx_lens,
    int items_per_seq, int tokens_per_item, uint32_t *__restrict__ out) {
  __shared__ int64_t ids[kMaxItemBlocks];
  __shared__ uint32_t part[kThreads / 64];
  const int b = blockIdx.x / items_per_seq;
  const int item = blockIdx.x % items_per_seq;
  const int64_t cap = max_blocks << bs_log2;
  int64_t ctx = ctx_lens[b];
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int64_t t0 = static_cast<int64_t>(item) * tokens_per_item;
  const int64_t t1 = t0 + tokens_per_item < ctx ? t0 + tokens_per_item : ctx;
  if (t0 >= t1) {
    if (threadIdx.x == 0) out[blockIdx.x] = 0;
    return;
  }
  const int64_t blk0 = t0 >> bs_log2;
  const int nblk = static_cast<int>(((t1 - 1) >> bs_log2) - blk0 + 1);
  for (int i = threadIdx.x; i < nblk; i += kThreads) ids[i] = bt[b * bt_stride + blk0 + i];
  __syncthreads();

  // Item-relative 32-bit positions: the item holds at most 512 blocks.
  const int bs_mask = (1 << bs_log2) - 1;
  const int nchunks = static_cast<int>(t1 - t0) * chunks_per_row;
  uint32_t acc = 0;
  for (int c0 = threadIdx.x; c0 < nchunks; c0 += kThreads * kUnroll) {
    uint4 kv[2 * kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = c0 + u * kThreads;
      const bool live = c < nchunks;
      const int tr = live ? (kPow2 ? c >> cpr_log2 : c / chunks_per_row) : 0;
      const int pc = kPow2 ? (c & (chunks_per_row - 1)) : c - tr * chunks_per_row;
      const int64_t blk = ids[tr >> bs_log2];  // t0 is block-aligned
      const bool ok = live && blk >= 0 && blk < num_blocks;
      const int64_t at =
          ok ? ((blk << bs_log2) + (tr & bs_mask)) * chunks_per_row + pc : 0;
      kv[2 * u] = ok ? kc[at] : make_uint4(0, 0, 0, 0);
      kv[2 * u + 1] = ok ? vc[at] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 2 * kUnroll; ++u) acc ^= kv[u].x ^ kv[u].y ^ kv[u].z ^ kv[u].w;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc ^= __shfl_xor(acc, m, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

}  // namespace
}  // namespace mlr

extern "C" size_t mlr_paged_kv_read_floor_outputs(int64_t batch, int64_t max_blocks,
                                                  int64_t block_size, int64_t tokens_per_item) {
  if (batch <= 0 || max_blocks <= 0 || block_size <= 0 || tokens_per_item <= 0) return 0;
  const int64_t items = (max_blocks * block_size + tokens_per_item - 1) / tokens_per_item;
  return static_cast<size_t>(batch * items);
}

extern "C" int mlr_paged_kv_read_floor(const void *k_cache, const void *v_cache,
                                       int64_t num_blocks, int64_t block_size,
                                       int64_t row_bytes, const int64_t *block_tables,
                                       int64_t bt_stride, int64_t max_blocks,
                                       const int64_t *context_lens, int64_t batch,
                                       int64_t tokens_per_item, uint32_t *out,
                                       int64_t out_len, void *stream) {
  using namespace mlr;
  clear_error();
  MLR_REQUIRE(batch > 0 && num_blocks > 0 && max_blocks > 0,
              "mlr_paged_kv_read_floor: batch, num_blocks and max_blocks must be > 0");
  MLR_REQUIRE(block_size > 0 && (block_size & (block_size - 1)) == 0,
              "mlr_paged_kv_read_floor: block_size must be a power of two");
  MLR_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0,
              "mlr_paged_kv_read_floor: row_bytes must be a positive multiple of 16");
  MLR_REQUIRE(tokens_per_item > 0 && tokens_per_item % block_size == 0 &&
                  tokens_per_item / block_size <= kMaxItemBlocks,
              "mlr_paged_kv_read_floor: tokens_per_item must be a multiple of block_size, "
              "at most %d blocks",
              kMaxItemBlocks);
  MLR_REQUIRE(bt_stride >= max_blocks, "mlr_paged_kv_read_floor: bt_stride < max_blocks");
  MLR_REQUIRE(k_cache && v_cache && block_tables && context_lens && out,
              "mlr_paged_kv_read_floor: null pointer argument");
  MLR_REQUIRE((reinterpret_cast<uintptr_t>(k_cache) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(v_cache) & 15u) == 0,
              "mlr_paged_kv_read_floor: caches must be 16-byte aligned");
  const int64_t items = (max_blocks * block_size + tokens_per_item - 1) / tokens_per_item;
  MLR_REQUIRE(out_len >= batch * items,
              "mlr_paged_kv_read_floor: out holds %lld words, needs %lld",
              static_cast<long long>(out_len), static_cast<long long>(batch * items));
  MLR_REQUIRE(batch * items <= INT32_MAX && items <= INT32_MAX,
              "mlr_paged_kv_read_floor: grid too large");
  MLR_REQUIRE(tokens_per_item * (row_bytes / 16) < (int64_t(1) << 30),
              "mlr_paged_kv_read_floor: tokens_per_item * row_bytes too large");
  int bs_log2 = 0;
  while ((int64_t(1) << bs_log2) < block_size) ++bs_log2;
  const int cpr = static_cast<int>(row_bytes / 16);
  int cpr_log2 = 0;
  while ((1 << cpr_log2) < cpr) ++cpr_log2;
  const dim3 grid(static_cast<unsigned>(batch * items));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto *k4 = static_cast<const uint4 *>(k_cache);
  const auto *v4 = static_cast<const uint4 *>(v_cache);
  if ((1 << cpr_log2) == cpr) {
    kv_read_floor_kernel<true><<<grid, kThreads, 0, s>>>(
        k4, v4, num_blocks, bs_log2, cpr, cpr_log2, block_tables, bt_stride, max_blocks,
        context_lens, static_cast<int>(items), static_cast<int>(tokens_per_item), out);
  } else {
    kv_read_floor_kernel<false><<<grid, kThreads, 0, s>>>(
        k4, v4, num_blocks, bs_log2, cpr, cpr_log2, block_tables, bt_stride, max_blocks,
        context_lens, static_cast<int>(items), static_cast<int>(tokens_per_item), out);
  }
  return check_launch("mlr_paged_kv_read_floor");
}
