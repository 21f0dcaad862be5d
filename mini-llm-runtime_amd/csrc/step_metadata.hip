// Per-step model-batch metadata on the device: positions, slot mapping,
// query start offsets and context lengths of a ModelBatch from one row per
// request.
//
// Replaces the per-token host loops of build_model_batch
// (runtime/model_runner.py:54-64 append_slots and the position, offset and
// context-length lists of :66-143). Request r schedules count_r tokens
// starting at position start_r; its tokens occupy rows
// [query_start_loc[r], query_start_loc[r+1]) of the packed batch and
//   positions[j]     = start_r + i
//   slot_mapping[j]  = block_tables[r, p / block_size] * block_size + p % block_size
//   context_lens[r]  = start_r + count_r
// for row j = query_start_loc[r] + i, p = positions[j]. A negative position,
// or one whose block index falls past max_blocks, gets slot -1 (the host
// rejects such requests before the launch, with the reference's message).
//
// Every workgroup prefix-sums the counts into LDS (int32 offsets), then its
// threads take one row each and find the row's request by binary search.
#include "mlr_common.h"

namespace mlr {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxRequests = 16384;

__global__ __launch_bounds__(kThreads) void step_metadata_kernel(
    const int64_t *__restrict__ req_info, const int64_t *__restrict__ bt, int64_t bt_stride,
    int64_t max_blocks, int num_reqs, int num_tokens, int64_t block_size,
    int64_t *__restrict__ positions, int64_t *__restrict__ slots, int64_t *__restrict__ qsl,
    int64_t *__restrict__ ctx) {
  __shared__ int offs[kMaxRequests + 1];
  __shared__ int part[kThreads];
  // Blocked scan: thread k sums the counts of requests [k*per, (k+1)*per).
  const int per = (num_reqs + kThreads - 1) / kThreads;
  const int r0 = threadIdx.x * per, r1 = min(num_reqs, r0 + per);
  int local = 0;
  for (int r = r0; r < r1; ++r) local += static_cast<int>(req_info[2 * r + 1]);
  part[threadIdx.x] = local;
  __syncthreads();
  for (int stride = 1; stride < kThreads; stride <<= 1) {  // inclusive scan of part
    const int add = threadIdx.x >= stride ? part[threadIdx.x - stride] : 0;
    __syncthreads();
    part[threadIdx.x] += add;
    __syncthreads();
  }
  int run = threadIdx.x == 0 ? 0 : part[threadIdx.x - 1];
  for (int r = r0; r < r1; ++r) {
    offs[r] = run;
    run += static_cast<int>(req_info[2 * r + 1]);
  }
  if (threadIdx.x == kThreads - 1) offs[num_reqs] = part[kThreads - 1];
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int r = threadIdx.x; r <= num_reqs; r += kThreads) {
      qsl[r] = offs[r];
      if (r < num_reqs) ctx[r] = req_info[2 * r] + req_info[2 * r + 1];
    }
  }
  const int j = blockIdx.x * kThreads + threadIdx.x;
  if (j >= num_tokens) return;
  // Last request whose first row is <= j (empty requests are skipped).
  int lo = 0, hi = num_reqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offs[mid] <= j) lo = mid; else hi = mid - 1;
  }
  const int64_t pos = req_info[2 * lo] + (j - offs[lo]);
  const int64_t blk = pos / block_size;
  positions[j] = pos;
  slots[j] = (pos >= 0 && blk < max_blocks)
                 ? bt[lo * bt_stride + blk] * block_size + pos % block_size
                 : -1;
}

}  // namespace
}  // namespace mlr

extern "C" int mlr_build_step_metadata(const int64_t *req_info, const int64_t *block_tables,
                                       int64_t block_table_stride, int64_t max_blocks,
                                       int64_t num_reqs, int64_t num_tokens,
                                       int64_t block_size, int64_t *positions,
                                       int64_t *slot_mapping, int64_t *query_start_loc,
                                       int64_t *context_lens, void *stream) {
  using namespace mlr;
  clear_error();
  MLR_REQUIRE(num_reqs >= 0 && num_reqs <= kMaxRequests,
              "mlr_build_step_metadata: num_reqs must be in [0, %d]", kMaxRequests);
  MLR_REQUIRE(num_tokens >= 0 && num_tokens < (int64_t(1) << 31),
              "mlr_build_step_metadata: num_tokens must be in [0, 2^31)");
  MLR_REQUIRE(block_size > 0, "mlr_build_step_metadata: block_size must be > 0");
  MLR_REQUIRE(max_blocks >= 0 && block_table_stride >= max_blocks,
              "mlr_build_step_metadata: block table stride smaller than its width");
  MLR_REQUIRE(num_reqs > 0 || num_tokens == 0,
              "mlr_build_step_metadata: tokens without requests");
  if (num_reqs == 0) return MLR_OK;
  MLR_REQUIRE(req_info && query_start_loc && context_lens, "mlr_build_step_metadata: null pointer");
  MLR_REQUIRE(num_tokens == 0 || (positions && slot_mapping && block_tables),
              "mlr_build_step_metadata: null pointer");
  const int64_t blocks = num_tokens > 0 ? (num_tokens + kThreads - 1) / kThreads : 1;
  step_metadata_kernel<<<static_cast<unsigned>(blocks), kThreads, 0,
                         static_cast<hipStream_t>(stream)>>>(
      req_info, block_tables, block_table_stride, max_blocks, static_cast<int>(num_reqs),
      static_cast<int>(num_tokens), block_size, positions, slot_mapping, query_start_loc,
      context_lens);
  return check_launch("mlr_build_step_metadata");
}
