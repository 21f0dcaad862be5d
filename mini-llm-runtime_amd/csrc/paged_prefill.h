// Declarations shared by the chunk-prefill translation units.
#pragma once

#include "mlr_common.h"

namespace mlr {

struct PrefillParams {
  const void *q;
  int64_t q_st, q_sh;
  const void *kc;
  const void *vc;
  int64_t num_blocks;
  int64_t block_size;
  int hkv;
  int d;
  const int64_t *bt;
  int64_t bt_stride;
  int64_t max_blocks;
  const int64_t *qsl;  // [num_seqs + 1] or null (single sequence, scalars below)
  const int64_t *ctx;  // [num_seqs] or null
  int64_t s_qlen;      // single-sequence chunk length
  int64_t s_ctx;       // single-sequence context length
  int num_seqs;
  int hq;
  int group;
  double scale;
  int kv_tile;
  int bs_log2;  // log2(block_size) when it is a power of two, else -1
  int n_qtiles; // query tiles per sequence (matrix-core kernel only)
  int ncu;      // compute units of the device (matrix-core kernel only)
  int pair_cu;  // 1: the launch fits two workgroups per CU (matrix-core kernel)
  void *out;
  int64_t o_st, o_sh;
};

// Sequence metadata as the kernels see it (clamped to the block-table span).
struct SeqRange {
  int64_t q0;      // first query row in q/out
  int64_t qlen;    // query rows
  int64_t prefix;  // absolute position of the first query row
  int64_t ctx;     // keys visible to the last query row
};

__device__ __forceinline__ SeqRange seq_range(const PrefillParams &p, int s) {
  SeqRange r;
  if (p.qsl) {
    r.q0 = p.qsl[s];
    r.qlen = p.qsl[s + 1] - r.q0;
    r.ctx = p.ctx[s];
  } else {
    r.q0 = 0;
    r.qlen = p.s_qlen;
    r.ctx = p.s_ctx;
  }
  const int64_t cap = p.max_blocks * p.block_size;
  if (r.ctx > cap) r.ctx = cap;
  if (r.qlen < 0) r.qlen = 0;
  if (r.qlen > r.ctx) r.qlen = r.ctx;  // never index past the context
  r.prefix = r.ctx - r.qlen;
  return r;
}

// True when the matrix-core kernel covers these arguments (bf16 or fp16,
// head_dim 64 or 128, power-of-two block_size >= 16, aligned rows, positive
// scale).
bool prefill_mfma_eligible(const PrefillParams &p, int dtype);
int launch_prefill_mfma(const PrefillParams &p, int dtype, int64_t max_query_len,
                        hipStream_t stream);

// True when the FP32 matrix-core kernel covers these arguments (FP32,
// head_dim 64 or 128, power-of-two block_size >= 16, 16-byte aligned rows,
// positive scale).
bool prefill_f32_eligible(const PrefillParams &p, int dtype);
int launch_prefill_f32(const PrefillParams &p, int64_t max_query_len, hipStream_t stream);

}  // namespace mlr
