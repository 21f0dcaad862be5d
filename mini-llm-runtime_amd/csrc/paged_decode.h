// Declarations shared by the decode translation units.
#pragma once

#include "mlr_common.h"

namespace mlr {

// Everything a decode kernel needs; built once by mlr_paged_decode.
struct DecodeParams {
  const void *q;
  int64_t q_sb, q_sh;
  const void *kc;
  const void *vc;
  int64_t num_blocks;
  int64_t block_size;
  int hkv;
  int d;
  const int64_t *bt;
  int64_t bt_stride;
  int64_t max_blocks;
  const int64_t *ctx;
  int batch;
  int hq;
  int group;
  double scale;
  int ts;          // tokens per split
  int max_splits;  // splits covering max_blocks * block_size tokens
  int split_stride;  // workspace rows per (sequence, query head): max_splits
                     // rounded up to kSplitRowPad
  uint32_t *ws_flag;  // failure word of the single-launch merge (zero: none)
  float2 *ws_ml;   // [batch][hq][max_splits] = (m, l)
  void *ws_acc;    // [batch][hq][max_splits][d], FP32 (FP64 for f64 inputs)
  int ml_base2;    // 1: m is a base-2 exponent, 0: natural-log units
  int dtype;       // mlr_dtype of q, the cache and out
  void *out;
  int64_t o_sb, o_sh;
  // Fused KV write (mlr_paged_decode_append); new_k == nullptr: none.
  const void *new_k;
  const void *new_v;
  int64_t new_sb, new_sh;
  const int64_t *new_slots;
  void *kc_w;  // writable views of kc / vc
  void *vc_w;
  // Fused rotary embedding (mlr_paged_decode_qkv; inv_freq == nullptr:
  // none): q and the new K/V rows are the QKV projection's rows; q and the
  // new K row are rotated for position context_lens[b] - 1.
  const float *inv_freq;
};

// Workspace: a 256-byte flag region, then the split partials (m, l) and acc,
// each 256-byte aligned. Every byte of it is zero between calls: each call
// returns the partial rows it wrote to zero once they are merged, whatever
// kernel wrote them, so calls of any shape can share one workspace.
constexpr int64_t kFlagBytes = 256;
// Rows per (sequence, query head) come in multiples of this, so the merge can
// read 16 consecutive split rows of one head without leaving that head's rows.
constexpr int64_t kSplitRowPad = 16;
struct DecodeWorkspace {
  int64_t ml_offset;
  int64_t acc_offset;
  int64_t total;
};

// Tokens per split of the head_dim-64 matrix-core kernel whose waves land a
// fifth tile in LDS.
constexpr int kLdsSplit64 = 320;

int64_t default_tokens_per_split(bool mfma, int64_t head_dim, int64_t max_context, int dtype);
DecodeWorkspace decode_workspace_layout(int64_t batch, int64_t hq, int64_t d,
                                        int64_t max_splits, int dtype);

// bf16, fp16 or FP32, head_dim 64/128, GQA group <= 16 and block_size a
// multiple of 16.
bool decode_mfma_eligible(int dtype, int64_t head_dim, int64_t group,
                          int64_t block_size);
int launch_decode_mfma(const DecodeParams &p, hipStream_t stream);

template <typename T>
int launch_combine(const DecodeParams &p, hipStream_t stream);

}  // namespace mlr
