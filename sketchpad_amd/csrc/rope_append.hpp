// Launch interface of the RoPE-fused KV-cache append (rope_append.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

struct RopeAppendArgs {
  char* kpool;
  char* vpool;
  const char* knew;
  const char* vnew;
  int64_t kv_tok_b;        // bytes between tokens of the new K/V rows
  int64_t kv_head_b;       // bytes between heads of the new K/V rows
  char* q;                 // rotated in place; nullptr: no Q rows
  int64_t q_tok_b;
  int64_t q_head_b;
  const int32_t* positions;  // [num_tokens] position of each token in its sequence
  const int32_t* slots;      // [num_tokens] slot mapping
  const float* cos_t;        // [table_rows][head_dim / 2]
  const float* sin_t;
  int table_rows;
  int num_tokens;
  int hkv;
  int hq;
  int head_dim;
  int block_size;
  int64_t block_stride_b;
  int64_t layer_off_b;
  int64_t num_slots;
};

int launch_rope_kv_append(const RopeAppendArgs& a, sp_dtype dtype, hipStream_t stream);

}  // namespace sp
