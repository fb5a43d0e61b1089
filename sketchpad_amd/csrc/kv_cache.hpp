// Launch interfaces of the paged KV-cache append / gather kernels (kv_cache.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

struct KvAppendArgs {
  char* kpool;
  char* vpool;
  const char* knew;
  const char* vnew;
  int64_t tok_stride_b;    // bytes between tokens of the new rows
  int64_t head_stride_b;   // bytes between heads of the new rows
  const int32_t* slots;    // [num_tokens] slot mapping (device)
  int num_tokens;
  int hkv;
  int row_bytes;           // head_dim * element size
  int block_size;
  int64_t block_stride_b;  // bytes between pool blocks
  int64_t layer_off_b;     // bytes from a block's start to the selected layer
  int64_t num_slots;       // num_blocks * block_size
};

struct KvGatherArgs {
  char* kout;
  char* vout;
  const char* kpool;
  const char* vpool;
  const int32_t* table;    // device block table of the sequence
  int seq_len;
  int hkv;
  int row_bytes;
  int block_size;
  int64_t block_stride_b;
  int64_t layer_off_b;
  int num_blocks;
};

int launch_kv_append(const KvAppendArgs& a, hipStream_t stream);
int launch_kv_gather(const KvGatherArgs& a, hipStream_t stream);

}  // namespace sp
