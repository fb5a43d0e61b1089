// Launch interface of the split-K paged decode kernel (paged_decode.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

constexpr int kDecodeWaves = 4;      // waves per workgroup
constexpr int kDecodeMaxGroup = 16;  // largest GQA group (Hq / Hkv): the MFMA N extent

struct DecodePlan {
  int group;            // Hq / Hkv
  int tt;               // tokens per tile
  int tps;              // tiles per split (one workgroup)
  int max_tiles;        // tiles a sequence can span
  int max_splits;       // splits a sequence can span
  size_t ws_bytes;      // fp32 partials [num_seqs][Hq][max_splits][D + 4]
};

enum class DecodeKind { Dense, Polar };

// The split plan of a decode call, a function of the batch shape only: tiles per split (at most
// 128, the block ids one workgroup prefetches), the splits a sequence can span and the
// partials' bytes. Dense and PolarQuant pools have rules of their own.
DecodePlan plan_decode(int num_seqs, int hq, int hkv, int head_dim, int max_context_len,
                       int window_left, DecodeKind kind);

struct DecodeArgs {
  void* out;
  const void* q;
  const char* kpool;
  const char* vpool;
  const int32_t* block_tables;
  const int32_t* context_lens;
  float* partials;
  int64_t block_stride_b;
  int64_t layer_off_b;
  int max_blocks_per_seq;
  int max_context_len;
  int num_blocks;
  int block_size;
  int num_seqs;
  int hq;
  int hkv;
  int group;
  int window_left;
  int tps;
  int max_splits;
  float scale_log2;  // softmax scale * log2(e)
  // Logit soft cap (head_dims 256 and 512 only): cap_out > 0 turns each raw product s into the
  // exponent softcap_log2(s, cap_in, cap_out) = cap log2(e) tanh(s scale / cap) instead of
  // s * scale_log2; 0: none.
  float cap_in, cap_out;
  // Fused append (sp_paged_append_decode), or null: the step's new token of sequence s, for KV
  // head h, at k_new + s * new_tok_stride_b + h * new_head_stride_b (same for v_new).
  const char* k_new;
  const char* v_new;
  int64_t new_tok_stride_b;
  int64_t new_head_stride_b;
};

int launch_paged_decode(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream);

// Library-owned scratch for the decode partials of sp_paged_decode_noalloc: a file-scope device
// array of kDecodeScratchBytes per GPU, held until the process ends. Returns its device address
// on the current device (looked up once per device with hipGetSymbolAddress), or nullptr with
// the error recorded.
constexpr size_t kDecodeScratchBytes = (size_t)32 << 20;
void* decode_scratch_on_current_device();

// The split merge alone (no-op when a.max_splits <= 1): for kernels that write the same
// (m, l, acc[D]) partials in 16-token tiles.
int launch_decode_combine(const DecodeArgs& a, sp_dtype dtype, int head_dim, hipStream_t stream);

}  // namespace sp
