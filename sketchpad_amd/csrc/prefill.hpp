// Launch interface of the causal / windowed prefill kernels (prefill.hip).
#pragma once

#include "sp_common.hpp"

namespace sp {

constexpr int kPrefillBM = 128;  // queries per workgroup (four waves x 32)
constexpr int kPrefillBN = 64;   // keys per step

struct PrefillArgs {
  void* out;
  const void* q;
  const void* k;  // packed / dense K (unused when paged)
  const void* v;
  // element strides
  int64_t q_tok, q_head, q_batch;
  int64_t o_tok, o_head, o_batch;
  int64_t kv_tok, kv_head, kv_batch;  // K (and V unless v_* differ)
  int64_t v_tok, v_head, v_batch;     // V element strides
  int dv;                             // value head dim (== head_dim except dense f32)
  int out_dtype;                      // sp_dtype of out
  const int32_t* cu_q;  // [num_seqs + 1] token offsets, or nullptr for dense batches
  const int32_t* cu_k;  // [num_seqs + 1] key offsets (packed K/V), or nullptr
  int lq, lk;           // dense lengths (cu_q / cu_k == nullptr)
  int num_seqs;
  int hq, hkv, group;
  int num_qblocks;      // ceil(max_seqlen_q / kPrefillBM)
  int causal;           // sp_causal
  int window_left;      // -1: none
  float scale_log2;     // softmax scale * log2(e)
  // paged K/V source
  const char* kpool;
  const char* vpool;
  const int32_t* block_tables;
  const int32_t* context_lens;
  int max_blocks_per_seq;
  int block_size;
  int num_blocks;
  int64_t block_stride_b;
  int64_t layer_off_b;
  // split key range (paged prefill with a workspace): nsplit > 1 makes every workgroup take
  // 1/nsplit of its sequence's key tiles and write fp32 partials [num_seqs][max_q][Hq][nsplit]
  // records of (m, l, pad, pad, acc[D]) that prefill_combine_kernel merges into out.
  float* partials;
  int nsplit;
  int max_q;  // max_seqlen_q: the partials' per-sequence row stride
  // additive mask of the dense f32 path (flash_attention_masked): mask[b][h][i][j] at element
  // offset b mask_b + h mask_h + i mask_q + j, added to score * scale; nullptr: none
  const float* mask;
  int64_t mask_b, mask_h, mask_q;
  float inv_scale;  // 1 / scale (log2(e) with the soft cap: the mask then adds to the exponent)
  // Logit soft cap (head_dims 256 and 512 only): cap_out > 0 turns each raw product s into the
  // exponent softcap_log2(s, cap_in, cap_out) = cap log2(e) tanh(s scale / cap) instead of
  // s * scale_log2; 0: none.
  float cap_in, cap_out;
};

// Split count for a chunked prefill of base_wgs workgroups whose sequences span up to
// max_ctx_tiles 64-key tiles: as many splits as keep the whole grid within one round of
// resident workgroups (2 per CU on 256 CUs), at least 16 tiles per split, at most 8 splits.
int plan_prefill_splits(int64_t base_wgs, int64_t max_ctx_tiles);
size_t prefill_partials_bytes(int num_seqs, int max_seqlen_q, int hq, int head_dim, int nsplit);

int launch_prefill(const PrefillArgs& a, sp_dtype dtype, int head_dim, bool paged,
                   hipStream_t stream);
// fp32 tensors (prefill_f32.hip); called by launch_prefill for SP_F32.
int launch_prefill_f32(const PrefillArgs& a, int head_dim, bool paged, hipStream_t stream);
// Head dims the fp32 kernel covers: dense K/V any of 40, 64, 80, 128, 160, 256 with a value head
// dim <= 256 (a multiple of 4); paged / packed K/V 64 or 128 with equal value head dim.
bool prefill_f32_supports(int head_dim, int v_head_dim, bool paged);

}  // namespace sp
