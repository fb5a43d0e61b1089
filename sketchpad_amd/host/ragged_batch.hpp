// Ragged batches over the paged cache: the metadata one iteration's kernels take, built from the
// per-sequence block tables, and one layer of batched attention through the C ABI.
//
// The reference runs attention one sequence at a time (PagedAttentionCache is batch 1,
// paged_attention.rs:485-558; Llama::generate drives batch 1, crates/sketchpad-llm/src/llama.rs:
// 316-364) while its schedulers decide which sequences run (ContinuousBatchingScheduler::schedule,
// continuous_batching.rs:218-316) and own their blocks (PagedScheduler, paged_attention.rs:
// 419-478). This layer turns one iteration of those decisions into a single ragged batch:
//   - every sequence contributes its new tokens (a prompt chunk or one decode token) at positions
//     seq_len .. seq_len + n - 1 of its block table, grown first exactly as
//     PagedSequence::allocate_for_tokens does (paged_attention.rs:398-415);
//   - slot_mapping[t] = table[pos / BS] * BS + pos % BS (BlockTable::get_block / get_slot,
//     paged_attention.rs:124-132), positions[t] = pos, cu_seqlens_q, context_lens (old + new
//     tokens: what each query attends), and the padded block tables;
//   - the batch is ordered chunks first (entries adding two or more tokens), then the entries
//     adding one token, each group in the caller's order, so that both groups are contiguous in
//     the packed token stream and in the per-sequence arrays;
//   - one layer appends K/V for every token (rotating K and Q when RoPE tables are given), then
//     runs chunked prefill over the chunk group and decode over the one-token group, the
//     decode on the library's side stream joined back into the cache's stream so the two
//     overlap. Both reduce to the reference's per-sequence forward_cached
//     (transformer.rs:184-254): no mask for one new token (llama.rs:255-260), and
//     prefill_causal_mask (llama.rs:374-388) for a chunk.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "paged_attention.hpp"

namespace sketchpad {

// One sequence's share of an iteration: num_new tokens after its current length.
struct BatchEntry {
  size_t seq_id;
  size_t num_new;
};

// Host form of a ragged batch's metadata (int32, as the C ABI takes it). Sequences
// [0, num_prefill_seqs) are the chunks (two or more new tokens each) and own tokens
// [0, num_prefill_tokens); the rest add one token each.
struct RaggedBatch {
  std::vector<size_t> seq_ids;        // batch order: chunks, then one-token entries
  std::vector<int32_t> cu_seqlens_q;  // [B + 1] token offsets of each sequence's new tokens
  std::vector<int32_t> positions;     // [T] position of each new token in its sequence
  std::vector<int32_t> slot_mapping;  // [T] pool slot of that position
  std::vector<int32_t> context_lens;  // [B] tokens each sequence attends after the step
  std::vector<int32_t> block_tables;  // [B, max_blocks], rows padded with 0
  int32_t max_blocks = 0;
  int32_t max_seqlen_q = 0;
  int32_t max_context_len = 0;
  int32_t num_prefill_seqs = 0;
  int32_t num_prefill_tokens = 0;
  int32_t prefill_max_seqlen_q = 0;     // over the chunks
  int32_t decode_max_context_len = 0;   // over the one-token entries

  size_t num_seqs() const { return seq_ids.size(); }
  size_t num_tokens() const { return positions.size(); }
  size_t num_decode_seqs() const { return num_seqs() - (size_t)num_prefill_seqs; }
  // every sequence adds exactly one token
  bool decode_only() const { return num_prefill_seqs == 0 && num_tokens() == num_seqs(); }
};

// Grows each entry's block table for its new tokens and reads the metadata off the tables.
// Errors as the reference: "Invalid sequence ID", "Out of memory: no free blocks" (blocks taken
// before the failure stay taken, as in allocate_for_tokens). An entry with no new tokens, or a
// sequence listed twice, is rejected before anything is allocated ("Empty batch entry",
// "Duplicate sequence ID").
Result<RaggedBatch> build_ragged_batch(PagedScheduler& sched,
                                       const std::vector<BatchEntry>& entries);

// After the iteration ran: advance each sequence by its new tokens (increment_seq_len).
void commit_ragged_batch(PagedScheduler& sched, const RaggedBatch& batch);

// Device copy of a RaggedBatch's int32 arrays, uploaded on a stream.
class DeviceRaggedBatch {
 public:
  DeviceRaggedBatch(const RaggedBatch& b, hipStream_t stream);
  const RaggedBatch& host() const { return host_; }
  const int32_t* cu_seqlens_q() const { return base() + off_cu_; }
  const int32_t* positions() const { return base() + off_pos_; }
  const int32_t* slot_mapping() const { return base() + off_slots_; }
  const int32_t* context_lens() const { return base() + off_ctx_; }
  const int32_t* block_tables() const { return base() + off_tables_; }

 private:
  const int32_t* base() const { return (const int32_t*)buf_.data(); }
  RaggedBatch host_;
  DeviceTensor buf_;
  size_t off_cu_ = 0, off_pos_ = 0, off_slots_ = 0, off_ctx_ = 0, off_tables_ = 0;
};

// Device RoPE tables (sp_rope_tables copied to the device): cos / sin [rows, head_dim / 2].
struct RopeTables {
  DeviceTensor cos;
  DeviceTensor sin;
  static RopeTables build(size_t rows, size_t head_dim, float base = 10000.0f);
};

// One attention layer of a ragged batch over a paged cache (the batched form of
// PagedAttentionCache::update_layer + forward_cached). q and out are [T, Hq, D], k_new / v_new
// [T, Hkv, D], packed in batch order. Keeps one workspace between calls for the decode partials
// and the chunked prefill's split-key partials, side by side (grown to what
// sp_ragged_attention_workspace_size asks for). Failures throw std::runtime_error with the
// library's message.
class BatchedPagedAttention {
 public:
  explicit BatchedPagedAttention(PagedKvCache& cache) : cache_(cache) {}
  void forward(size_t layer_idx, const DeviceRaggedBatch& batch, DeviceTensor& q,
               const DeviceTensor& k_new, const DeviceTensor& v_new, DeviceTensor& out,
               float scale, const RopeTables* rope = nullptr);

 private:
  PagedKvCache& cache_;
  DeviceTensor workspace_;
};

// One iteration through every layer: the batched form of the layer loop of Llama::forward
// with a cache (llama.rs:247-271), where start_pos = cache.seq_len() is read once and every layer
// attends with it. Builds the ragged batch once (growing the block tables), uploads it on
// `stream`, calls layer_fn(layer, device_batch) for layer = 0 .. num_layers - 1 (the caller
// computes that layer's q / k / v and runs BatchedPagedAttention::forward on it), and only then
// advances every sequence by its new tokens. So all layers append at the same positions and
// attend the same context lengths (layer-0 semantics for every layer; the reference's
// PagedAttentionCache advances the length inside layer 0, paged_attention.rs:525-533). Returns
// the host batch, or the builder's error with nothing advanced.
template <typename LayerFn>
Result<RaggedBatch> run_batched_step(PagedScheduler& sched, const std::vector<BatchEntry>& entries,
                                     size_t num_layers, hipStream_t stream, LayerFn&& layer_fn) {
  Result<RaggedBatch> r = build_ragged_batch(sched, entries);
  if (r.is_err()) return r;
  const DeviceRaggedBatch db(r.unwrap(), stream);
  for (size_t layer = 0; layer < num_layers; ++layer) layer_fn(layer, db);
  commit_ragged_batch(sched, r.unwrap());
  return r;
}

}  // namespace sketchpad
