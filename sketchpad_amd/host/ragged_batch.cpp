// Ragged batches over the paged cache: see ragged_batch.hpp.
#include "ragged_batch.hpp"

#include <algorithm>

namespace sketchpad {

namespace {

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void check_sp(int rc, const char* what) {
  if (rc != SP_OK) throw std::runtime_error(std::string(what) + ": " + sp_last_error());
}

}  // namespace

Result<RaggedBatch> build_ragged_batch(PagedScheduler& sched,
                                       const std::vector<BatchEntry>& entries) {
  RaggedBatch b;
  const size_t bs = sched.cache.block_size();
  {
    std::vector<size_t> ids;
    for (const BatchEntry& e : entries) {
      if (e.num_new == 0) return Result<RaggedBatch>::Err("Empty batch entry");
      ids.push_back(e.seq_id);
    }
    std::sort(ids.begin(), ids.end());
    if (std::adjacent_find(ids.begin(), ids.end()) != ids.end())
      return Result<RaggedBatch>::Err("Duplicate sequence ID");
  }
  // grow every table first (allocate_for_tokens, paged_attention.rs:398-415)
  for (const BatchEntry& e : entries) {
    Result<Unit> r = sched.allocate(e.seq_id, e.num_new);
    if (r.is_err()) return Result<RaggedBatch>::Err(r.error());
  }
  // batch order: chunks first, then one-token entries (stable within each group)
  std::vector<const BatchEntry*> order;
  for (const BatchEntry& e : entries)
    if (e.num_new > 1) order.push_back(&e);
  const size_t num_chunks = order.size();
  for (const BatchEntry& e : entries)
    if (e.num_new == 1) order.push_back(&e);
  size_t max_blocks = 1;
  for (const BatchEntry& e : entries)
    max_blocks = std::max(max_blocks, sched.get_sequence(e.seq_id)->block_table.num_blocks());
  b.max_blocks = (int32_t)max_blocks;
  b.num_prefill_seqs = (int32_t)num_chunks;
  b.cu_seqlens_q.push_back(0);
  for (size_t s = 0; s < order.size(); ++s) {
    const BatchEntry& e = *order[s];
    const BlockTable& table = sched.get_sequence(e.seq_id)->block_table;
    const size_t start = table.seq_len();
    for (size_t i = 0; i < e.num_new; ++i) {
      const size_t pos = start + i;
      // the table covers every new position after the allocation above
      const size_t blk = *table.get_block(pos);
      b.positions.push_back((int32_t)pos);
      b.slot_mapping.push_back((int32_t)(blk * bs + table.get_slot(pos)));
    }
    b.seq_ids.push_back(e.seq_id);
    b.cu_seqlens_q.push_back((int32_t)b.positions.size());
    const int32_t ctx = (int32_t)(start + e.num_new);
    b.context_lens.push_back(ctx);
    b.max_seqlen_q = std::max(b.max_seqlen_q, (int32_t)e.num_new);
    b.max_context_len = std::max(b.max_context_len, ctx);
    if (s < num_chunks) {
      b.num_prefill_tokens = (int32_t)b.positions.size();
      b.prefill_max_seqlen_q = std::max(b.prefill_max_seqlen_q, (int32_t)e.num_new);
    } else {
      b.decode_max_context_len = std::max(b.decode_max_context_len, ctx);
    }
    std::vector<int32_t> row(max_blocks, 0);
    for (size_t j = 0; j < table.num_blocks(); ++j) row[j] = (int32_t)table.blocks()[j];
    b.block_tables.insert(b.block_tables.end(), row.begin(), row.end());
  }
  return Result<RaggedBatch>::Ok(std::move(b));
}

void commit_ragged_batch(PagedScheduler& sched, const RaggedBatch& batch) {
  for (size_t i = 0; i < batch.num_seqs(); ++i) {
    PagedSequence* s = sched.get_sequence_mut(batch.seq_ids[i]);
    s->block_table.increment_seq_len(
        (size_t)(batch.cu_seqlens_q[i + 1] - batch.cu_seqlens_q[i]));
  }
}

DeviceRaggedBatch::DeviceRaggedBatch(const RaggedBatch& b, hipStream_t stream) : host_(b) {
  std::vector<int32_t> all;
  auto put = [&](const std::vector<int32_t>& v) {
    const size_t off = all.size();
    all.insert(all.end(), v.begin(), v.end());
    all.resize((all.size() + 63) / 64 * 64);  // 256-byte aligned sections
    return off;
  };
  off_cu_ = put(b.cu_seqlens_q);
  off_pos_ = put(b.positions);
  off_slots_ = put(b.slot_mapping);
  off_ctx_ = put(b.context_lens);
  off_tables_ = put(b.block_tables);
  buf_ = DeviceTensor({(int64_t)all.size()}, SP_F32);
  check_hip(hipMemcpyAsync(buf_.data(), all.data(), all.size() * 4, hipMemcpyHostToDevice,
                           stream),
            "DeviceRaggedBatch upload");
  check_hip(hipStreamSynchronize(stream), "DeviceRaggedBatch upload");  // `all` is local
}

RopeTables RopeTables::build(size_t rows, size_t head_dim, float base) {
  std::vector<float> c(rows * (head_dim / 2)), s(c.size());
  check_sp(sp_rope_tables(c.data(), s.data(), (int32_t)rows, (int32_t)head_dim, base),
           "sp_rope_tables");
  RopeTables t;
  t.cos = DeviceTensor::from_host(c.data(), {(int64_t)rows, (int64_t)(head_dim / 2)}, SP_F32);
  t.sin = DeviceTensor::from_host(s.data(), {(int64_t)rows, (int64_t)(head_dim / 2)}, SP_F32);
  return t;
}

void BatchedPagedAttention::forward(size_t layer_idx, const DeviceRaggedBatch& batch,
                                    DeviceTensor& q, const DeviceTensor& k_new,
                                    const DeviceTensor& v_new, DeviceTensor& out, float scale,
                                    const RopeTables* rope) {
  const RaggedBatch& hb = batch.host();
  if (hb.num_seqs() == 0) return;
  const PagedKvCacheConfig& cfg = cache_.config();
  const int32_t hkv = (int32_t)cfg.num_kv_heads, d = (int32_t)cfg.head_dim;
  const int32_t T = (int32_t)hb.num_tokens();
  const int32_t hq = (int32_t)(q.numel() / ((int64_t)T * d));
  if ((int64_t)T * hkv * d != k_new.numel() || k_new.numel() != v_new.numel() ||
      out.numel() != q.numel() || q.dtype() != cache_.dtype())
    throw std::runtime_error("BatchedPagedAttention: tensor shapes do not match the batch");
  const sp_cache_layout lay = cache_.layout(layer_idx);
  const hipStream_t stream = cache_.stream();
  void* kp = cache_.k_cache().data();
  void* vp = cache_.v_cache().data();
  // 1. append the iteration's K/V rows (rotating K, and Q in place, when tables are given)
  if (rope) {
    check_sp(sp_rope_kv_append(kp, vp, &lay, k_new.data(), v_new.data(), (int64_t)hkv * d, d,
                               q.data(), (int64_t)hq * d, d, hq, batch.positions(),
                               batch.slot_mapping(), T, (const float*)rope->cos.data(),
                               (const float*)rope->sin.data(), (int32_t)rope->cos.dims()[0],
                               cache_.dtype(), stream),
             "sp_rope_kv_append");
  } else {
    check_sp(sp_kv_append(kp, vp, &lay, k_new.data(), v_new.data(), (int64_t)hkv * d, d,
                          batch.slot_mapping(), T, cache_.dtype(), stream),
             "sp_kv_append");
  }
  // 2. attention: chunked prefill over the chunks [0, P), decode over the one-token entries
  //    [P, B): one sp_ragged_paged_attention call, ordered on the cache's stream
  const int32_t P = hb.num_prefill_seqs, B = (int32_t)hb.num_seqs();
  const size_t need = sp_ragged_attention_workspace_size(B, P, hb.prefill_max_seqlen_q,
                                                         hb.decode_max_context_len, hq, -1,
                                                         &lay, hb.max_blocks);
  if (need > workspace_.nbytes())
    workspace_ = DeviceTensor({(int64_t)((need + 3) / 4)}, SP_F32);  // zero-filled
  check_sp(sp_ragged_paged_attention(out.data(), q.data(), kp, vp, &lay, batch.block_tables(),
                                     hb.max_blocks, batch.cu_seqlens_q(), batch.context_lens(),
                                     B, P, hb.num_prefill_tokens, hb.prefill_max_seqlen_q,
                                     hb.decode_max_context_len, hq, scale, -1, cache_.dtype(),
                                     workspace_.nbytes() ? workspace_.data() : nullptr,
                                     workspace_.nbytes(), stream),
           "sp_ragged_paged_attention");
}

}  // namespace sketchpad
