// C++ mirror of rhi-zone/sketchpad's paged/flash attention API, over the C ABI of
// include/sketchpad_attn.h.
//
// The reference's host side is Rust (Burn tensors). This header keeps its names, argument
// meaning and error behaviour so that code written against
//   crates/sketchpad-core/src/paged_attention.rs   (PagedKvCacheConfig, BlockTable, PagedKvCache,
//                                                   PagedSequence, PagedScheduler,
//                                                   PagedAttentionCache)
//   crates/sketchpad-core/src/kv_cache.rs          (CacheUpdate, AttentionCache, KvCache,
//                                                   ModelKvCache)
//   crates/sketchpad-core/src/attention.rs         (qkv_attention, causal_mask)
//   crates/sketchpad-cubecl/src/attention.rs       (FlashAttentionOptions, flash_attention)
// maps one to one:
//   - Burn `Tensor<B, N>` (a ref-counted device handle) -> DeviceTensor (shared device buffer +
//     shape + dtype; copying a DeviceTensor is O(1) like Tensor::clone).
//   - a Rust panic (`expect`, index out of range)  -> std::runtime_error with the same message.
//   - `Result<T, &'static str>`                     -> Result<T> (value or error message).
//   - `Option<usize>`                               -> std::optional<size_t>.
// Device work is enqueued on the stream given at construction (default stream when null) and
// goes through the library's kernels only; there is no CPU fallback.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <deque>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sketchpad_attn.h"

namespace sketchpad {

// ---------------------------------------------------------------------------------------------
// Result<T>: the reference's Result<T, &'static str>.
// ---------------------------------------------------------------------------------------------
template <typename T>
class Result {
 public:
  static Result Ok(T v) { return Result(std::move(v), nullptr); }
  static Result Err(const char* e) { return Result(std::nullopt, e); }
  bool is_ok() const { return error_ == nullptr; }
  bool is_err() const { return error_ != nullptr; }
  const T& unwrap() const {
    if (error_) throw std::runtime_error(std::string("called `Result::unwrap()` on an `Err` value: ") + error_);
    return *value_;
  }
  const char* error() const { return error_; }

 private:
  Result(std::optional<T> v, const char* e) : value_(std::move(v)), error_(e) {}
  std::optional<T> value_;
  const char* error_;
};

struct Unit {};

// ---------------------------------------------------------------------------------------------
// DeviceTensor: a shared device buffer with a shape and an element type.
// ---------------------------------------------------------------------------------------------
class DeviceTensor {
 public:
  DeviceTensor() = default;
  // Zero-filled allocation (Tensor::zeros).
  DeviceTensor(std::vector<int64_t> shape, sp_dtype dtype);
  // Copy of host data of this shape / dtype (Tensor::from_data).
  static DeviceTensor from_host(const void* data, std::vector<int64_t> shape, sp_dtype dtype);

  void to_host(void* out) const;  // synchronous copy of the whole tensor
  void* data() const { return buf_.get(); }
  const std::vector<int64_t>& dims() const { return shape_; }
  sp_dtype dtype() const { return dtype_; }
  int64_t numel() const;
  size_t nbytes() const;
  // Same buffer, new shape of the same element count (Tensor::reshape on a contiguous tensor).
  DeviceTensor reshape(std::vector<int64_t> shape) const;

 private:
  std::shared_ptr<void> buf_;
  std::vector<int64_t> shape_;
  sp_dtype dtype_ = SP_F32;
};

size_t dtype_bytes(sp_dtype dtype);

// ---------------------------------------------------------------------------------------------
// paged_attention.rs
// ---------------------------------------------------------------------------------------------

// PagedKvCacheConfig (paged_attention.rs:35-86).
struct PagedKvCacheConfig {
  size_t block_size = 0;
  size_t num_blocks = 0;
  size_t num_kv_heads = 0;
  size_t head_dim = 0;
  size_t num_layers = 0;

  PagedKvCacheConfig() = default;
  // PagedKvCacheConfig::new (paged_attention.rs:50-64)
  PagedKvCacheConfig(size_t block_size, size_t num_blocks, size_t num_kv_heads, size_t head_dim,
                     size_t num_layers)
      : block_size(block_size), num_blocks(num_blocks), num_kv_heads(num_kv_heads),
        head_dim(head_dim), num_layers(num_layers) {}
  // from_memory_budget (paged_attention.rs:67-85): bytes per block assume 4-byte elements, as
  // the reference does.
  static PagedKvCacheConfig from_memory_budget(size_t memory_bytes, size_t num_kv_heads,
                                               size_t head_dim, size_t num_layers,
                                               size_t block_size);
};

// BlockTable (paged_attention.rs:89-148).
class BlockTable {
 public:
  explicit BlockTable(size_t block_size) : block_size_(block_size) {}
  size_t num_blocks() const { return block_indices_.size(); }
  size_t seq_len() const { return seq_len_; }
  void add_block(size_t block_idx) { block_indices_.push_back(block_idx); }
  std::optional<size_t> get_block(size_t pos) const {
    const size_t n = pos / block_size_;
    if (n < block_indices_.size()) return block_indices_[n];
    return std::nullopt;
  }
  size_t get_slot(size_t pos) const { return pos % block_size_; }
  bool needs_new_block() const { return seq_len_ > 0 && seq_len_ % block_size_ == 0; }
  void increment_seq_len(size_t count) { seq_len_ += count; }
  const std::vector<size_t>& blocks() const { return block_indices_; }
  size_t block_size() const { return block_size_; }

 private:
  std::vector<size_t> block_indices_;
  size_t seq_len_ = 0;
  size_t block_size_;
};

// PagedKvCache (paged_attention.rs:151-379): K and V pools of
// [num_blocks, num_layers, num_kv_heads, block_size, head_dim], zero-initialised, and a FIFO
// free list over 0..num_blocks. `dtype` is the element type of the pools (the reference is
// generic over the backend; NdArray<f32> is its CPU default).
class PagedKvCache {
 public:
  PagedKvCache(const PagedKvCacheConfig& config, sp_dtype dtype = SP_F32,
               hipStream_t stream = nullptr);

  std::optional<size_t> allocate_block();
  void free_block(size_t block_idx);
  void free_sequence(const BlockTable& block_table);
  size_t num_free_blocks() const { return free_blocks_.size(); }
  size_t num_blocks() const { return config_.num_blocks; }
  size_t block_size() const { return config_.block_size; }

  // store_kv (paged_attention.rs:230-265): k, v are [num_kv_heads, seq_len, head_dim]; token i
  // goes to position start_pos + i. Throws "Block not allocated" (the reference's panic) before
  // any device work when a position has no block.
  void store_kv(size_t layer_idx, const BlockTable& block_table, const DeviceTensor& k,
                const DeviceTensor& v, size_t start_pos);
  // gather_kv (paged_attention.rs:313-378): [num_kv_heads, seq_len, head_dim] copies of the
  // sequence's rows; seq_len == 0 gives [num_kv_heads, 0, head_dim].
  std::pair<DeviceTensor, DeviceTensor> gather_kv(size_t layer_idx,
                                                  const BlockTable& block_table) const;

  const PagedKvCacheConfig& config() const { return config_; }
  const DeviceTensor& k_cache() const { return k_cache_; }
  const DeviceTensor& v_cache() const { return v_cache_; }
  sp_dtype dtype() const { return dtype_; }
  hipStream_t stream() const { return stream_; }
  sp_cache_layout layout(size_t layer_idx) const;

 private:
  PagedKvCacheConfig config_;
  sp_dtype dtype_;
  hipStream_t stream_;
  DeviceTensor k_cache_, v_cache_;
  std::deque<size_t> free_blocks_;
};

// PagedSequence (paged_attention.rs:382-416).
struct PagedSequence {
  BlockTable block_table;
  bool finished = false;
  explicit PagedSequence(size_t block_size) : block_table(block_size) {}
  // "Out of memory: no free blocks" when the pool runs dry (blocks taken so far stay taken).
  Result<Unit> allocate_for_tokens(size_t num_tokens, PagedKvCache& cache);
};

// PagedScheduler (paged_attention.rs:419-478).
class PagedScheduler {
 public:
  PagedScheduler(const PagedKvCacheConfig& config, sp_dtype dtype = SP_F32,
                 hipStream_t stream = nullptr)
      : cache(config, dtype, stream) {}
  Result<size_t> add_sequence();
  const PagedSequence* get_sequence(size_t seq_id) const;
  PagedSequence* get_sequence_mut(size_t seq_id);
  Result<Unit> allocate(size_t seq_id, size_t num_tokens);  // "Invalid sequence ID"
  // Returns the sequence's blocks to the pool (the table itself is left as is, as in the
  // reference).
  void free_sequence(size_t seq_id);
  size_t num_sequences() const { return sequences_.size(); }
  size_t available_tokens() const { return cache.num_free_blocks() * cache.block_size(); }

  PagedKvCache cache;

 private:
  std::vector<PagedSequence> sequences_;
};

// ---------------------------------------------------------------------------------------------
// kv_cache.rs: the cache trait and the default concat cache
// ---------------------------------------------------------------------------------------------

// CacheUpdate (kv_cache.rs:14-19): full K/V [batch, num_kv_heads, total_seq_len, head_dim].
struct CacheUpdate {
  DeviceTensor k;
  DeviceTensor v;
};

// AttentionCache (kv_cache.rs:25-45).
class AttentionCache {
 public:
  virtual ~AttentionCache() = default;
  // k, v: new keys / values [batch, num_kv_heads, new_seq_len, head_dim].
  virtual CacheUpdate update_layer(size_t layer_idx, const DeviceTensor& k,
                                   const DeviceTensor& v) = 0;
  virtual size_t seq_len() const = 0;
  virtual void clear() = 0;
};

// KvCache (kv_cache.rs:70-150): one layer, concatenation along the sequence dimension.
class KvCache {
 public:
  explicit KvCache(size_t max_seq_len, hipStream_t stream = nullptr)
      : max_seq_len_(max_seq_len), stream_(stream) {}
  std::pair<DeviceTensor, DeviceTensor> update(const DeviceTensor& k, const DeviceTensor& v);
  size_t seq_len() const { return current_pos_; }
  void clear() {
    k_.reset();
    v_.reset();
    current_pos_ = 0;
  }
  bool is_empty() const { return !k_.has_value(); }
  size_t max_seq_len() const { return max_seq_len_; }

 private:
  std::optional<DeviceTensor> k_, v_;
  size_t current_pos_ = 0;
  size_t max_seq_len_;
  hipStream_t stream_;
};

// ModelKvCache (kv_cache.rs:154-193) + its AttentionCache impl (kv_cache.rs:47-65).
class ModelKvCache : public AttentionCache {
 public:
  ModelKvCache(size_t num_layers, size_t max_seq_len, hipStream_t stream = nullptr);
  KvCache& layer(size_t idx) { return layers.at(idx); }
  CacheUpdate update_layer(size_t layer_idx, const DeviceTensor& k,
                           const DeviceTensor& v) override;
  size_t seq_len() const override { return layers.empty() ? 0 : layers.front().seq_len(); }
  void clear() override {
    for (auto& l : layers) l.clear();
  }

  std::vector<KvCache> layers;
  size_t max_seq_len;
};

// PagedAttentionCache (paged_attention.rs:485-558): a single sequence (batch 1) over a paged
// pool. Layer 0 grows the block table; every layer stores the new rows at the positions layer 0
// assigned (the reference's layers >= 1 read an already advanced start position,
// paged_attention.rs:525-543; that is not reproduced) and gathers the full sequence.
class PagedAttentionCache : public AttentionCache {
 public:
  PagedAttentionCache(const PagedKvCacheConfig& config, sp_dtype dtype = SP_F32,
                      hipStream_t stream = nullptr)
      : cache_(config, dtype, stream), block_table_(config.block_size) {}
  CacheUpdate update_layer(size_t layer_idx, const DeviceTensor& k,
                           const DeviceTensor& v) override;
  size_t seq_len() const override { return block_table_.seq_len(); }
  void clear() override;
  const PagedKvCache& cache() const { return cache_; }
  const BlockTable& block_table() const { return block_table_; }

 private:
  void ensure_capacity(size_t additional_tokens);
  PagedKvCache cache_;
  BlockTable block_table_;
};

// ---------------------------------------------------------------------------------------------
// attention.rs / sketchpad-cubecl attention.rs
// ---------------------------------------------------------------------------------------------

// causal_mask (attention.rs:33-42): host copy of the [seq_len, seq_len] additive mask.
std::vector<float> causal_mask(size_t seq_len);
// causal_mask as the reference returns it: an f32 device tensor [seq_len, seq_len].
DeviceTensor causal_mask_tensor(size_t seq_len);

// qkv_attention (attention.rs:4-27): softmax((q d^-1/4)(k d^-1/4)^T + mask) v on
// [batch, heads, seq, head_dim] tensors, i.e. scale d^-1/2 on the product; mask is the
// reference's Option<Tensor<B, 2>>: an additive f32 [seq_q, seq_k] tensor added to every batch
// and head (std::nullopt: none). Throws on shapes or dtypes the kernels do not cover.
DeviceTensor qkv_attention(const DeviceTensor& q, const DeviceTensor& k, const DeviceTensor& v,
                           const std::optional<DeviceTensor>& mask, hipStream_t stream = nullptr);

// FlashAttentionOptions (sketchpad-cubecl attention.rs:39-69).
struct FlashAttentionOptions {
  std::optional<sp_dtype> out_dtype;
  bool causal = false;
  static FlashAttentionOptions causal_() {
    FlashAttentionOptions o;
    o.causal = true;
    return o;
  }
  FlashAttentionOptions with_dtype(sp_dtype dt) const {
    FlashAttentionOptions o = *this;
    o.out_dtype = dt;
    return o;
  }
  FlashAttentionOptions with_causal(bool c) const {
    FlashAttentionOptions o = *this;
    o.causal = c;
    return o;
  }
};

// AttentionSetupError: why a flash-attention launch could not be set up.
struct AttentionSetupError {
  std::string message;
};

// flash_attention (sketchpad-cubecl attention.rs:97-104): q, k [batch, heads, seq, head_dim],
// v [batch, heads, seq_k, val_dim] -> out [batch, heads, seq_q, val_dim] of options.out_dtype
// (q's dtype when unset); causal masks key j > query i. Errors (instead of launching) on shapes
// or dtypes the kernels do not cover.
struct FlashResult {
  std::optional<DeviceTensor> out;
  std::optional<AttentionSetupError> error;
  bool is_ok() const { return out.has_value(); }
};
FlashResult flash_attention(const DeviceTensor& query, const DeviceTensor& key,
                            const DeviceTensor& value, const FlashAttentionOptions& options,
                            hipStream_t stream = nullptr);

// flash_attention_masked (sketchpad-cubecl attention.rs:119-128): additive f32 mask,
// [B, H, Sq, Sk] or one [Sq, Sk] mask for every batch and head (the reference's tests expand
// one [Sq, Sk] mask).
FlashResult flash_attention_masked(const DeviceTensor& query, const DeviceTensor& key,
                                   const DeviceTensor& value, const DeviceTensor& mask,
                                   const FlashAttentionOptions& options,
                                   hipStream_t stream = nullptr);

}  // namespace sketchpad
