// C++ mirror of rhi-zone/sketchpad's paged/flash attention API over the C ABI (see
// paged_attention.hpp for the mapping of Rust types and errors). Every device operation goes
// through an sp_* entry point of libsketchpad_attn.so, or a HIP runtime copy for the
// concatenating KvCache.
#include "paged_attention.hpp"

#include <optional>

#include <math.h>

#include <numeric>

namespace sketchpad {

namespace {

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void check_sp(int rc, const char* what) {
  if (rc != SP_OK) throw std::runtime_error(std::string(what) + ": " + sp_last_error());
}

// Growable device scratch for small host-built metadata (slot mappings, block tables). The copy
// is synchronous with respect to the host buffer, ordered on `stream` for the device.
class DeviceInts {
 public:
  const int32_t* upload(const std::vector<int32_t>& v, hipStream_t stream) {
    if (v.empty()) return nullptr;
    if (v.size() > cap_) {
      buf_ = DeviceTensor({(int64_t)v.size()}, SP_F32);
      cap_ = v.size();
    }
    check_hip(hipMemcpyAsync(buf_.data(), v.data(), v.size() * 4, hipMemcpyHostToDevice, stream),
              "upload");
    check_hip(hipStreamSynchronize(stream), "upload");
    return (const int32_t*)buf_.data();
  }

 private:
  DeviceTensor buf_;
  size_t cap_ = 0;
};

thread_local DeviceInts g_ints;

}  // namespace

// ---------------------------------------------------------------------------------------------
// DeviceTensor
// ---------------------------------------------------------------------------------------------

size_t dtype_bytes(sp_dtype dtype) { return dtype == SP_F32 ? 4 : 2; }

DeviceTensor::DeviceTensor(std::vector<int64_t> shape, sp_dtype dtype)
    : shape_(std::move(shape)), dtype_(dtype) {
  const size_t n = nbytes();
  if (n == 0) return;
  void* p = nullptr;
  check_hip(hipMalloc(&p, n), "hipMalloc");
  buf_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
  check_hip(hipMemset(p, 0, n), "hipMemset");
}

DeviceTensor DeviceTensor::from_host(const void* data, std::vector<int64_t> shape,
                                     sp_dtype dtype) {
  DeviceTensor t(std::move(shape), dtype);
  if (t.nbytes())
    check_hip(hipMemcpy(t.data(), data, t.nbytes(), hipMemcpyHostToDevice), "from_host");
  return t;
}

void DeviceTensor::to_host(void* out) const {
  if (nbytes()) check_hip(hipMemcpy(out, data(), nbytes(), hipMemcpyDeviceToHost), "to_host");
}

int64_t DeviceTensor::numel() const {
  return std::accumulate(shape_.begin(), shape_.end(), (int64_t)1, std::multiplies<int64_t>());
}

size_t DeviceTensor::nbytes() const { return (size_t)numel() * dtype_bytes(dtype_); }

DeviceTensor DeviceTensor::reshape(std::vector<int64_t> shape) const {
  DeviceTensor t = *this;
  t.shape_ = std::move(shape);
  if (t.numel() != numel()) throw std::runtime_error("reshape: element count differs");
  return t;
}

// ---------------------------------------------------------------------------------------------
// PagedKvCacheConfig / PagedKvCache
// ---------------------------------------------------------------------------------------------

PagedKvCacheConfig PagedKvCacheConfig::from_memory_budget(size_t memory_bytes,
                                                          size_t num_kv_heads, size_t head_dim,
                                                          size_t num_layers, size_t block_size) {
  const size_t bytes_per_block = 2 * num_layers * num_kv_heads * head_dim * block_size * 4;
  return PagedKvCacheConfig(block_size, memory_bytes / bytes_per_block, num_kv_heads, head_dim,
                            num_layers);
}

PagedKvCache::PagedKvCache(const PagedKvCacheConfig& config, sp_dtype dtype, hipStream_t stream)
    : config_(config), dtype_(dtype), stream_(stream) {
  const std::vector<int64_t> shape = {(int64_t)config.num_blocks, (int64_t)config.num_layers,
                                      (int64_t)config.num_kv_heads, (int64_t)config.block_size,
                                      (int64_t)config.head_dim};
  k_cache_ = DeviceTensor(shape, dtype);
  v_cache_ = DeviceTensor(shape, dtype);
  for (size_t i = 0; i < config.num_blocks; ++i) free_blocks_.push_back(i);
}

std::optional<size_t> PagedKvCache::allocate_block() {
  if (free_blocks_.empty()) return std::nullopt;
  const size_t b = free_blocks_.front();
  free_blocks_.pop_front();
  return b;
}

void PagedKvCache::free_block(size_t block_idx) { free_blocks_.push_back(block_idx); }

void PagedKvCache::free_sequence(const BlockTable& block_table) {
  for (size_t b : block_table.blocks()) free_block(b);
}

sp_cache_layout PagedKvCache::layout(size_t layer_idx) const {
  sp_cache_layout l;
  l.num_blocks = (int32_t)config_.num_blocks;
  l.num_layers = (int32_t)config_.num_layers;
  l.layer = (int32_t)layer_idx;
  l.num_kv_heads = (int32_t)config_.num_kv_heads;
  l.block_size = (int32_t)config_.block_size;
  l.head_dim = (int32_t)config_.head_dim;
  return l;
}

void PagedKvCache::store_kv(size_t layer_idx, const BlockTable& block_table,
                            const DeviceTensor& k, const DeviceTensor& v, size_t start_pos) {
  const auto& d = k.dims();
  if (d.size() != 3 || (size_t)d[0] != config_.num_kv_heads || (size_t)d[2] != config_.head_dim ||
      v.dims() != d)
    throw std::runtime_error("store_kv: k and v must be [num_kv_heads, seq_len, head_dim]");
  if (k.dtype() != dtype_ || v.dtype() != dtype_)
    throw std::runtime_error("store_kv: k / v dtype differs from the cache's");
  const size_t seq_len = (size_t)d[1];
  std::vector<int32_t> slots(seq_len);
  for (size_t i = 0; i < seq_len; ++i) {
    const size_t pos = start_pos + i;
    const auto blk = block_table.get_block(pos);
    if (!blk) throw std::runtime_error("Block not allocated");
    slots[i] = (int32_t)(*blk * config_.block_size + block_table.get_slot(pos));
  }
  if (seq_len == 0) return;
  const sp_cache_layout lay = layout(layer_idx);
  const int32_t* dslots = g_ints.upload(slots, stream_);
  // head-major input: element (t, h, e) at h * seq_len * D + t * D + e
  check_sp(sp_kv_append(k_cache_.data(), v_cache_.data(), &lay, k.data(), v.data(),
                        (int64_t)config_.head_dim, (int64_t)(seq_len * config_.head_dim), dslots,
                        (int32_t)seq_len, dtype_, stream_),
           "store_kv");
  check_hip(hipStreamSynchronize(stream_), "store_kv");  // the slot buffer is reused
}

std::pair<DeviceTensor, DeviceTensor> PagedKvCache::gather_kv(
    size_t layer_idx, const BlockTable& block_table) const {
  const size_t seq_len = block_table.seq_len();
  const int64_t H = (int64_t)config_.num_kv_heads, D = (int64_t)config_.head_dim;
  if (seq_len == 0) return {DeviceTensor({H, 0, D}, dtype_), DeviceTensor({H, 0, D}, dtype_)};
  // The reference concatenates min(block_size, seq_len - start) rows of every block in the
  // table: rows past the table's end are simply absent, and a block that starts past seq_len
  // underflows the usize subtraction (a panic).
  size_t rows = 0;
  for (size_t b = 0; b < block_table.num_blocks(); ++b) {
    const size_t start = b * config_.block_size;
    if (start > seq_len) throw std::runtime_error("attempt to subtract with overflow");
    rows += std::min(config_.block_size, seq_len - start);
  }
  DeviceTensor k_out({H, (int64_t)rows, D}, dtype_), v_out({H, (int64_t)rows, D}, dtype_);
  if (rows == 0) return {k_out, v_out};
  std::vector<int32_t> table(block_table.blocks().begin(), block_table.blocks().end());
  const sp_cache_layout lay = layout(layer_idx);
  const int32_t* dtable = g_ints.upload(table, stream_);
  check_sp(sp_kv_gather(k_out.data(), v_out.data(), k_cache_.data(), v_cache_.data(), &lay,
                        dtable, (int32_t)table.size(), (int32_t)rows, dtype_, stream_),
           "gather_kv");
  check_hip(hipStreamSynchronize(stream_), "gather_kv");
  return {k_out, v_out};
}

// ---------------------------------------------------------------------------------------------
// PagedSequence / PagedScheduler
// ---------------------------------------------------------------------------------------------

Result<Unit> PagedSequence::allocate_for_tokens(size_t num_tokens, PagedKvCache& cache) {
  const size_t new_len = block_table.seq_len() + num_tokens;
  const size_t needed = (new_len + cache.block_size() - 1) / cache.block_size();
  for (size_t i = block_table.num_blocks(); i < needed; ++i) {
    const auto b = cache.allocate_block();
    if (!b) return Result<Unit>::Err("Out of memory: no free blocks");
    block_table.add_block(*b);
  }
  return Result<Unit>::Ok(Unit{});
}

Result<size_t> PagedScheduler::add_sequence() {
  const size_t id = sequences_.size();
  sequences_.emplace_back(cache.block_size());
  return Result<size_t>::Ok(id);
}

const PagedSequence* PagedScheduler::get_sequence(size_t seq_id) const {
  return seq_id < sequences_.size() ? &sequences_[seq_id] : nullptr;
}

PagedSequence* PagedScheduler::get_sequence_mut(size_t seq_id) {
  return seq_id < sequences_.size() ? &sequences_[seq_id] : nullptr;
}

Result<Unit> PagedScheduler::allocate(size_t seq_id, size_t num_tokens) {
  PagedSequence* s = get_sequence_mut(seq_id);
  if (!s) return Result<Unit>::Err("Invalid sequence ID");
  return s->allocate_for_tokens(num_tokens, cache);
}

void PagedScheduler::free_sequence(size_t seq_id) {
  if (const PagedSequence* s = get_sequence(seq_id)) cache.free_sequence(s->block_table);
}

// ---------------------------------------------------------------------------------------------
// KvCache / ModelKvCache
// ---------------------------------------------------------------------------------------------

std::pair<DeviceTensor, DeviceTensor> KvCache::update(const DeviceTensor& k,
                                                      const DeviceTensor& v) {
  const auto& d = k.dims();
  if (d.size() != 4 || v.dims() != d)
    throw std::runtime_error("KvCache::update: k and v must be [batch, heads, new_len, dim]");
  const size_t new_len = (size_t)d[2];
  DeviceTensor full_k = k, full_v = v;
  if (k_ && v_) {
    const auto& c = k_->dims();
    if (c[0] != d[0] || c[1] != d[1] || c[3] != d[3] || k_->dtype() != k.dtype())
      throw std::runtime_error("KvCache::update: shape mismatch with the cached tensors");
    const int64_t L = c[2], S = d[2], rows = c[0] * c[1];
    const size_t es = dtype_bytes(k.dtype()), row_old = (size_t)(L * d[3]) * es,
                 row_new = (size_t)(S * d[3]) * es;
    // Tensor::cat along dim 2: per (batch, head) row, the cached rows then the new ones.
    for (int w = 0; w < 2; ++w) {
      const DeviceTensor& cached = w == 0 ? *k_ : *v_;
      const DeviceTensor& fresh = w == 0 ? k : v;
      DeviceTensor out({c[0], c[1], L + S, d[3]}, k.dtype());
      if (row_old)
        check_hip(hipMemcpy2DAsync(out.data(), row_old + row_new, cached.data(), row_old,
                                   row_old, (size_t)rows, hipMemcpyDeviceToDevice, stream_),
                  "cat");
      if (row_new)
        check_hip(hipMemcpy2DAsync((char*)out.data() + row_old, row_old + row_new, fresh.data(),
                                   row_new, row_new, (size_t)rows, hipMemcpyDeviceToDevice,
                                   stream_),
                  "cat");
      (w == 0 ? full_k : full_v) = out;
    }
  }
  k_ = full_k;
  v_ = full_v;
  current_pos_ += new_len;
  return {full_k, full_v};
}

ModelKvCache::ModelKvCache(size_t num_layers, size_t max_seq_len, hipStream_t stream)
    : max_seq_len(max_seq_len) {
  for (size_t i = 0; i < num_layers; ++i) layers.emplace_back(max_seq_len, stream);
}

CacheUpdate ModelKvCache::update_layer(size_t layer_idx, const DeviceTensor& k,
                                       const DeviceTensor& v) {
  auto kv = layer(layer_idx).update(k, v);
  return CacheUpdate{kv.first, kv.second};
}

// ---------------------------------------------------------------------------------------------
// PagedAttentionCache
// ---------------------------------------------------------------------------------------------

void PagedAttentionCache::ensure_capacity(size_t additional_tokens) {
  const size_t new_len = block_table_.seq_len() + additional_tokens;
  const size_t needed = (new_len + cache_.block_size() - 1) / cache_.block_size();
  for (size_t i = block_table_.num_blocks(); i < needed; ++i) {
    const auto b = cache_.allocate_block();
    if (!b) throw std::runtime_error("PagedAttentionCache: out of memory");
    block_table_.add_block(*b);
  }
}

CacheUpdate PagedAttentionCache::update_layer(size_t layer_idx, const DeviceTensor& k,
                                              const DeviceTensor& v) {
  const auto& d = k.dims();
  if (d.size() != 4 || d[0] != 1 || v.dims() != d)
    throw std::runtime_error(
        "PagedAttentionCache::update_layer: k and v must be [1, num_kv_heads, new_len, dim]");
  const size_t new_len = (size_t)d[2];
  size_t start_pos;
  if (layer_idx == 0) {
    start_pos = block_table_.seq_len();
    ensure_capacity(new_len);
    block_table_.increment_seq_len(new_len);
  } else {
    if (block_table_.seq_len() < new_len)
      throw std::runtime_error("PagedAttentionCache::update_layer: layer 0 must come first");
    start_pos = block_table_.seq_len() - new_len;
  }
  cache_.store_kv(layer_idx, block_table_, k.reshape({d[1], d[2], d[3]}),
                  v.reshape({d[1], d[2], d[3]}), start_pos);
  auto kv = cache_.gather_kv(layer_idx, block_table_);
  const auto& g = kv.first.dims();
  return CacheUpdate{kv.first.reshape({1, g[0], g[1], g[2]}),
                     kv.second.reshape({1, g[0], g[1], g[2]})};
}

void PagedAttentionCache::clear() {
  cache_.free_sequence(block_table_);
  block_table_ = BlockTable(cache_.block_size());
}

// ---------------------------------------------------------------------------------------------
// attention functions
// ---------------------------------------------------------------------------------------------

std::vector<float> causal_mask(size_t seq_len) {
  std::vector<float> m(seq_len * seq_len, 0.f);
  for (size_t i = 0; i < seq_len; ++i)
    for (size_t j = i + 1; j < seq_len; ++j) m[i * seq_len + j] = -INFINITY;
  return m;
}

DeviceTensor causal_mask_tensor(size_t seq_len) {
  const std::vector<float> m = causal_mask(seq_len);
  return DeviceTensor::from_host(m.data(), {(int64_t)seq_len, (int64_t)seq_len}, SP_F32);
}

// Shapes and dtypes flash_attention / flash_attention_masked accept; the message otherwise (the
// kernels' own head-dim limits are reported by the library).
static std::optional<std::string> flash_shape_error(const DeviceTensor& query,
                                                    const DeviceTensor& key,
                                                    const DeviceTensor& value) {
  const auto& q = query.dims();
  const auto& k = key.dims();
  const auto& v = value.dims();
  if (q.size() != 4 || k.size() != 4 || v.size() != 4 || k[0] != q[0] || k[1] != q[1] ||
      k[3] != q[3] || v[0] != k[0] || v[1] != k[1] || v[2] != k[2])
    return std::string("flash_attention: expected q [B,H,Sq,D], k [B,H,Sk,D], v [B,H,Sk,Dv]");
  if (key.dtype() != query.dtype() || value.dtype() != query.dtype())
    return std::string("flash_attention: q, k and v must share one dtype");
  return std::nullopt;
}

// flash_attention_impl (sketchpad-cubecl attention.rs:130-178): out [B, H, Sq, Dv] of
// out_dtype (or q's), then the kernel; mask strides 0 broadcast one [Sq, Sk] mask.
static FlashResult flash_impl(const DeviceTensor& query, const DeviceTensor& key,
                              const DeviceTensor& value, const DeviceTensor* mask,
                              const FlashAttentionOptions& options, hipStream_t stream) {
  FlashResult r;
  if (auto e = flash_shape_error(query, key, value)) {
    r.error = AttentionSetupError{*e};
    return r;
  }
  const auto& q = query.dims();
  const auto& k = key.dims();
  const auto& v = value.dims();
  int64_t sb = 0, sh = 0, sq = 0;
  if (mask) {
    const auto& m = mask->dims();
    if (mask->dtype() != SP_F32) {
      r.error = AttentionSetupError{"flash_attention_masked: the mask must be f32"};
      return r;
    }
    if (m.size() == 4 && m[0] == q[0] && m[1] == q[1] && m[2] == q[2] && m[3] == k[2]) {
      sb = q[1] * q[2] * k[2];
      sh = q[2] * k[2];
    } else if (!(m.size() == 2 && m[0] == q[2] && m[1] == k[2])) {
      r.error = AttentionSetupError{"flash_attention_masked: mask must be [B,H,Sq,Sk] or [Sq,Sk]"};
      return r;
    }
    sq = k[2];
  }
  const sp_dtype out_dtype = options.out_dtype.value_or(query.dtype());
  DeviceTensor out({q[0], q[1], q[2], v[3]}, out_dtype);
  const int rc = sp_flash_attention_ex(
      out.data(), query.data(), key.data(), value.data(),
      mask ? (const float*)mask->data() : nullptr, sb, sh, sq, (int32_t)q[0], (int32_t)q[1],
      (int32_t)q[2], (int32_t)k[2], (int32_t)q[3], (int32_t)v[3], (float)pow((double)q[3], -0.5),
      options.causal ? 1 : 0, query.dtype(), out_dtype, stream);
  if (rc != SP_OK) {
    r.error = AttentionSetupError{sp_last_error()};
    return r;
  }
  r.out = out;
  return r;
}

FlashResult flash_attention(const DeviceTensor& query, const DeviceTensor& key,
                            const DeviceTensor& value, const FlashAttentionOptions& options,
                            hipStream_t stream) {
  return flash_impl(query, key, value, nullptr, options, stream);
}

FlashResult flash_attention_masked(const DeviceTensor& query, const DeviceTensor& key,
                                   const DeviceTensor& value, const DeviceTensor& mask,
                                   const FlashAttentionOptions& options, hipStream_t stream) {
  return flash_impl(query, key, value, &mask, options, stream);
}

DeviceTensor qkv_attention(const DeviceTensor& q, const DeviceTensor& k, const DeviceTensor& v,
                           const std::optional<DeviceTensor>& mask, hipStream_t stream) {
  if (mask && mask->dims().size() != 2)
    throw std::runtime_error("qkv_attention: the mask must be [seq_q, seq_k]");
  FlashResult r = flash_impl(q, k, v, mask ? &*mask : nullptr, FlashAttentionOptions(), stream);
  if (!r.is_ok()) throw std::runtime_error(r.error->message);
  return *r.out;
}

}  // namespace sketchpad
