// Tests of ragged batches over the paged cache (sketchpad_amd/host/ragged_batch.hpp): batch
// metadata against the block tables' closed form (BlockTable::get_block / get_slot,
// paged_attention.rs:124-132), the builder's input checks, and on the GPU
//   - a serving loop driven by a small schedule local to this file (sequences join as others
//     finish, prompts are prefilled in chunks next to decoding sequences, so most steps are
//     mixed batches that run chunked prefill and decode side by side), and
//   - a multi-layer step through one interleaved-layer pool (run_batched_step: every layer
//     appends at the same positions, the lengths advance once per step),
// whose every attention output is compared with the f64 oracle's attention (test infrastructure,
// oracle/) over the sequence's own history.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <deque>
#include <map>
#include <random>

#include "ragged_batch.hpp"
#include "sp_oracle.h"
#include "test_harness.hpp"

using namespace sketchpad;

// ---- ragged batches: metadata from the block tables --------------------------------------------

TEST(test_ragged_batch_metadata, true) {
  PagedScheduler ps(PagedKvCacheConfig(4, 32, 2, 64, 1), SP_BF16);
  std::vector<size_t> ids;
  for (int i = 0; i < 4; ++i) ids.push_back(ps.add_sequence().unwrap());
  // interleave growth so the tables are not contiguous
  CHECK(ps.allocate(ids[0], 5).is_ok());
  CHECK(ps.allocate(ids[1], 2).is_ok());
  ps.get_sequence_mut(ids[0])->block_table.increment_seq_len(5);
  ps.get_sequence_mut(ids[1])->block_table.increment_seq_len(2);
  const std::vector<BatchEntry> entries = {{ids[0], 1}, {ids[1], 7}, {ids[3], 1}, {ids[2], 3}};
  Result<RaggedBatch> r = build_ragged_batch(ps, entries);
  CHECK(r.is_ok());
  const RaggedBatch& b = r.unwrap();
  // chunks first (ids[1], ids[2]), then the one-token entries (ids[0], ids[3]), each group in
  // the caller's order
  CHECK((b.seq_ids == std::vector<size_t>{ids[1], ids[2], ids[0], ids[3]}));
  CHECK(b.num_seqs() == 4 && b.num_tokens() == 12);
  CHECK(b.num_prefill_seqs == 2 && b.num_prefill_tokens == 10 && b.num_decode_seqs() == 2);
  CHECK((b.cu_seqlens_q == std::vector<int32_t>{0, 7, 10, 11, 12}));
  CHECK((b.context_lens == std::vector<int32_t>{9, 3, 6, 1}));
  CHECK(b.max_seqlen_q == 7 && b.max_context_len == 9 && !b.decode_only());
  CHECK(b.prefill_max_seqlen_q == 7 && b.decode_max_context_len == 6);
  size_t t = 0;
  for (size_t s = 0; s < b.num_seqs(); ++s) {
    const BlockTable& table = ps.get_sequence(b.seq_ids[s])->block_table;
    const size_t start = table.seq_len();
    const size_t n = (size_t)(b.cu_seqlens_q[s + 1] - b.cu_seqlens_q[s]);
    for (size_t i = 0; i < n; ++i, ++t) {
      const size_t pos = start + i;
      CHECK(b.positions[t] == (int32_t)pos);
      CHECK(b.slot_mapping[t] == (int32_t)(table.blocks()[pos / 4] * 4 + pos % 4));
    }
    for (size_t j = 0; j < table.num_blocks(); ++j)
      CHECK(b.block_tables[s * b.max_blocks + j] == (int32_t)table.blocks()[j]);
  }
  // slots are distinct across the batch
  std::vector<int32_t> sl = b.slot_mapping;
  std::sort(sl.begin(), sl.end());
  CHECK(std::adjacent_find(sl.begin(), sl.end()) == sl.end());
  commit_ragged_batch(ps, b);
  CHECK(ps.get_sequence(ids[1])->block_table.seq_len() == 9);
  CHECK(ps.get_sequence(ids[0])->block_table.seq_len() == 6);
  // a batch of one-token entries only is a decode batch
  Result<RaggedBatch> d = build_ragged_batch(ps, {{ids[2], 1}, {ids[3], 1}});
  CHECK(d.is_ok() && d.unwrap().decode_only() && d.unwrap().num_prefill_seqs == 0);
}

TEST(test_ragged_batch_rejects_bad_entries, true) {
  PagedScheduler ps(PagedKvCacheConfig(4, 8, 1, 64, 1), SP_BF16);
  const size_t a = ps.add_sequence().unwrap();
  const size_t b = ps.add_sequence().unwrap();
  const size_t free0 = ps.cache.num_free_blocks();
  Result<RaggedBatch> r0 = build_ragged_batch(ps, {{a, 1}, {b, 0}});
  CHECK(r0.is_err() && strcmp(r0.error(), "Empty batch entry") == 0);
  Result<RaggedBatch> r1 = build_ragged_batch(ps, {{a, 2}, {b, 1}, {a, 1}});
  CHECK(r1.is_err() && strcmp(r1.error(), "Duplicate sequence ID") == 0);
  CHECK(ps.cache.num_free_blocks() == free0);  // rejected before anything was allocated
  Result<RaggedBatch> r2 = build_ragged_batch(ps, {});
  CHECK(r2.is_ok() && r2.unwrap().num_seqs() == 0);
}

TEST(test_ragged_batch_out_of_memory, true) {
  PagedScheduler ps(PagedKvCacheConfig(4, 2, 1, 64, 1), SP_BF16);
  const size_t a = ps.add_sequence().unwrap();
  Result<RaggedBatch> r = build_ragged_batch(ps, {{a, 9}});  // needs 3 of 2 blocks
  CHECK(r.is_err() && strcmp(r.error(), "Out of memory: no free blocks") == 0);
  Result<RaggedBatch> r2 = build_ragged_batch(ps, {{a + 7, 1}});
  CHECK(r2.is_err() && strcmp(r2.error(), "Invalid sequence ID") == 0);
}

// ---- GPU loops ----------------------------------------------------------------------------------

namespace {

float bf16_round(float x) {  // round to nearest even bf16, returned as float
  uint32_t u;
  memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float y;
  memcpy(&y, &u, 4);
  return y;
}
uint16_t bf16_bits(float x) {
  const float r = bf16_round(x);
  uint32_t u;
  memcpy(&u, &r, 4);
  return (uint16_t)(u >> 16);
}
float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

struct History {  // one sequence's appended K/V rows of one layer, [pos][Hkv][D]
  std::vector<float> k, v;
};

// Random bf16 q / k / v rows of one layer of a batch, on the host and the device.
struct LayerInputs {
  std::vector<uint16_t> qh, kh, vh;
  DeviceTensor q, k, v, o;
  LayerInputs(size_t T, int hq, int hkv, int d, std::mt19937& rng) {
    std::normal_distribution<float> nd(0.f, 1.f);
    qh.resize(T * hq * d);
    kh.resize(T * hkv * d);
    vh.resize(T * hkv * d);
    for (auto& x : qh) x = bf16_bits(nd(rng));
    for (auto& x : kh) x = bf16_bits(nd(rng));
    for (auto& x : vh) x = bf16_bits(nd(rng));
    q = DeviceTensor::from_host(qh.data(), {(int64_t)T, hq, d}, SP_BF16);
    k = DeviceTensor::from_host(kh.data(), {(int64_t)T, hkv, d}, SP_BF16);
    v = DeviceTensor::from_host(vh.data(), {(int64_t)T, hkv, d}, SP_BF16);
    o = DeviceTensor({(int64_t)T, hq, d}, SP_BF16);
  }
};

// Appends the batch's new rows to each sequence's history, then checks every output row against
// the f64 oracle's attention (spo_attention_f64, oracle/sp_oracle.c, pinned by tests/test_oracle*.py)
// over the history up to the row's position: no mask for one new token, the causal rule inside a
// chunk (the row sees keys 0 .. pos), GQA head h -> KV head h / (hq / hkv). Returns the worst
// |error|.
double check_layer(const RaggedBatch& b, const LayerInputs& in, const std::vector<uint16_t>& oh,
                   std::map<size_t, History>& hist, int hq, int hkv, int d, float scale) {
  double worst = 0.0;
  std::vector<float> q1((size_t)hq * d);
  std::vector<double> o1((size_t)hq * d);
  for (size_t s = 0; s < b.num_seqs(); ++s) {
    History& H = hist[b.seq_ids[s]];
    for (int t = b.cu_seqlens_q[s]; t < b.cu_seqlens_q[s + 1]; ++t)
      for (int x = 0; x < hkv * d; ++x) {
        H.k.push_back(bf16_value(in.kh[(size_t)t * hkv * d + x]));
        H.v.push_back(bf16_value(in.vh[(size_t)t * hkv * d + x]));
      }
    for (int t = b.cu_seqlens_q[s]; t < b.cu_seqlens_q[s + 1]; ++t) {
      const int64_t pos = b.positions[t];
      for (int x = 0; x < hq * d; ++x) q1[x] = bf16_value(in.qh[(size_t)t * hq * d + x]);
      // one query row [1, hq, d] against keys [pos + 1, hkv, d], all visible
      spo_attention_f64(q1.data(), (int64_t)hq * d, d, H.k.data(), H.v.data(), (int64_t)hkv * d,
                        d, 1, pos + 1, hq, hkv, d, scale, nullptr, 0, 0, -1, SPO_F32, o1.data());
      for (int x = 0; x < hq * d; ++x)
        worst = std::max(worst, fabs(o1[x] - bf16_value(oh[(size_t)t * hq * d + x])));
    }
  }
  return worst;
}

// A request of the serving loop below: prompt tokens still to prefill, tokens still to generate.
struct Request {
  size_t prompt_left;
  size_t gen_left;
  size_t paged_id = 0;
  bool admitted = false;
};

}  // namespace

// Serving loop: at most `slots` requests run at once; each step gives every running request its
// next prompt chunk (up to `chunk` tokens) or one decode token, retires requests whose last
// token was produced (their blocks go back to the pool) and admits waiting requests in arrival
// order into the freed slots. Steps therefore mix chunks and decode tokens in one batch.
TEST(test_serving_loop_mixed_batches, true) {
  const int hq = 8, hkv = 2, d = 64, bs = 16, chunk = 24, slots = 4;
  const float scale = 1.0f / sqrtf((float)d);
  PagedScheduler ps(PagedKvCacheConfig(bs, 96, hkv, d, 1), SP_BF16);
  BatchedPagedAttention attn(ps.cache);
  std::mt19937 rng(1234);
  std::deque<Request> waiting;
  for (int i = 0; i < 7; ++i) waiting.push_back({1 + rng() % 57, 2 + rng() % 5});
  std::vector<Request> running;
  std::map<size_t, History> hist;
  int steps = 0, mixed_steps = 0, prefill_only = 0, decode_only = 0;
  double worst = 0.0;
  while ((!waiting.empty() || !running.empty()) && steps < 200) {
    ++steps;
    while ((int)running.size() < slots && !waiting.empty()) {
      running.push_back(waiting.front());
      waiting.pop_front();
      running.back().paged_id = ps.add_sequence().unwrap();
    }
    std::vector<BatchEntry> entries;
    for (const Request& r : running)
      entries.push_back({r.paged_id, r.prompt_left > 0 ? std::min<size_t>(r.prompt_left, chunk)
                                                       : (size_t)1});
    Result<RaggedBatch> rb = build_ragged_batch(ps, entries);
    CHECK(rb.is_ok());
    if (rb.is_err()) return;
    const RaggedBatch& b = rb.unwrap();
    LayerInputs in(b.num_tokens(), hq, hkv, d, rng);
    DeviceRaggedBatch db(b, ps.cache.stream());
    attn.forward(0, db, in.q, in.k, in.v, in.o, scale);
    std::vector<uint16_t> oh(b.num_tokens() * hq * d);
    in.o.to_host(oh.data());
    if (b.decode_only()) ++decode_only;
    else if (b.num_decode_seqs() == 0) ++prefill_only;
    else ++mixed_steps;
    worst = std::max(worst, check_layer(b, in, oh, hist, hq, hkv, d, scale));
    commit_ragged_batch(ps, b);
    // the step's outputs: a prompt's last chunk and every decode step produce one token
    std::vector<Request> still;
    for (Request& r : running) {
      const size_t n = entries[&r - running.data()].num_new;
      if (r.prompt_left > 0) {
        r.prompt_left -= n;
        if (r.prompt_left == 0) --r.gen_left;
      } else {
        --r.gen_left;
      }
      if (r.gen_left == 0) ps.free_sequence(r.paged_id);
      else still.push_back(r);
    }
    running.swap(still);
  }
  printf("  %d steps (%d mixed, %d chunks only, %d decode only), worst |err| %.3g\n", steps,
         mixed_steps, prefill_only, decode_only, worst);
  CHECK(waiting.empty() && running.empty());
  CHECK(mixed_steps > 0 && decode_only > 0);
  CHECK(worst <= 2e-2);
  CHECK(ps.cache.num_free_blocks() == 96);  // every block returned
}

// Three layers interleaved in one pool ([num_blocks][3][Hkv][BS][D]): each step appends every
// layer's rows at the same positions and attends the same lengths, the sequence lengths advance
// once per step, and no layer's rows overwrite another's.
TEST(test_multi_layer_step, true) {
  const int hq = 8, hkv = 2, d = 128, bs = 16, layers = 3;
  const float scale = 1.0f / sqrtf((float)d);
  PagedScheduler ps(PagedKvCacheConfig(bs, 64, hkv, d, layers), SP_BF16);
  BatchedPagedAttention attn(ps.cache);
  std::mt19937 rng(99);
  std::vector<size_t> ids;
  for (int i = 0; i < 3; ++i) ids.push_back(ps.add_sequence().unwrap());
  std::vector<std::map<size_t, History>> hist(layers);
  // a prefill step (two prompts and an empty-history one-token start), then mixed and decode
  const std::vector<std::vector<BatchEntry>> plan = {
      {{ids[0], 37}, {ids[1], 70}, {ids[2], 1}},
      {{ids[0], 1}, {ids[1], 1}, {ids[2], 45}},
      {{ids[0], 1}, {ids[1], 1}, {ids[2], 1}},
      {{ids[0], 19}, {ids[1], 1}, {ids[2], 1}},
  };
  double worst = 0.0;
  for (const auto& entries : plan) {
    std::vector<size_t> before;
    for (size_t id : ids) before.push_back(ps.get_sequence(id)->block_table.seq_len());
    Result<RaggedBatch> r = run_batched_step(
        ps, entries, layers, ps.cache.stream(), [&](size_t layer, const DeviceRaggedBatch& db) {
          const RaggedBatch& b = db.host();
          // lengths are not advanced while the layers run
          for (size_t i = 0; i < ids.size(); ++i)
            CHECK(ps.get_sequence(ids[i])->block_table.seq_len() == before[i]);
          LayerInputs in(b.num_tokens(), hq, hkv, d, rng);
          attn.forward(layer, db, in.q, in.k, in.v, in.o, scale);
          std::vector<uint16_t> oh(b.num_tokens() * hq * d);
          in.o.to_host(oh.data());
          worst = std::max(worst, check_layer(b, in, oh, hist[layer], hq, hkv, d, scale));
        });
    CHECK(r.is_ok());
    for (size_t i = 0; i < ids.size(); ++i) {
      size_t add = 0;
      for (const BatchEntry& e : entries)
        if (e.seq_id == ids[i]) add = e.num_new;
      CHECK(ps.get_sequence(ids[i])->block_table.seq_len() == before[i] + add);
    }
  }
  printf("  %zu steps x %d layers, worst |err| %.3g\n", plan.size(), layers, worst);
  CHECK(worst <= 2e-2);
}
