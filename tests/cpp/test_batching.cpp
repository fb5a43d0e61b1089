// Tests of the iteration-level scheduler mirror (sketchpad_amd/host/continuous_batching.hpp) and
// of ragged batches over the paged cache (sketchpad_amd/host/ragged_batch.hpp). The first group
// restates the reference's own scheduler tests (crates/sketchpad-core/src/continuous_batching.rs:
// 419-566) plus its tie-breaking; the second checks batch metadata against the block tables'
// closed form, and runs a continuous-batching loop on the GPU (sequences join as others finish,
// prompts are prefilled in chunks next to decoding sequences) whose every attention output is
// compared with a float64 host computation over the sequence's own history.
#include <math.h>
#include <string.h>

#include <map>
#include <random>

#include "continuous_batching.hpp"
#include "ragged_batch.hpp"
#include "test_harness.hpp"

using namespace sketchpad;

// ---- continuous_batching.rs:419-566 -----------------------------------------------------------

TEST(test_sequence_lifecycle, false) {
  Sequence seq(0, {1, 2, 3}, 5, 0);
  CHECK(seq.total_len() == 3);
  CHECK(!seq.is_finished());
  CHECK(seq.status == SequenceStatus::Waiting);
  seq.add_token(4);
  seq.add_token(5);
  CHECK(seq.total_len() == 5);
  CHECK(seq.generated_len == 2);
  seq.add_token(6);
  seq.add_token(7);
  seq.add_token(8);
  CHECK(seq.is_finished());
}

TEST(test_scheduler_add_and_schedule, false) {
  ContinuousBatchingConfig config;
  config.max_batch_size = 2;
  config.total_blocks = 100;
  config.block_size = 4;
  ContinuousBatchingScheduler scheduler(config);
  const size_t id0 = scheduler.add_sequence({1, 2, 3}, 10);
  scheduler.add_sequence({4, 5}, 10);
  scheduler.add_sequence({6, 7, 8, 9}, 10);
  CHECK(scheduler.num_sequences() == 3);
  CHECK(scheduler.num_waiting() == 3);
  ScheduleOutput out = scheduler.schedule();
  CHECK(out.running.size() == 2);
  CHECK(scheduler.num_waiting() == 1);
  scheduler.finish_sequence(id0);
  out = scheduler.schedule();
  CHECK(std::find(out.finished.begin(), out.finished.end(), id0) != out.finished.end());
  CHECK(out.running.size() == 2);
}

TEST(test_scheduler_memory_limits, false) {
  ContinuousBatchingConfig config;
  config.max_batch_size = 10;
  config.total_blocks = 5;
  config.block_size = 4;
  config.enable_preemption = false;
  ContinuousBatchingScheduler scheduler(config);
  for (int i = 0; i < 10; ++i) scheduler.add_sequence(std::vector<int64_t>(3, i), 10);
  const ScheduleOutput out = scheduler.schedule();
  CHECK(out.running.size() <= 5);
  CHECK(out.running.size() == 5);  // each needs ceil(4/4) = 1 block: exactly five fit
}

TEST(test_scheduler_preemption, false) {
  ContinuousBatchingConfig config;
  config.max_batch_size = 10;
  config.total_blocks = 10;
  config.block_size = 4;
  config.enable_preemption = true;
  ContinuousBatchingScheduler scheduler(config);
  const size_t id0 = scheduler.add_sequence(std::vector<int64_t>(15, 1), 100);
  ScheduleOutput out = scheduler.schedule();
  CHECK(std::find(out.running.begin(), out.running.end(), id0) != out.running.end());
  for (int i = 0; i < 30; ++i) scheduler.update_sequence(id0, 99);
  for (int i = 0; i < 10; ++i) scheduler.add_sequence(std::vector<int64_t>(10, 1), 50);
  out = scheduler.schedule();
  CHECK(!out.preempted.empty() || out.running.size() < 10);
}

TEST(test_scheduling_policies, false) {
  ContinuousBatchingConfig config;
  config.max_batch_size = 1;
  config.total_blocks = 100;
  config.policy = SchedulingPolicy::ShortestFirst;
  ContinuousBatchingScheduler scheduler(config);
  scheduler.add_sequence({1}, 100);
  const size_t short_id = scheduler.add_sequence({2}, 10);
  const ScheduleOutput out = scheduler.schedule();
  CHECK(out.running.size() == 1 && out.running[0] == short_id);
}

TEST(test_stats, false) {
  ContinuousBatchingScheduler scheduler((ContinuousBatchingConfig()));
  scheduler.add_sequence({1, 2, 3}, 10);
  scheduler.add_sequence({4, 5}, 10);
  scheduler.schedule();
  const BatchingStats stats = scheduler.stats();
  CHECK(stats.num_running == 2);
  CHECK(stats.total_running_tokens == 5);
  CHECK(stats.utilization > 0.0f);
  // each needs ceil((len + 1) / 16) = 1 block of the default 1000
  CHECK(stats.free_blocks == 998);
}

// ---- tie-breaking and bookkeeping the reference fixes through Rust's iterator semantics --------

TEST(test_policy_ties, false) {
  // max_by_key keeps the last maximum, min_by_key the first minimum
  for (SchedulingPolicy p : {SchedulingPolicy::LongestFirst, SchedulingPolicy::ShortestFirst}) {
    ContinuousBatchingConfig config;
    config.max_batch_size = 1;
    config.policy = p;
    ContinuousBatchingScheduler scheduler(config);
    const size_t a = scheduler.add_sequence({1}, 7);
    const size_t b = scheduler.add_sequence({2}, 7);
    const ScheduleOutput out = scheduler.schedule();
    CHECK(out.running.size() == 1);
    CHECK(out.running[0] == (p == SchedulingPolicy::LongestFirst ? b : a));
  }
}

TEST(test_preemption_order_and_requeue, false) {
  // Two running sequences hold 2 blocks each and none is free; a's growth to 3 blocks fails, so
  // the preemption loop (while no block is free) evicts the last of the two with the most blocks,
  // b, which frees 2 blocks and ends the loop. b goes to the front of the queue and is admitted
  // again in the same call (it still needs 2 blocks); a keeps its 2.
  ContinuousBatchingConfig config;
  config.max_batch_size = 4;
  config.total_blocks = 4;
  config.block_size = 4;
  ContinuousBatchingScheduler s(config);
  const size_t a = s.add_sequence(std::vector<int64_t>(7, 1), 100);  // ceil(8/4) = 2 blocks
  const size_t b = s.add_sequence(std::vector<int64_t>(7, 1), 100);
  ScheduleOutput out = s.schedule();
  CHECK(out.running.size() == 2 && out.free_blocks == 0);
  s.update_sequence(a, 0);  // a now needs ceil(9/4) = 3 blocks
  out = s.schedule();
  CHECK(out.preempted.size() == 1 && out.preempted[0] == b);
  CHECK((out.running == std::vector<size_t>{a, b}));
  CHECK(s.get_sequence(b)->status == SequenceStatus::Running);
  CHECK(s.get_sequence(a)->num_blocks == 2 && s.get_sequence(b)->num_blocks == 2);
  CHECK(out.free_blocks == 0);
}

TEST(test_finished_blocks_return, false) {
  ContinuousBatchingConfig config;
  config.max_batch_size = 8;
  config.total_blocks = 10;
  config.block_size = 4;
  ContinuousBatchingScheduler s(config);
  const size_t a = s.add_sequence({1, 2, 3, 4, 5}, 1);  // ceil(6/4) = 2 blocks
  s.schedule();
  CHECK(s.stats().free_blocks == 8);
  s.update_sequence(a, 9);  // generated 1 of 1: finished
  const ScheduleOutput out = s.schedule();
  CHECK(out.finished.size() == 1 && out.finished[0] == a);
  CHECK(out.free_blocks == 10);
  CHECK(s.remove_sequence(a).has_value() && s.is_empty());
}

// ---- ragged batches: metadata from the block tables --------------------------------------------

TEST(test_ragged_batch_metadata, true) {
  PagedScheduler ps(PagedKvCacheConfig(4, 32, 2, 64, 1), SP_BF16);
  std::vector<size_t> ids;
  for (int i = 0; i < 3; ++i) ids.push_back(ps.add_sequence().unwrap());
  // interleave growth so the tables are not contiguous
  CHECK(ps.allocate(ids[0], 5).is_ok());
  CHECK(ps.allocate(ids[1], 2).is_ok());
  ps.get_sequence_mut(ids[0])->block_table.increment_seq_len(5);
  ps.get_sequence_mut(ids[1])->block_table.increment_seq_len(2);
  const std::vector<BatchEntry> entries = {{ids[0], 1}, {ids[1], 7}, {ids[2], 3}};
  Result<RaggedBatch> r = build_ragged_batch(ps, entries);
  CHECK(r.is_ok());
  const RaggedBatch& b = r.unwrap();
  CHECK(b.num_seqs() == 3 && b.num_tokens() == 11);
  CHECK((b.cu_seqlens_q == std::vector<int32_t>{0, 1, 8, 11}));
  CHECK((b.context_lens == std::vector<int32_t>{6, 9, 3}));
  CHECK(b.max_seqlen_q == 7 && b.max_context_len == 9 && !b.decode_only());
  size_t t = 0;
  for (size_t s = 0; s < 3; ++s) {
    const BlockTable& table = ps.get_sequence(ids[s])->block_table;
    const size_t start = table.seq_len();
    for (size_t i = 0; i < entries[s].num_new; ++i, ++t) {
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
}

TEST(test_ragged_batch_out_of_memory, true) {
  PagedScheduler ps(PagedKvCacheConfig(4, 2, 1, 64, 1), SP_BF16);
  const size_t a = ps.add_sequence().unwrap();
  Result<RaggedBatch> r = build_ragged_batch(ps, {{a, 9}});  // needs 3 of 2 blocks
  CHECK(r.is_err() && strcmp(r.error(), "Out of memory: no free blocks") == 0);
  Result<RaggedBatch> r2 = build_ragged_batch(ps, {{a + 7, 1}});
  CHECK(r2.is_err() && strcmp(r2.error(), "Invalid sequence ID") == 0);
}

// ---- a continuous-batching loop on the GPU ------------------------------------------------------

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

struct History {  // one sequence's appended K/V rows, [pos][Hkv][D]
  std::vector<float> k, v;
  size_t len = 0;
};

}  // namespace

TEST(test_continuous_batching_loop, true) {
  const int hq = 8, hkv = 2, d = 64, bs = 16, chunk = 24;
  const float scale = 1.0f / sqrtf((float)d);
  PagedScheduler ps(PagedKvCacheConfig(bs, 96, hkv, d, 1), SP_BF16);
  BatchedPagedAttention attn(ps.cache);
  ContinuousBatchingConfig cfg;
  cfg.max_batch_size = 4;
  cfg.block_size = bs;
  cfg.total_blocks = 96;
  cfg.enable_preemption = false;
  ContinuousBatchingScheduler cb(cfg);
  std::mt19937 rng(1234);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::map<size_t, size_t> paged_id;    // scheduler id -> PagedScheduler id
  std::map<size_t, size_t> prompt_left;  // prompt tokens not yet in the cache
  std::map<size_t, History> hist;
  for (int i = 0; i < 7; ++i) {
    const size_t plen = 1 + rng() % 57;
    const size_t id = cb.add_sequence(std::vector<int64_t>(plen, 1), 2 + rng() % 5);
    prompt_left[id] = plen;
  }
  int iterations = 0, prefill_steps = 0, decode_steps = 0;
  double worst = 0.0;
  while (!cb.is_empty() && iterations < 200) {
    ++iterations;
    const ScheduleOutput so = cb.schedule();
    for (size_t f : so.finished) {
      ps.free_sequence(paged_id.at(f));
      cb.remove_sequence(f);
    }
    if (so.running.empty()) continue;
    std::vector<BatchEntry> entries;
    std::vector<size_t> sched_ids;
    for (size_t id : so.running) {
      if (!paged_id.count(id)) paged_id[id] = ps.add_sequence().unwrap();
      const size_t n = prompt_left[id] > 0 ? std::min<size_t>(prompt_left[id], chunk) : 1;
      entries.push_back({paged_id[id], n});
      sched_ids.push_back(id);
    }
    Result<RaggedBatch> rb = build_ragged_batch(ps, entries);
    CHECK(rb.is_ok());
    if (rb.is_err()) return;
    const RaggedBatch& b = rb.unwrap();
    const size_t T = b.num_tokens();
    std::vector<uint16_t> qh(T * hq * d), kh(T * hkv * d), vh(T * hkv * d);
    for (auto& x : qh) x = bf16_bits(nd(rng));
    for (auto& x : kh) x = bf16_bits(nd(rng));
    for (auto& x : vh) x = bf16_bits(nd(rng));
    DeviceTensor q = DeviceTensor::from_host(qh.data(), {(int64_t)T, hq, d}, SP_BF16);
    DeviceTensor k = DeviceTensor::from_host(kh.data(), {(int64_t)T, hkv, d}, SP_BF16);
    DeviceTensor v = DeviceTensor::from_host(vh.data(), {(int64_t)T, hkv, d}, SP_BF16);
    DeviceTensor o({(int64_t)T, hq, d}, SP_BF16);
    DeviceRaggedBatch db(b, ps.cache.stream());
    attn.forward(0, db, q, k, v, o, scale);
    std::vector<uint16_t> oh(T * hq * d);
    o.to_host(oh.data());
    (b.decode_only() ? decode_steps : prefill_steps) += 1;
    // host reference: each new token attends its sequence's keys 0..pos (the history plus the
    // new rows up to itself), GQA head h -> kv head h / (hq / hkv)
    for (size_t s = 0; s < b.num_seqs(); ++s) {
      History& H = hist[sched_ids[s]];
      for (int t = b.cu_seqlens_q[s]; t < b.cu_seqlens_q[s + 1]; ++t) {
        for (int x = 0; x < hkv * d; ++x) {
          H.k.push_back(bf16_value(kh[(size_t)t * hkv * d + x]));
          H.v.push_back(bf16_value(vh[(size_t)t * hkv * d + x]));
        }
        H.len += 1;
      }
      for (int t = b.cu_seqlens_q[s]; t < b.cu_seqlens_q[s + 1]; ++t) {
        const size_t pos = (size_t)b.positions[t];
        for (int h = 0; h < hq; ++h) {
          const int g = h / (hq / hkv);
          std::vector<double> sc(pos + 1);
          double mx = -1e300;
          for (size_t j = 0; j <= pos; ++j) {
            double acc = 0;
            for (int e = 0; e < d; ++e)
              acc += (double)bf16_value(qh[((size_t)t * hq + h) * d + e]) *
                     H.k[(j * hkv + g) * d + e];
            sc[j] = acc * scale;
            mx = std::max(mx, sc[j]);
          }
          double den = 0;
          for (auto& x : sc) den += (x = exp(x - mx));
          for (int e = 0; e < d; ++e) {
            double num = 0;
            for (size_t j = 0; j <= pos; ++j) num += sc[j] * H.v[(j * hkv + g) * d + e];
            const double err =
                fabs(num / den - bf16_value(oh[((size_t)t * hq + h) * d + e]));
            worst = std::max(worst, err);
          }
        }
      }
    }
    commit_ragged_batch(ps, b);
    for (size_t s = 0; s < b.num_seqs(); ++s) {
      const size_t id = sched_ids[s];
      const size_t n = (size_t)(b.cu_seqlens_q[s + 1] - b.cu_seqlens_q[s]);
      if (prompt_left[id] > 0) {
        prompt_left[id] -= n;
        if (prompt_left[id] == 0) cb.update_sequence(id, 0);  // the prompt's last step emits one
      } else {
        cb.update_sequence(id, 0);
      }
    }
  }
  printf("  %d iterations (%d with prompt chunks, %d decode-only), worst |err| %.3g\n",
         iterations, prefill_steps, decode_steps, worst);
  CHECK(cb.is_empty());
  CHECK(prefill_steps > 0 && decode_steps > 0);
  CHECK(worst <= 2e-2);
  CHECK(ps.cache.num_free_blocks() == 96);  // every block returned
}
