// C++ mirror of rhi-zone/sketchpad's iteration-level scheduler,
// crates/sketchpad-core/src/continuous_batching.rs, with the reference's names, fields and
// decisions (including its tie-breaking: Rust's Iterator::max_by_key returns the last maximum,
// min_by_key the first minimum). Host-only bookkeeping: it counts blocks; the block ids
// themselves come from PagedScheduler / PagedKvCache (paged_attention.hpp), and
// RaggedBatchBuilder (ragged_batch.hpp) turns one iteration's decision into kernel metadata.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <deque>
#include <optional>
#include <unordered_map>
#include <vector>

namespace sketchpad {

// SequenceStatus (continuous_batching.rs:31-42).
enum class SequenceStatus { Waiting, Running, Finished, Preempted };

// Sequence (continuous_batching.rs:44-96).
struct Sequence {
  size_t id = 0;
  std::vector<int64_t> input_ids;
  std::vector<int64_t> output_ids;
  SequenceStatus status = SequenceStatus::Waiting;
  size_t generated_len = 0;
  size_t max_new_tokens = 0;
  uint64_t arrival_time = 0;
  size_t num_blocks = 0;

  Sequence() = default;
  Sequence(size_t id, std::vector<int64_t> input_ids, size_t max_new_tokens, uint64_t arrival_time)
      : id(id), input_ids(std::move(input_ids)), max_new_tokens(max_new_tokens),
        arrival_time(arrival_time) {}
  // prompt + generated (:79-82)
  size_t total_len() const { return input_ids.size() + output_ids.size(); }
  // :84-87
  bool is_finished() const {
    return generated_len >= max_new_tokens || status == SequenceStatus::Finished;
  }
  // :89-93
  void add_token(int64_t token) {
    output_ids.push_back(token);
    generated_len += 1;
  }
  void finish() { status = SequenceStatus::Finished; }
};

// SchedulingPolicy (continuous_batching.rs:98-107).
enum class SchedulingPolicy { Fcfs, ShortestFirst, LongestFirst };

// ContinuousBatchingConfig (continuous_batching.rs:109-147), same defaults.
struct ContinuousBatchingConfig {
  size_t max_batch_size = 256;
  size_t max_seq_len = 4096;
  size_t block_size = 16;
  size_t total_blocks = 1000;
  SchedulingPolicy policy = SchedulingPolicy::Fcfs;
  bool enable_preemption = true;

  ContinuousBatchingConfig() = default;
  // ContinuousBatchingConfig::new (:139-146)
  ContinuousBatchingConfig(size_t max_batch_size, size_t total_blocks)
      : max_batch_size(max_batch_size), total_blocks(total_blocks) {}
};

// ScheduleOutput (continuous_batching.rs:149-160).
struct ScheduleOutput {
  std::vector<size_t> running;
  std::vector<size_t> preempted;
  std::vector<size_t> finished;
  size_t free_blocks = 0;
};

// BatchingStats (continuous_batching.rs:408-417).
struct BatchingStats {
  size_t num_running = 0;
  size_t num_waiting = 0;
  size_t total_running_tokens = 0;
  size_t free_blocks = 0;
  size_t total_blocks = 0;
  float utilization = 0.f;
};

// ContinuousBatchingScheduler (continuous_batching.rs:162-406).
class ContinuousBatchingScheduler {
 public:
  explicit ContinuousBatchingScheduler(ContinuousBatchingConfig config)
      : config_(config), free_blocks_(config.total_blocks) {}

  size_t add_sequence(std::vector<int64_t> input_ids, size_t max_new_tokens);  // :190-200
  const Sequence* get_sequence(size_t id) const;                                // :202-205
  Sequence* get_sequence_mut(size_t id);                                        // :207-210
  ScheduleOutput schedule();                                                    // :218-316
  void update_sequence(size_t seq_id, int64_t token);                           // :352-357
  void finish_sequence(size_t seq_id);                                          // :359-364
  std::optional<Sequence> remove_sequence(size_t seq_id);                       // :366-371
  size_t num_sequences() const { return sequences_.size(); }
  size_t num_running() const { return running_.size(); }
  size_t num_waiting() const { return waiting_queue_.size(); }
  bool is_empty() const { return sequences_.empty(); }
  BatchingStats stats() const;  // :388-405
  const ContinuousBatchingConfig& config() const { return config_; }

 private:
  size_t blocks_needed(const Sequence& seq) const;  // :212-216
  std::optional<size_t> select_next_waiting() const;  // :318-342
  std::optional<size_t> select_for_preemption() const;  // :344-350

  ContinuousBatchingConfig config_;
  std::unordered_map<size_t, Sequence> sequences_;
  std::deque<size_t> waiting_queue_;
  std::vector<size_t> running_;
  size_t next_id_ = 0;
  uint64_t current_time_ = 0;
  size_t free_blocks_;
};

}  // namespace sketchpad
