// Iteration-level scheduler: see continuous_batching.hpp. Each member follows the reference
// function named next to it (crates/sketchpad-core/src/continuous_batching.rs).
#include "continuous_batching.hpp"

#include <algorithm>

namespace sketchpad {

size_t ContinuousBatchingScheduler::add_sequence(std::vector<int64_t> input_ids,
                                                 size_t max_new_tokens) {
  const size_t id = next_id_++;
  sequences_.emplace(id, Sequence(id, std::move(input_ids), max_new_tokens, current_time_));
  waiting_queue_.push_back(id);
  return id;
}

const Sequence* ContinuousBatchingScheduler::get_sequence(size_t id) const {
  auto it = sequences_.find(id);
  return it == sequences_.end() ? nullptr : &it->second;
}

Sequence* ContinuousBatchingScheduler::get_sequence_mut(size_t id) {
  auto it = sequences_.find(id);
  return it == sequences_.end() ? nullptr : &it->second;
}

// Blocks for the sequence plus the token about to be generated: ceil((len + 1) / block_size).
size_t ContinuousBatchingScheduler::blocks_needed(const Sequence& seq) const {
  const size_t total_tokens = seq.total_len() + 1;
  return (total_tokens + config_.block_size - 1) / config_.block_size;
}

ScheduleOutput ContinuousBatchingScheduler::schedule() {
  current_time_ += 1;
  ScheduleOutput output;
  output.free_blocks = free_blocks_;

  // finished sequences leave the running set and return their blocks (:230-245)
  std::vector<size_t> still_running;
  for (size_t seq_id : running_) {
    auto it = sequences_.find(seq_id);
    if (it == sequences_.end()) continue;
    if (it->second.is_finished()) {
      output.finished.push_back(seq_id);
      free_blocks_ += it->second.num_blocks;
    } else {
      still_running.push_back(seq_id);
    }
  }
  running_ = std::move(still_running);

  // running sequences grow by the blocks they need, while blocks remain (:247-264)
  for (size_t seq_id : running_) {
    auto it = sequences_.find(seq_id);
    if (it == sequences_.end()) continue;
    const size_t needed = blocks_needed(it->second);
    if (needed > it->second.num_blocks) {
      const size_t additional = needed - it->second.num_blocks;
      if (additional <= free_blocks_) {
        free_blocks_ -= additional;
        it->second.num_blocks = needed;
      }
      // otherwise the reference leaves it to the preemption loop below
    }
  }

  // preempt the sequence holding the most blocks while none are free (:266-286)
  if (config_.enable_preemption) {
    while (free_blocks_ == 0 && !running_.empty()) {
      const std::optional<size_t> id = select_for_preemption();
      if (!id) break;
      auto it = sequences_.find(*id);
      if (it != sequences_.end()) {
        free_blocks_ += it->second.num_blocks;
        it->second.num_blocks = 0;
        it->second.status = SequenceStatus::Preempted;
        output.preempted.push_back(*id);
      }
      running_.erase(std::remove(running_.begin(), running_.end(), *id), running_.end());
      waiting_queue_.push_front(*id);
    }
  }

  // admit waiting sequences in policy order while batch slots and blocks allow (:288-310)
  while (running_.size() < config_.max_batch_size) {
    const std::optional<size_t> next = select_next_waiting();
    if (!next) break;
    auto it = sequences_.find(*next);
    if (it == sequences_.end()) break;
    const size_t need = blocks_needed(it->second);
    if (need > free_blocks_) break;  // not enough memory
    free_blocks_ -= need;
    waiting_queue_.erase(std::remove(waiting_queue_.begin(), waiting_queue_.end(), *next),
                         waiting_queue_.end());
    running_.push_back(*next);
    it->second.status = SequenceStatus::Running;
    it->second.num_blocks = need;
  }

  output.running = running_;
  output.free_blocks = free_blocks_;
  return output;
}

// Fcfs: the queue's front; ShortestFirst / LongestFirst: fewest / most remaining tokens
// (max_new_tokens - generated_len, wrapping like the reference's usize in release builds), the
// first minimum / last maximum in queue order.
std::optional<size_t> ContinuousBatchingScheduler::select_next_waiting() const {
  if (waiting_queue_.empty()) return std::nullopt;
  auto remaining = [&](size_t id, size_t missing) {
    auto it = sequences_.find(id);
    return it == sequences_.end() ? missing
                                  : it->second.max_new_tokens - it->second.generated_len;
  };
  switch (config_.policy) {
    case SchedulingPolicy::Fcfs:
      return waiting_queue_.front();
    case SchedulingPolicy::ShortestFirst: {
      size_t best = waiting_queue_.front();
      size_t best_key = remaining(best, SIZE_MAX);
      for (size_t id : waiting_queue_) {
        const size_t k = remaining(id, SIZE_MAX);
        if (k < best_key) best = id, best_key = k;
      }
      return best;
    }
    case SchedulingPolicy::LongestFirst: {
      size_t best = waiting_queue_.front();
      size_t best_key = remaining(best, 0);
      for (size_t id : waiting_queue_) {
        const size_t k = remaining(id, 0);
        if (k >= best_key) best = id, best_key = k;
      }
      return best;
    }
  }
  return std::nullopt;
}

// The running sequence holding the most blocks (the last one on ties).
std::optional<size_t> ContinuousBatchingScheduler::select_for_preemption() const {
  if (running_.empty()) return std::nullopt;
  size_t best = running_.front();
  size_t best_key = 0;
  bool first = true;
  for (size_t id : running_) {
    auto it = sequences_.find(id);
    const size_t k = it == sequences_.end() ? 0 : it->second.num_blocks;
    if (first || k >= best_key) best = id, best_key = k, first = false;
  }
  return best;
}

void ContinuousBatchingScheduler::update_sequence(size_t seq_id, int64_t token) {
  if (Sequence* s = get_sequence_mut(seq_id)) s->add_token(token);
}

void ContinuousBatchingScheduler::finish_sequence(size_t seq_id) {
  if (Sequence* s = get_sequence_mut(seq_id)) s->finish();
}

std::optional<Sequence> ContinuousBatchingScheduler::remove_sequence(size_t seq_id) {
  running_.erase(std::remove(running_.begin(), running_.end(), seq_id), running_.end());
  waiting_queue_.erase(std::remove(waiting_queue_.begin(), waiting_queue_.end(), seq_id),
                       waiting_queue_.end());
  auto it = sequences_.find(seq_id);
  if (it == sequences_.end()) return std::nullopt;
  Sequence s = std::move(it->second);
  sequences_.erase(it);
  return s;
}

BatchingStats ContinuousBatchingScheduler::stats() const {
  BatchingStats st;
  for (size_t id : running_) {
    auto it = sequences_.find(id);
    if (it != sequences_.end()) st.total_running_tokens += it->second.total_len();
  }
  st.num_running = running_.size();
  st.num_waiting = waiting_queue_.size();
  st.free_blocks = free_blocks_;
  st.total_blocks = config_.total_blocks;
  st.utilization = 1.0f - (float)free_blocks_ / (float)config_.total_blocks;
  return st;
}

}  // namespace sketchpad
