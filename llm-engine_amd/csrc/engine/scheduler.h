// Sequences, steps and the iteration-level scheduler.
//
// Interfaces follow the reference (include/engine/sequence.h:42-89,
// include/engine/scheduler.h:22-95): every step mixes prefill chunks of newly
// admitted or still-prefilling sequences with one decode token per running
// sequence, under a token budget; the prefill slices come first. The
// scheduler admits first-come-first-served with an optional lookahead and a
// starvation bound, keeps a free-block watermark, preempts the youngest
// sequence (recompute on resume) when decode runs out of blocks, and has a
// static-batching mode as a baseline.
#pragma once

#include <chrono>
#include <cstdint>
#include <deque>
#include <memory>
#include <vector>

#include "kv_cache.h"

namespace le::engine {

using Clock = std::chrono::steady_clock;

struct SamplingParams {
  int max_tokens = 128;
  float temperature = 0.f;  // this engine samples greedily
  std::vector<int32_t> stop_ids;
  bool ignore_eos = false;
};

enum class SeqStatus { Waiting, Running, Finished };
enum class FinishReason { None, Stop, Length, Abort, Timeout };

struct Sequence {
  uint64_t id = 0;
  std::vector<int32_t> tokens;  // prompt, then generated tokens
  int prompt_len = 0;
  int num_computed = 0;         // positions whose K/V are in the cache
  BlockTable block_table;
  SamplingParams params;
  SeqStatus status = SeqStatus::Waiting;
  FinishReason finish = FinishReason::None;
  int num_preemptions = 0;
  int wait_steps = 0;
  Clock::time_point t_arrival{}, t_first_scheduled{}, t_first_token{}, t_finish{};

  int num_generated() const { return static_cast<int>(tokens.size()) - prompt_len; }
  int num_tokens() const { return static_cast<int>(tokens.size()); }
  bool prefill_done() const { return num_tokens() - num_computed <= 1; }
  bool is_finished() const { return status == SeqStatus::Finished; }
};

using SequencePtr = std::shared_ptr<Sequence>;

// Tokens [start, start + len) of one sequence; needs_logits when the slice
// ends at the sequence's last token.
struct StepSlice {
  Sequence* seq = nullptr;
  int start = 0;
  int len = 0;
  bool needs_logits = false;
  bool is_prefill = false;
};

struct StepInput {
  std::vector<StepSlice> slices;  // prefill slices first, then decode
  int num_prefill_tokens = 0;
  int num_decode_tokens = 0;
  int num_logits = 0;
  bool empty() const { return slices.empty(); }
  int num_tokens() const { return num_prefill_tokens + num_decode_tokens; }
};

struct SchedulerConfig {
  bool continuous = true;
  int max_num_seqs = 32;
  int max_num_batched_tokens = 2048;
  int prefill_chunk_size = 512;
  int admission_lookahead = 1;
  int starvation_wait_steps = 64;
  double max_queue_wait_seconds = 0;
  int watermark_blocks = -1;  // -1: one block per resident sequence; 0: off
};

struct SchedulerStats {
  uint64_t steps = 0, preemptions = 0, admitted = 0, finished = 0, timed_out = 0;
  uint64_t recomputed_tokens = 0;
  uint64_t max_wait_steps = 0;
};

class Scheduler {
 public:
  Scheduler(SchedulerConfig cfg, KVCacheManager& kv) : cfg_(cfg), kv_(kv) {}

  void add(SequencePtr seq);
  void abort(uint64_t seq_id);
  StepInput schedule();
  // sampled[i] belongs to the i-th slice with needs_logits.
  void on_step_done(const StepInput& step, const std::vector<int32_t>& sampled);

  bool has_work() const { return !waiting_.empty() || !running_.empty(); }
  size_t num_waiting() const { return waiting_.size(); }
  size_t num_running() const { return running_.size(); }
  const SchedulerStats& stats() const { return stats_; }
  const std::vector<SequencePtr>& running() const { return running_; }

 private:
  // The running sequences that take part in a step, by phase. A preempted or
  // released sequence leaves both lists.
  struct Residents {
    std::vector<Sequence*> prefilling, decoding;
    void remove(const Sequence* s);
  };
  // The step being built and the tokens left in its budget.
  struct Draft {
    StepInput step;
    int budget = 0;
    void add_chunk(Sequence& s, int len);
    void add_decode(Sequence& s);
  };

  Residents residents() const;
  void grant_decode_slots(Residents& r);
  bool reclaim_memory(Residents& r);
  void requeue(const SequencePtr& s);  // preempted: back to the queue head, to be recomputed
  int chunk_len(const Sequence& s, int budget) const;
  void drop_expired();
  void admit(Draft& d);
  size_t pick_admission();
  bool reserve_blocks(Sequence& s);
  bool leaves_headroom(const Sequence& s) const;
  bool take_token(Sequence& s, int32_t tok, Clock::time_point now);
  void retire(const SequencePtr& s, FinishReason r);

  SchedulerConfig cfg_;
  KVCacheManager& kv_;
  std::deque<SequencePtr> waiting_;
  std::vector<SequencePtr> running_;  // admission order: back() is the youngest
  bool static_batch_open_ = true;
  SchedulerStats stats_;
};

}  // namespace le::engine
