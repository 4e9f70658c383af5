// Iteration-level scheduler. The decisions (which sequences run, in which
// order, how long each prefill chunk is, who is preempted) follow the
// reference's src/scheduler/scheduler.cpp so that a step built here packs to
// the same ragged batch; tests/golden/schedule_ref.npz holds the reference's
// own traces and the host tests replay them against this class.
#include "scheduler.h"

#include <algorithm>
#include <cassert>

namespace le::engine {

void Scheduler::add(SequencePtr seq) {
  seq->status = SeqStatus::Waiting;
  seq->t_arrival = Clock::now();
  waiting_.push_back(std::move(seq));
}

void Scheduler::abort(uint64_t id) {
  auto match = [id](const SequencePtr& s) { return s->id == id; };
  auto w = std::find_if(waiting_.begin(), waiting_.end(), match);
  if (w != waiting_.end()) {
    const SequencePtr s = *w;
    waiting_.erase(w);
    retire(s, FinishReason::Abort);
    return;
  }
  auto r = std::find_if(running_.begin(), running_.end(), match);
  if (r != running_.end()) {
    const SequencePtr s = *r;
    running_.erase(r);
    retire(s, FinishReason::Abort);
  }
}

void Scheduler::retire(const SequencePtr& s, FinishReason r) {
  s->status = SeqStatus::Finished;
  s->finish = r;
  s->t_finish = Clock::now();
  kv_.free(s->block_table);
  stats_.finished++;
}

void Scheduler::add_prefill_slice(StepInput& step, Sequence& s, int len) {
  StepSlice sl;
  sl.seq = &s;
  sl.start = s.num_computed;
  sl.len = len;
  sl.is_prefill = true;
  sl.needs_logits = s.num_computed + len == s.num_tokens();
  step.slices.push_back(sl);
  step.num_prefill_tokens += len;
  if (sl.needs_logits) step.num_logits++;
}

// Free blocks that must remain after an admission: one per resident sequence
// by default, so residents can all cross their next block boundary.
bool Scheduler::admission_fits(const Sequence& s) const {
  const int reserve = cfg_.watermark_blocks >= 0 ? cfg_.watermark_blocks
                                                 : static_cast<int>(running_.size());
  if (reserve == 0) return true;
  const int bs = kv_.block_size();
  const int fresh = KVCacheManager::blocks_needed(s.num_tokens(), bs) -
                    kv_.lookup_cached_prefix(s.tokens) / bs;
  return kv_.num_available_blocks() - fresh >= reserve;
}

bool Scheduler::admit_one(StepInput& step, int& budget) {
  if (waiting_.empty() || budget <= 0) return false;
  if (static_cast<int>(running_.size()) >= cfg_.max_num_seqs) return false;
  const size_t window = cfg_.admission_lookahead <= 1
                            ? 1
                            : std::min(waiting_.size(), static_cast<size_t>(cfg_.admission_lookahead));
  for (size_t i = 0; i < window; i++) {
    const SequencePtr s = waiting_[i];
    if (s->block_table.empty()) {
      // A request that has waited past the bound may not be overtaken.
      const bool starving = s->wait_steps >= cfg_.starvation_wait_steps;
      if (!admission_fits(*s)) {
        if (starving) break;
        continue;
      }
      const auto cached = kv_.allocate_prompt(s->block_table, s->tokens);
      if (!cached) {
        if (starving) break;
        continue;
      }
      s->num_computed = std::min(*cached, s->num_tokens() - 1);
      if (s->t_first_scheduled == Clock::time_point{}) s->t_first_scheduled = Clock::now();
    }
    const int len = std::min({s->num_tokens() - s->num_computed, budget, cfg_.prefill_chunk_size});
    if (len <= 0) return false;
    add_prefill_slice(step, *s, len);
    budget -= len;
    waiting_.erase(waiting_.begin() + static_cast<long>(i));
    running_.push_back(s);
    s->status = SeqStatus::Running;
    stats_.admitted++;
    stats_.max_wait_steps = std::max(stats_.max_wait_steps, static_cast<uint64_t>(s->wait_steps));
    return true;
  }
  return false;
}

// Frees blocks so a resident sequence can grow: first a finished member still
// holding blocks (static batching only), else the youngest resident, which is
// sent back to the queue to be recomputed.
bool Scheduler::evict_for_memory(std::vector<Sequence*>& mid_prefill, std::vector<Sequence*>& decode) {
  auto drop = [&](Sequence* v) {
    mid_prefill.erase(std::remove(mid_prefill.begin(), mid_prefill.end(), v), mid_prefill.end());
    decode.erase(std::remove(decode.begin(), decode.end(), v), decode.end());
  };
  for (size_t i = running_.size(); i-- > 0;) {
    if (!running_[i]->is_finished()) continue;
    const SequencePtr s = running_[i];
    running_.erase(running_.begin() + static_cast<long>(i));
    kv_.free(s->block_table);
    stats_.finished++;
    drop(s.get());
    return true;
  }
  if (running_.empty()) return false;
  const SequencePtr s = running_.back();
  running_.pop_back();
  kv_.free(s->block_table);
  stats_.recomputed_tokens += static_cast<uint64_t>(s->num_computed);
  s->num_computed = 0;
  s->num_preemptions++;
  s->status = SeqStatus::Waiting;
  waiting_.push_front(s);
  stats_.preemptions++;
  drop(s.get());
  return true;
}

StepInput Scheduler::schedule() {
  StepInput step;
  int budget = cfg_.max_num_batched_tokens;
  stats_.steps++;
  if (!cfg_.continuous && running_.empty()) static_batch_open_ = true;
  const bool may_admit = cfg_.continuous || static_batch_open_;

  // Residents split by phase; slices are built only after preemption settles.
  std::vector<Sequence*> mid_prefill, decode;
  for (const auto& s : running_) {
    if (s->is_finished()) continue;
    (s->prefill_done() ? decode : mid_prefill).push_back(s.get());
  }

  // Every decode token needs a slot; preempt until it has one.
  for (size_t i = 0; i < decode.size();) {
    Sequence* s = decode[i];
    if (kv_.ensure_slot(s->block_table, s->num_tokens())) {
      i++;
      continue;
    }
    if (!evict_for_memory(mid_prefill, decode)) decode.erase(decode.begin() + static_cast<long>(i));
  }

  for (Sequence* s : mid_prefill) {
    const int len = std::min({s->num_tokens() - s->num_computed, budget, cfg_.prefill_chunk_size});
    if (len > 0) {
      add_prefill_slice(step, *s, len);
      budget -= len;
    }
  }
  if (static_cast<int>(decode.size()) > budget) decode.resize(static_cast<size_t>(budget));
  budget -= static_cast<int>(decode.size());

  if (cfg_.max_queue_wait_seconds > 0 && !waiting_.empty()) {
    const auto now = Clock::now();
    std::vector<SequencePtr> expired;
    for (auto it = waiting_.begin(); it != waiting_.end();) {
      const double waited = std::chrono::duration<double>(now - (*it)->t_arrival).count();
      if (waited > cfg_.max_queue_wait_seconds && (*it)->block_table.empty()) {
        expired.push_back(*it);
        it = waiting_.erase(it);
      } else {
        ++it;
      }
    }
    for (auto& s : expired) {
      stats_.timed_out++;
      retire(s, FinishReason::Timeout);
    }
  }

  if (may_admit) {
    for (auto& w : waiting_) w->wait_steps++;
    while (admit_one(step, budget)) {
    }
    if (!cfg_.continuous && !waiting_.empty()) {
      const bool full = static_cast<int>(running_.size()) >= cfg_.max_num_seqs;
      const bool memory_bound = budget > 0 && !running_.empty();
      if (full || memory_bound) static_batch_open_ = false;
    }
    if (!waiting_.empty() && running_.empty() && decode.empty()) {
      // Nothing runs and the head still does not fit: larger than the pool.
      const SequencePtr s = waiting_.front();
      waiting_.pop_front();
      retire(s, FinishReason::Abort);
    }
  }

  for (Sequence* s : decode) {
    StepSlice sl;
    sl.seq = s;
    sl.start = s->num_computed;
    sl.len = 1;
    sl.needs_logits = true;
    step.slices.push_back(sl);
    step.num_decode_tokens++;
    step.num_logits++;
  }
  return step;
}

void Scheduler::on_step_done(const StepInput& step, const std::vector<int32_t>& sampled) {
  size_t k = 0;
  std::vector<SequencePtr> done;
  const auto now = Clock::now();
  for (const auto& sl : step.slices) {
    Sequence& s = *sl.seq;
    s.num_computed += sl.len;
    kv_.commit_computed(s.block_table, s.tokens, s.num_computed);
    if (!sl.needs_logits) continue;
    assert(k < sampled.size());
    const int32_t tok = sampled[k++];
    if (s.is_finished()) continue;  // static batching: padded member
    s.tokens.push_back(tok);
    if (s.t_first_token == Clock::time_point{}) s.t_first_token = now;
    const bool stop = !s.params.ignore_eos &&
                      std::find(s.params.stop_ids.begin(), s.params.stop_ids.end(), tok) !=
                          s.params.stop_ids.end();
    const FinishReason r = stop ? FinishReason::Stop
                           : s.num_generated() >= s.params.max_tokens ? FinishReason::Length
                                                                       : FinishReason::None;
    if (r == FinishReason::None) continue;
    s.finish = r;
    auto it = std::find_if(running_.begin(), running_.end(),
                           [&](const SequencePtr& p) { return p.get() == &s; });
    if (cfg_.continuous) {
      done.push_back(*it);
      running_.erase(it);
    } else {
      s.status = SeqStatus::Finished;
      s.t_finish = now;
    }
  }
  for (auto& s : done) retire(s, s->finish);
  if (!cfg_.continuous && !running_.empty() &&
      std::all_of(running_.begin(), running_.end(), [](const SequencePtr& p) { return p->is_finished(); })) {
    for (auto& s : running_) {
      kv_.free(s->block_table);
      stats_.finished++;
    }
    running_.clear();
    static_batch_open_ = true;
  }
}

}  // namespace le::engine
