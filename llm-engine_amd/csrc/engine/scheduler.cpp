// Iteration-level scheduler: builds each step's ragged batch.
//
// The decisions are the reference's (src/scheduler/scheduler.cpp; behaviour
// pinned by the reference's own step-by-step traces in
// tests/golden/schedule_ref.npz, which the host tests replay here):
//   * a step holds the residents' prefill chunks first, then one decode
//     token per resident whose prompt is done, then chunks of newly admitted
//     requests, all under one token budget and a chunk-size cap;
//   * a decode token that finds no free block first releases a finished
//     member of a static batch, else preempts the youngest resident, which
//     goes back to the queue head to be recomputed;
//   * admission is first come first served, optionally looking a few requests
//     down the queue, except that a request waiting past the starvation bound
//     may not be overtaken; an admission must leave a free-block headroom;
//   * requests waiting past a deadline are dropped; in static-batching mode a
//     batch closes once full (or memory-bound) and reopens when it drains.
//
// The step is built in phases over explicit state: the residents by phase
// (Residents), the draft step and its remaining budget (Draft).
#include "scheduler.h"

#include <algorithm>
#include <cassert>

namespace le::engine {

namespace {
constexpr size_t kNone = static_cast<size_t>(-1);
}

// ---- step drafting ----

void Scheduler::Draft::add_chunk(Sequence& s, int len) {
  StepSlice sl;
  sl.seq = &s;
  sl.start = s.num_computed;
  sl.len = len;
  sl.is_prefill = true;
  sl.needs_logits = sl.start + len == s.num_tokens();  // the chunk reaches the last token
  step.slices.push_back(sl);
  step.num_prefill_tokens += len;
  step.num_logits += sl.needs_logits ? 1 : 0;
  budget -= len;
}

void Scheduler::Draft::add_decode(Sequence& s) {
  StepSlice sl;
  sl.seq = &s;
  sl.start = s.num_computed;
  sl.len = 1;
  sl.needs_logits = true;
  step.slices.push_back(sl);
  step.num_decode_tokens++;
  step.num_logits++;
}

void Scheduler::Residents::remove(const Sequence* s) {
  for (auto* list : {&prefilling, &decoding}) list->erase(std::remove(list->begin(), list->end(), s), list->end());
}

int Scheduler::chunk_len(const Sequence& s, int budget) const {
  return std::min({s.num_tokens() - s.num_computed, budget, cfg_.prefill_chunk_size});
}

// ---- queue operations ----

void Scheduler::add(SequencePtr seq) {
  seq->status = SeqStatus::Waiting;
  seq->t_arrival = Clock::now();
  waiting_.push_back(std::move(seq));
}

void Scheduler::retire(const SequencePtr& s, FinishReason r) {
  s->status = SeqStatus::Finished;
  s->finish = r;
  s->t_finish = Clock::now();
  kv_.free(s->block_table);
  stats_.finished++;
}

void Scheduler::abort(uint64_t id) {
  const auto is_id = [id](const SequencePtr& s) { return s->id == id; };
  SequencePtr found;
  if (auto w = std::find_if(waiting_.begin(), waiting_.end(), is_id); w != waiting_.end()) {
    found = *w;
    waiting_.erase(w);
  } else if (auto r = std::find_if(running_.begin(), running_.end(), is_id); r != running_.end()) {
    found = *r;
    running_.erase(r);
  }
  if (found) retire(found, FinishReason::Abort);
}

void Scheduler::requeue(const SequencePtr& s) {
  kv_.free(s->block_table);
  stats_.recomputed_tokens += static_cast<uint64_t>(s->num_computed);
  stats_.preemptions++;
  s->num_computed = 0;
  s->num_preemptions++;
  s->status = SeqStatus::Waiting;
  waiting_.push_front(s);
}

void Scheduler::drop_expired() {
  if (cfg_.max_queue_wait_seconds <= 0 || waiting_.empty()) return;
  const auto now = Clock::now();
  std::deque<SequencePtr> keep;
  std::vector<SequencePtr> expired;
  for (const SequencePtr& s : waiting_) {
    const double waited = std::chrono::duration<double>(now - s->t_arrival).count();
    const bool late = waited > cfg_.max_queue_wait_seconds && s->block_table.empty();
    (late ? expired.emplace_back(s) : keep.emplace_back(s));
  }
  waiting_.swap(keep);
  for (const SequencePtr& s : expired) {
    stats_.timed_out++;
    retire(s, FinishReason::Timeout);
  }
}

// ---- residents and memory ----

Scheduler::Residents Scheduler::residents() const {
  Residents r;
  for (const SequencePtr& s : running_)
    if (!s->is_finished())  // static batching keeps finished members resident
      (s->prefill_done() ? r.decoding : r.prefilling).push_back(s.get());
  return r;
}

// Picks the resident whose blocks return to the pool. Only static batching
// leaves a finished member resident (it holds its place to mimic padded
// generation); such a member is released outright, since nothing reads its
// cache again and a preemption would put it back in the queue with its token
// cap already spent. With none, the newest live resident is preempted and
// recomputed later.
bool Scheduler::reclaim_memory(Residents& r) {
  const auto drained = std::find_if(running_.rbegin(), running_.rend(),
                                    [](const SequencePtr& s) { return s->is_finished(); });
  SequencePtr victim;
  if (drained != running_.rend()) {
    victim = *drained;
    running_.erase(std::next(drained).base());
    kv_.free(victim->block_table);
    stats_.finished++;
  } else if (!running_.empty()) {
    victim = running_.back();
    running_.pop_back();
    requeue(victim);
  } else {
    return false;
  }
  r.remove(victim.get());
  return true;
}

// Every decode token needs a cache slot. When the pool is out of blocks,
// memory is reclaimed and the same token is tried again (the victim may be
// that token's own sequence, which then leaves the list).
void Scheduler::grant_decode_slots(Residents& r) {
  size_t i = 0;
  while (i < r.decoding.size()) {
    Sequence& s = *r.decoding[i];
    if (kv_.ensure_slot(s.block_table, s.num_tokens())) {
      i++;
    } else if (!reclaim_memory(r)) {
      r.decoding.erase(r.decoding.begin() + static_cast<std::ptrdiff_t>(i));
    }
  }
}

// ---- admission ----

// Would `s` leave the headroom the residents need to reach their next block
// boundary (one block each, or the configured watermark)? Blocks its prompt
// can reuse from the prefix cache cost nothing.
bool Scheduler::leaves_headroom(const Sequence& s) const {
  const int headroom = cfg_.watermark_blocks >= 0 ? cfg_.watermark_blocks : static_cast<int>(running_.size());
  if (headroom == 0) return true;
  const int bs = kv_.block_size();
  const int fresh = KVCacheManager::blocks_needed(s.num_tokens(), bs) - kv_.lookup_cached_prefix(s.tokens) / bs;
  return kv_.num_available_blocks() - fresh >= headroom;
}

bool Scheduler::reserve_blocks(Sequence& s) {
  if (!leaves_headroom(s)) return false;
  const std::optional<int> cached = kv_.allocate_prompt(s.block_table, s.tokens);
  if (!cached) return false;
  // At least the last prompt token is computed, to produce its logits.
  s.num_computed = std::min(*cached, s.num_tokens() - 1);
  if (s.t_first_scheduled == Clock::time_point{}) s.t_first_scheduled = Clock::now();
  return true;
}

// Index of the request to admit next (its blocks reserved), or kNone.
size_t Scheduler::pick_admission() {
  const size_t window = cfg_.admission_lookahead > 1
                            ? std::min(waiting_.size(), static_cast<size_t>(cfg_.admission_lookahead))
                            : 1;
  for (size_t i = 0; i < window; i++) {
    Sequence& s = *waiting_[i];
    if (!s.block_table.empty() || reserve_blocks(s)) return i;
    if (s.wait_steps >= cfg_.starvation_wait_steps) break;  // may not be overtaken
  }
  return kNone;
}

void Scheduler::admit(Draft& d) {
  while (!waiting_.empty() && d.budget > 0 && static_cast<int>(running_.size()) < cfg_.max_num_seqs) {
    const size_t i = pick_admission();
    if (i == kNone) return;
    const SequencePtr s = waiting_[i];
    const int len = chunk_len(*s, d.budget);
    if (len <= 0) return;
    d.add_chunk(*s, len);
    waiting_.erase(waiting_.begin() + static_cast<std::ptrdiff_t>(i));
    running_.push_back(s);
    s->status = SeqStatus::Running;
    stats_.admitted++;
    stats_.max_wait_steps = std::max<uint64_t>(stats_.max_wait_steps, static_cast<uint64_t>(s->wait_steps));
  }
}

// ---- the step ----

StepInput Scheduler::schedule() {
  stats_.steps++;
  Draft d;
  d.budget = cfg_.max_num_batched_tokens;
  if (!cfg_.continuous && running_.empty()) static_batch_open_ = true;

  // Residents first: slots for their decode tokens (this may preempt some of
  // them, so no slice is drafted before it settles), then their chunks.
  Residents r = residents();
  grant_decode_slots(r);
  for (Sequence* s : r.prefilling) {
    const int len = chunk_len(*s, d.budget);
    if (len > 0) d.add_chunk(*s, len);
  }
  if (static_cast<int>(r.decoding.size()) > d.budget) r.decoding.resize(static_cast<size_t>(d.budget));
  d.budget -= static_cast<int>(r.decoding.size());

  drop_expired();
  if (cfg_.continuous || static_batch_open_) {
    for (const SequencePtr& w : waiting_) w->wait_steps++;
    admit(d);
    if (!cfg_.continuous && !waiting_.empty()) {
      // A static batch stops accepting members once it holds max_num_seqs or
      // the pool refused a request while budget was left over.
      const bool full = static_cast<int>(running_.size()) >= cfg_.max_num_seqs;
      if (full || (d.budget > 0 && !running_.empty())) static_batch_open_ = false;
    }
    if (!waiting_.empty() && running_.empty() && r.decoding.empty()) {
      // An empty engine that still cannot place the queue head never will
      // (the prompt needs more blocks than the pool has): abort that request
      // so the queue keeps moving.
      const SequencePtr s = waiting_.front();
      waiting_.pop_front();
      retire(s, FinishReason::Abort);
    }
  }

  for (Sequence* s : r.decoding) d.add_decode(*s);
  return std::move(d.step);
}

// Appends a sampled token; true when the sequence is now complete.
bool Scheduler::take_token(Sequence& s, int32_t tok, Clock::time_point now) {
  s.tokens.push_back(tok);
  if (s.t_first_token == Clock::time_point{}) s.t_first_token = now;
  const auto& stops = s.params.stop_ids;
  const bool stop = !s.params.ignore_eos && std::find(stops.begin(), stops.end(), tok) != stops.end();
  s.finish = stop ? FinishReason::Stop
             : s.num_generated() >= s.params.max_tokens ? FinishReason::Length
                                                         : FinishReason::None;
  return s.finish != FinishReason::None;
}

void Scheduler::on_step_done(const StepInput& step, const std::vector<int32_t>& sampled) {
  const auto now = Clock::now();
  // The step's K/V are computed: advance every slice's sequence and publish
  // its newly completed blocks.
  for (const StepSlice& sl : step.slices) {
    sl.seq->num_computed += sl.len;
    kv_.commit_computed(sl.seq->block_table, sl.seq->tokens, sl.seq->num_computed);
  }
  // Sampled tokens, in the order of the slices that asked for logits.
  std::vector<Sequence*> complete;
  size_t k = 0;
  for (const StepSlice& sl : step.slices) {
    if (!sl.needs_logits) continue;
    assert(k < sampled.size());
    const int32_t tok = sampled[k++];
    Sequence& s = *sl.seq;
    if (s.is_finished()) continue;  // a finished static-batch member: padding
    if (take_token(s, tok, now)) complete.push_back(&s);
  }
  for (Sequence* s : complete) {
    const auto it = std::find_if(running_.begin(), running_.end(),
                                 [s](const SequencePtr& p) { return p.get() == s; });
    if (!cfg_.continuous) {  // keeps its slot and blocks until the batch drains
      s->status = SeqStatus::Finished;
      s->t_finish = now;
      continue;
    }
    const SequencePtr owner = *it;
    running_.erase(it);
    retire(owner, owner->finish);
  }
  const bool drained = !running_.empty() && std::all_of(running_.begin(), running_.end(),
                                                        [](const SequencePtr& p) { return p->is_finished(); });
  if (!cfg_.continuous && drained) {
    for (const SequencePtr& s : running_) {
      kv_.free(s->block_table);
      stats_.finished++;
    }
    running_.clear();
    static_batch_open_ = true;
  }
}

}  // namespace le::engine
