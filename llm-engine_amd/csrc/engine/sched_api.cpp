// le_sched_trace: the scheduler and block allocator driven by a deterministic
// fake model, recorded step by step in the stream format the reference's trace
// harness uses, so the two can be compared entry for entry.
#include <cstring>
#include <vector>

#include "le_engine.h"
#include "scheduler.h"

static_assert(le::engine::kPoolShuffled == LE_POOL_SHUFFLED, "pool preparation codes");

extern "C" int64_t le_sched_trace(int num_blocks, int block_size, int prefix_caching,
                                  const le_sched_config* cfg, int fragment_blocks, int n_seqs,
                                  const int32_t* prompt_lens, const int32_t* prompts_flat,
                                  const int32_t* max_tokens, int max_steps, int32_t* out,
                                  int64_t out_cap) {
  using namespace le::engine;
  if (!cfg || n_seqs < 0) return 0;
  try {
    KVCacheManager kv(num_blocks, block_size, prefix_caching != 0);
    std::vector<BlockTable> held = prepare_pool(kv, fragment_blocks);
    SchedulerConfig sc;
    sc.continuous = cfg->continuous != 0;
    sc.max_num_seqs = cfg->max_num_seqs;
    sc.max_num_batched_tokens = cfg->max_num_batched_tokens;
    sc.prefill_chunk_size = cfg->prefill_chunk_size;
    sc.admission_lookahead = cfg->admission_lookahead;
    sc.starvation_wait_steps = cfg->starvation_wait_steps;
    sc.watermark_blocks = cfg->watermark_blocks;
    sc.max_queue_wait_seconds = cfg->max_queue_wait_seconds;
    Scheduler sch(sc, kv);
    std::vector<SequencePtr> seqs;
    size_t off = 0;
    for (int i = 0; i < n_seqs; i++) {
      auto s = std::make_shared<Sequence>();
      s->id = static_cast<uint64_t>(i);
      s->tokens.assign(prompts_flat + off, prompts_flat + off + prompt_lens[i]);
      off += static_cast<size_t>(prompt_lens[i]);
      s->prompt_len = prompt_lens[i];
      s->params.max_tokens = max_tokens[i];
      s->params.ignore_eos = true;
      sch.add(s);
      seqs.push_back(s);
    }
    std::vector<int32_t> rec;
    int32_t next = 1000;
    for (int step = 0; step < max_steps && sch.has_work(); step++) {
      StepInput st = sch.schedule();
      if (st.empty()) break;
      rec.push_back(static_cast<int32_t>(st.slices.size()));
      std::vector<int32_t> sampled;
      for (const auto& sl : st.slices) {
        rec.push_back(static_cast<int32_t>(sl.seq->id));
        rec.push_back(sl.start);
        rec.push_back(sl.len);
        rec.push_back(sl.needs_logits ? 1 : 0);
        rec.push_back(sl.is_prefill ? 1 : 0);
        rec.push_back(sl.seq->block_table.num_blocks());
        for (BlockId b : sl.seq->block_table.blocks) rec.push_back(b);
        if (sl.needs_logits) sampled.push_back(next++);
      }
      sch.on_step_done(st, sampled);
    }
    rec.push_back(-1);
    for (auto& s : seqs) {
      rec.push_back(s->num_tokens());
      for (int32_t t : s->tokens) rec.push_back(t);
    }
    for (BlockTable& bt : held) kv.free(bt);
    if (static_cast<int64_t>(rec.size()) > out_cap) return -static_cast<int64_t>(rec.size());
    std::memcpy(out, rec.data(), rec.size() * sizeof(int32_t));
    return static_cast<int64_t>(rec.size());
  } catch (...) {
    return 0;
  }
}

namespace {
struct SchedHandle {
  le::engine::KVCacheManager kv;
  le::engine::Scheduler sch;
  std::vector<le::engine::BlockTable> held;
  std::vector<le::engine::SequencePtr> seqs;
  le::engine::StepInput last;
  SchedHandle(int nb, int bs, bool prefix, const le::engine::SchedulerConfig& c)
      : kv(nb, bs, prefix), sch(c, kv) {}
  ~SchedHandle() {
    for (le::engine::BlockTable& bt : held) kv.free(bt);
  }
};

le::engine::SchedulerConfig to_config(const le_sched_config* cfg) {
  le::engine::SchedulerConfig sc;
  sc.continuous = cfg->continuous != 0;
  sc.max_num_seqs = cfg->max_num_seqs;
  sc.max_num_batched_tokens = cfg->max_num_batched_tokens;
  sc.prefill_chunk_size = cfg->prefill_chunk_size;
  sc.admission_lookahead = cfg->admission_lookahead;
  sc.starvation_wait_steps = cfg->starvation_wait_steps;
  sc.watermark_blocks = cfg->watermark_blocks;
  sc.max_queue_wait_seconds = cfg->max_queue_wait_seconds;
  return sc;
}
}  // namespace

struct le_sched {
  SchedHandle h;
  le_sched(int nb, int bs, bool prefix, const le::engine::SchedulerConfig& c) : h(nb, bs, prefix, c) {}
};

extern "C" {

le_sched* le_sched_create(int num_blocks, int block_size, int prefix_caching,
                          const le_sched_config* cfg, int fragment_blocks) {
  if (!cfg || num_blocks <= 0 || block_size <= 0) return nullptr;
  try {
    auto* s = new le_sched(num_blocks, block_size, prefix_caching != 0, to_config(cfg));
    s->h.held = le::engine::prepare_pool(s->h.kv, fragment_blocks);
    return s;
  } catch (...) {
    return nullptr;
  }
}

void le_sched_destroy(le_sched* s) { delete s; }

int le_sched_add(le_sched* s, int64_t id, const int32_t* prompt, int n, int max_tokens) {
  if (!s || !prompt || n <= 0) return LE_EINVAL;
  auto q = std::make_shared<le::engine::Sequence>();
  q->id = static_cast<uint64_t>(id);
  q->tokens.assign(prompt, prompt + n);
  q->prompt_len = n;
  q->params.max_tokens = max_tokens;
  q->params.ignore_eos = true;
  s->h.seqs.push_back(q);
  s->h.sch.add(q);
  return LE_OK;
}

int le_sched_has_work(const le_sched* s) { return s && s->h.sch.has_work() ? 1 : 0; }

int le_sched_step(le_sched* s, le_step_slice* out, int cap, int* n_slices) {
  if (!s || !n_slices) return LE_EINVAL;
  s->h.last = s->h.sch.schedule();
  const auto& sl = s->h.last.slices;
  *n_slices = static_cast<int>(sl.size());
  if (static_cast<int>(sl.size()) > cap) return LE_ENOSPACE;
  for (size_t i = 0; i < sl.size(); i++) {
    const le::engine::Sequence& q = *sl[i].seq;
    out[i] = le_step_slice{static_cast<int64_t>(q.id), sl[i].start, sl[i].len, sl[i].needs_logits ? 1 : 0,
                           q.block_table.num_blocks(), q.block_table.blocks.data(), q.tokens.data()};
  }
  return LE_OK;
}

int le_sched_done(le_sched* s, const int32_t* sampled, int n) {
  if (!s || n != s->h.last.num_logits || (n > 0 && !sampled)) return LE_EINVAL;
  s->h.sch.on_step_done(s->h.last, std::vector<int32_t>(sampled, sampled + n));
  s->h.last = le::engine::StepInput{};
  return LE_OK;
}

int le_sched_generated(const le_sched* s, int64_t id, int32_t* out, int cap) {
  if (!s) return LE_EINVAL;
  for (const auto& q : s->h.seqs) {
    if (static_cast<int64_t>(q->id) != id) continue;
    const int n = q->num_generated();
    for (int j = 0; j < n && j < cap; j++) out[j] = q->tokens[q->prompt_len + j];
    return n;
  }
  return LE_EINVAL;
}

}  // extern "C"
