// Continuous-batching scheduler over the step runner: the request lifecycle of the reference
// Engine (src/engine.cpp:45-184) without a model around it. A request is a prompt length and a
// number of tokens to generate; "sampling" a token only advances the sequence, because the
// attention step is all this library runs.
//
//   * admission (same contract as reference :62-91): requests start in arrival order; the pages of
//     the whole request, min(prompt + max_new, max_context) tokens, are reserved when it starts,
//     so no sequence is ever preempted; a request that could not run even alone is refused (here
//     as soon as it reaches the head of the queue, rather than after the engine has drained);
//   * one iteration = at most one prefill chunk (the oldest sequence still consuming its prompt)
//     plus one decode row for every sequence that has a sampled token not yet in the cache;
//   * policy 0 (reference :133-182): the chunk runs as its own prefill launch, then one decode
//     launch whose rows already include a sequence whose prompt the chunk just completed;
//   * policy 1 (mixed): the decode rows of earlier iterations and the chunk form one ragged batch
//     (decode rows first, then the chunk) and run as one attention launch per layer; a sequence
//     whose prompt completes decodes from the next iteration on;
//   * a sequence finishes once it has sampled max_new tokens or reaches the context limit; its
//     slot and pages return to the free lists (reference :93-108).
// plan() only decides; execute() launches and then advances the sequences, so a caller can fill
// the planned proj rows in between.
#include <algorithm>
#include <deque>
#include <new>
#include <vector>

#include "q38a_runtime.h"
#include "common.hpp"

namespace {

struct Sequence {
  int id = -1;
  int prompt = 0, max_new = 0;
  int slot = -1;
  int prefilled = 0;   // prompt tokens in the cache
  int position = 0;    // next position to write
  int sampled = 0;     // tokens generated so far
  bool decoding() const { return prefilled == prompt; }
};

}  // namespace

struct q38a_engine {
  q38a_runner* runner = nullptr;
  q38a_engine_options opt{};
  int max_context = 0;
  std::deque<Sequence> waiting;
  std::vector<Sequence> active;
  std::vector<int> free_slots;
  std::vector<int> finished;
  q38a_engine_stats stats{};
  int next_id = 0;
  // the planned iteration
  bool planned = false;
  int chunk = -1, chunk_n = 0;  // index into `active` and tokens of the prefill chunk
  std::vector<int> rows;        // indices into `active` of the decode rows
  std::vector<q38a_plan_entry> plan;
};

using namespace q38a;

namespace {

void finish(q38a_engine* e, Sequence& s, bool failed) {
  if (s.slot >= 0) {
    (void)q38a_kv_cache_release(q38a_runner_kv(e->runner), s.slot);
    e->free_slots.push_back(s.slot);
    s.slot = -1;
  }
  e->finished.push_back(failed ? -1 - s.id : s.id);
  if (failed) ++e->stats.requests_failed;
  else ++e->stats.requests_done;
}

// One sampled token: returns true when the sequence is done (reference engine.cpp:115-131).
bool on_sample(q38a_engine* e, Sequence& s) {
  ++s.sampled;
  if (s.sampled >= s.max_new || s.position >= e->max_context) {
    finish(e, s, false);
    return true;
  }
  return false;
}

// Pages a request holds from admission to its end: its prompt plus every token it may generate,
// capped by the context limit.
int footprint_pages(const q38a_engine* e, const Sequence& s) {
  const long long tokens = std::min<long long>(static_cast<long long>(s.prompt) + s.max_new, e->max_context);
  return int((tokens + kPageTokens - 1) / kPageTokens);
}

// Pages that are free now or held by running sequences, i.e. free once every one of them ends.
int reclaimable_pages(q38a_engine* e) {
  q38a_kv_cache* kv = q38a_runner_kv(e->runner);
  int pages = q38a_kv_cache_free_pages(kv);
  for (const Sequence& s : e->active) pages += q38a_kv_cache_pages_of(kv, s.slot);
  return pages;
}

// Moves requests from the head of the queue into `active`, strictly in arrival order. A request is
// refused outright when it can never run (its prompt reaches the context limit, or its footprint
// exceeds what the pool holds even with nothing else running); the head request otherwise waits
// until a slot and its whole footprint are free, and nothing behind it overtakes it.
int admit(q38a_engine* e) {
  q38a_kv_cache* kv = q38a_runner_kv(e->runner);
  while (!e->waiting.empty()) {
    Sequence head = e->waiting.front();
    const int pages = footprint_pages(e, head);
    if (head.prompt >= e->max_context || pages > reclaimable_pages(e)) {
      e->waiting.pop_front();
      finish(e, head, true);
      continue;
    }
    if (e->free_slots.empty() || pages > q38a_kv_cache_free_pages(kv)) break;
    head.slot = e->free_slots.back();
    int granted = 0;
    if (int rc = q38a_kv_cache_ensure(kv, head.slot, pages * kPageTokens, &granted)) return rc;
    if (!granted) return set_error(Q38A_ERR_CAPACITY, "engine: %d free pages did not cover %d", q38a_kv_cache_free_pages(kv), pages);
    e->free_slots.pop_back();
    e->waiting.pop_front();
    e->active.push_back(head);
  }
  return Q38A_OK;
}

}  // namespace

extern "C" {

int q38a_engine_create(q38a_runner* runner, const q38a_engine_options* opt, q38a_engine** out) {
  clear_error();
  if (!runner || !opt || !out) return set_error(Q38A_ERR_INVALID, "engine_create: null argument");
  *out = nullptr;
  q38a_runner_buffers buf{};
  if (int rc = q38a_runner_get_buffers(runner, &buf)) return rc;
  if (opt->prefill_chunk <= 0 || opt->prefill_chunk > buf.rows - buf.prefill_row)
    return set_error(Q38A_ERR_INVALID, "engine_create: prefill_chunk %d outside [1, %d]", opt->prefill_chunk,
                     buf.rows - buf.prefill_row);
  auto* e = new (std::nothrow) q38a_engine();
  if (!e) return set_error(Q38A_ERR_INVALID, "engine_create: out of host memory");
  e->runner = runner;
  e->opt = *opt;
  // the runner's context limit: positions the KV block table can address
  q38a_kv_cache_desc d{};
  if (int rc = q38a_kv_cache_desc_get(q38a_runner_kv(runner), &d)) {
    delete e;
    return rc;
  }
  e->max_context = d.max_pages_per_seq * kPageTokens;
  for (int s = q38a_runner_num_slots(runner) - 1; s >= 0; --s) e->free_slots.push_back(s);
  *out = e;
  return Q38A_OK;
}

void q38a_engine_destroy(q38a_engine* e) { delete e; }

int q38a_engine_submit(q38a_engine* e, int prompt_tokens, int max_new_tokens) {
  clear_error();
  if (!e) return -set_error(Q38A_ERR_INVALID, "engine_submit: null engine");
  if (prompt_tokens <= 0 || max_new_tokens <= 0)
    return -set_error(Q38A_ERR_INVALID, "engine_submit: empty prompt or nothing to generate");
  Sequence s;
  s.id = e->next_id++;
  s.prompt = prompt_tokens;
  s.max_new = max_new_tokens;
  e->waiting.push_back(s);
  return s.id;
}

int q38a_engine_idle(const q38a_engine* e) { return !e || (e->waiting.empty() && e->active.empty()); }

int q38a_engine_plan(q38a_engine* e, q38a_plan_entry* entries, int cap, int* n) {
  clear_error();
  if (!e || !n || (cap > 0 && !entries)) return set_error(Q38A_ERR_INVALID, "engine_plan: bad arguments");
  *n = 0;
  if (int rc = admit(e)) return rc;
  e->planned = false;
  e->chunk = -1;
  e->chunk_n = 0;
  e->rows.clear();
  e->plan.clear();
  if (e->active.empty()) return Q38A_OK;
  q38a_runner_buffers buf{};
  if (int rc = q38a_runner_get_buffers(e->runner, &buf)) return rc;
  for (int i = 0; i < int(e->active.size()); ++i) {
    const Sequence& s = e->active[size_t(i)];
    if (s.decoding()) continue;
    e->chunk = i;
    e->chunk_n = std::min(e->opt.prefill_chunk, s.prompt - s.prefilled);
    break;
  }
  const int slots = q38a_runner_num_slots(e->runner);
  for (int i = 0; i < int(e->active.size()) && int(e->rows.size()) < slots; ++i) {
    const Sequence& s = e->active[size_t(i)];
    if (s.decoding() && s.sampled > 0) {
      e->rows.push_back(i);
    } else if (i == e->chunk && !e->opt.mixed && s.prefilled + e->chunk_n == s.prompt) {
      // policy 0: the chunk completes the prompt and samples; the sequence decodes right after
      // unless that first token already finishes it
      const bool done = s.max_new <= 1 || s.prompt >= e->max_context;
      if (!done) e->rows.push_back(i);
    }
  }
  int row = 0;
  for (int i : e->rows) {
    const Sequence& s = e->active[size_t(i)];
    const int pos = i == e->chunk ? s.prompt : s.position;
    e->plan.push_back(q38a_plan_entry{s.id, s.slot, pos, 1, row++});
  }
  if (e->chunk >= 0) {
    const Sequence& s = e->active[size_t(e->chunk)];
    e->plan.push_back(q38a_plan_entry{s.id, s.slot, s.prefilled, e->chunk_n, e->opt.mixed ? row : buf.prefill_row});
  }
  e->planned = !e->plan.empty();
  *n = int(e->plan.size());
  for (int i = 0; i < cap && i < *n; ++i) entries[i] = e->plan[size_t(i)];
  return Q38A_OK;
}

int q38a_engine_execute(q38a_engine* e, void* stream) {
  clear_error();
  if (!e) return set_error(Q38A_ERR_INVALID, "engine_execute: null engine");
  if (!e->planned) return set_error(Q38A_ERR_INVALID, "engine_execute: nothing planned");
  e->planned = false;
  const int ndec = int(e->rows.size());
  std::vector<q38a_step_seq> dec;
  for (int k = 0; k < ndec; ++k) dec.push_back(q38a_step_seq{e->plan[size_t(k)].slot, e->plan[size_t(k)].pos0, 1});
  if (e->opt.mixed) {
    std::vector<q38a_step_seq> all = dec;
    if (e->chunk >= 0) {
      const q38a_plan_entry& c = e->plan.back();
      all.push_back(q38a_step_seq{c.slot, c.pos0, c.n});
    }
    if (int rc = q38a_runner_step(e->runner, all.data(), int(all.size()), stream)) return rc;
    ++e->stats.launches;
  } else {
    if (e->chunk >= 0) {
      const q38a_plan_entry& c = e->plan.back();
      if (int rc = q38a_runner_prefill(e->runner, c.slot, c.pos0, c.n, stream)) return rc;
      ++e->stats.launches;
    }
    if (ndec) {
      if (int rc = q38a_runner_decode(e->runner, dec.data(), ndec, stream)) return rc;
      ++e->stats.launches;
    }
  }
  ++e->stats.iterations;
  // advance: the chunk first (it precedes the decode launch in policy 0), then the decode rows
  std::vector<char> gone(e->active.size(), 0);
  if (e->chunk >= 0) {
    Sequence& s = e->active[size_t(e->chunk)];
    s.prefilled += e->chunk_n;
    s.position = s.prefilled;
    e->stats.prefill_tokens += e->chunk_n;
    if (s.decoding() && on_sample(e, s)) gone[size_t(e->chunk)] = 1;
  }
  for (int i : e->rows) {
    Sequence& s = e->active[size_t(i)];
    if (gone[size_t(i)]) continue;
    s.position += 1;  // this step appended the row's token at its position
    ++e->stats.decode_tokens;
    if (on_sample(e, s)) gone[size_t(i)] = 1;
  }
  std::vector<Sequence> keep;
  for (size_t i = 0; i < e->active.size(); ++i)
    if (!gone[i]) keep.push_back(e->active[i]);
  e->active.swap(keep);
  return Q38A_OK;
}

int q38a_engine_get_stats(const q38a_engine* e, q38a_engine_stats* out) {
  clear_error();
  if (!e || !out) return set_error(Q38A_ERR_INVALID, "engine_get_stats: null argument");
  *out = e->stats;
  return Q38A_OK;
}

int q38a_engine_take_finished(q38a_engine* e, int* ids, int cap, int* n) {
  clear_error();
  if (!e || !n || (cap > 0 && !ids)) return set_error(Q38A_ERR_INVALID, "engine_take_finished: bad arguments");
  *n = int(e->finished.size());
  const int k = std::min(cap, *n);
  for (int i = 0; i < k; ++i) ids[i] = e->finished[size_t(i)];
  e->finished.erase(e->finished.begin(), e->finished.begin() + k);
  return Q38A_OK;
}

int q38a_engine_position(const q38a_engine* e, int request_id) {
  if (!e) return -1;
  for (const Sequence& s : e->active)
    if (s.id == request_id) return s.position;
  return -1;
}

}  // extern "C"
