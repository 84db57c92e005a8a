// Step runner of the full-attention layers: the launch interface of the reference ModelRunner
// (src/model_runner.cpp:47-67 MetaLayout, :326-357 the attention branch of forward, :488-560 the
// bucketed decode graph), rebuilt around the q38a kernels.
//
//   * step metadata (tok_pos, tok_seq, seq_start, seq_slot, seq_pos0) lives in one pinned host
//     buffer and one device buffer of the same layout and travels with a single H2D copy per step;
//   * every step runs, for each attention layer, the fused norm/RoPE/append and then attention
//     (decode, prefill or the ragged mixed launch) on the runner's own proj/out/q16 buffers;
//   * a decode step is padded to its bucket with a private dummy slot at position 0 and, with
//     graphs on, replays one hipGraph per bucket (captured on a private stream, launched on the
//     caller's): the captured metadata copy reads the pinned
//     buffer at launch time, so refilling that buffer is all a replay needs. A step waits for the
//     previous step's copy before it overwrites the pinned buffer.
// Nothing here allocates after creation.
#include <algorithm>
#include <map>
#include <new>
#include <vector>

#include "q38a_runtime.h"
#include "common.hpp"

namespace {

constexpr int kBuckets[] = {1, 2, 4, 8, 12, 16, 24, 32, 48, 64};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct MetaLayout {
  size_t tok_pos = 0, tok_seq = 0, seq_start = 0, seq_slot = 0, seq_pos0 = 0, bytes = 0;
  explicit MetaLayout(int rows = 1) {
    size_t o = 0;
    auto take = [&](size_t n) {
      const size_t at = o;
      o = align256(o + n * sizeof(int32_t));
      return at;
    };
    tok_pos = take(size_t(rows));
    tok_seq = take(size_t(rows));
    seq_start = take(size_t(rows) + 1);
    seq_slot = take(size_t(rows));
    seq_pos0 = take(size_t(rows));
    bytes = o;
  }
};

}  // namespace

struct q38a_runner {
  q38a_runner_options opt{};
  int ld = 0, rows = 0, prefill_row = 0, dummy_slot = 0;
  q38a_kv_cache* kv = nullptr;
  uint16_t* proj = nullptr;
  uint16_t* out = nullptr;
  uint16_t* q16 = nullptr;
  float* rope = nullptr;
  float* scratch = nullptr;   // decode split partials
  float* rscratch = nullptr;  // ragged launches: counters at the front must stay zero between launches,
                              // so they do not share the decode launch's partials
  MetaLayout meta;
  uint8_t* meta_dev = nullptr;
  uint8_t* meta_host = nullptr;
  hipEvent_t meta_done = nullptr;
  bool meta_pending = false;
  hipStream_t capture_stream = nullptr;  // graphs are captured here (the caller's may be the null stream)
  std::map<int, hipGraphExec_t> graphs;

  ~q38a_runner() {
    for (auto& g : graphs) (void)hipGraphExecDestroy(g.second);
    if (meta_done) (void)hipEventDestroy(meta_done);
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
    if (meta_host) (void)hipHostFree(meta_host);
    for (void* p : {static_cast<void*>(meta_dev), static_cast<void*>(proj), static_cast<void*>(out),
                    static_cast<void*>(q16), static_cast<void*>(rope), static_cast<void*>(scratch), static_cast<void*>(rscratch)})
      if (p) (void)hipFree(p);
    if (kv) q38a_kv_cache_destroy(kv);
  }

  int32_t* host_i32(size_t off) { return reinterpret_cast<int32_t*>(meta_host + off); }
  const int32_t* dev_i32(size_t off) const { return reinterpret_cast<const int32_t*>(meta_dev + off); }

  q38a_batch_desc batch(int num_seqs, int num_tokens, int max_run) const {
    return q38a_batch_desc{num_seqs, num_tokens, max_run, dev_i32(meta.seq_start), dev_i32(meta.seq_slot),
                           dev_i32(meta.seq_pos0), dev_i32(meta.tok_pos), dev_i32(meta.tok_seq)};
  }
};

using namespace q38a;

namespace {

// Waits until the previous step has copied the pinned metadata (the copy may still be queued).
int wait_meta(q38a_runner* r) {
  if (!r->meta_pending) return Q38A_OK;
  r->meta_pending = false;
  return check_hip(hipEventSynchronize(r->meta_done), "runner: wait for the metadata copy");
}

// Fills the pinned metadata for `seqs` (packed in order from token row 0).
void fill_meta(q38a_runner* r, const q38a_step_seq* seqs, int num_seqs) {
  int32_t* tok_pos = r->host_i32(r->meta.tok_pos);
  int32_t* tok_seq = r->host_i32(r->meta.tok_seq);
  int32_t* seq_start = r->host_i32(r->meta.seq_start);
  int32_t* seq_slot = r->host_i32(r->meta.seq_slot);
  int32_t* seq_pos0 = r->host_i32(r->meta.seq_pos0);
  int t = 0;
  for (int b = 0; b < num_seqs; ++b) {
    seq_start[b] = t;
    seq_slot[b] = seqs[b].slot;
    seq_pos0[b] = seqs[b].pos0;
    for (int i = 0; i < seqs[b].n; ++i, ++t) {
      tok_pos[t] = seqs[b].pos0 + i;
      tok_seq[t] = b;
    }
  }
  seq_start[num_seqs] = t;
}

int upload_meta(q38a_runner* r, hipStream_t s) {
  return check_hip(hipMemcpyAsync(r->meta_dev, r->meta_host, r->meta.bytes, hipMemcpyHostToDevice, s),
                   "runner: metadata upload");
}

int mark_meta(q38a_runner* r, hipStream_t s) {
  if (int rc = check_hip(hipEventRecord(r->meta_done, s), "runner: event record")) return rc;
  r->meta_pending = true;
  return Q38A_OK;
}

// Checks slots, positions and reserved pages of a step's sequences.
int check_seqs(const q38a_runner* r, const q38a_step_seq* seqs, int num_seqs, int max_slot) {
  if (!seqs || num_seqs <= 0) return set_error(Q38A_ERR_INVALID, "runner: empty step");
  for (int b = 0; b < num_seqs; ++b) {
    const q38a_step_seq& q = seqs[b];
    if (q.slot < 0 || q.slot > max_slot) return set_error(Q38A_ERR_INVALID, "runner: slot %d out of range", q.slot);
    if (q.n <= 0 || q.pos0 < 0 || q.pos0 + q.n > r->opt.max_context)
      return set_error(Q38A_ERR_INVALID, "runner: positions [%d, %d) outside the context", q.pos0, q.pos0 + q.n);
    if (q38a_kv_cache_pages_of(r->kv, q.slot) * kPageTokens < q.pos0 + q.n)
      return set_error(Q38A_ERR_CAPACITY, "runner: KV pages of slot %d do not cover position %d", q.slot,
                       q.pos0 + q.n - 1);
  }
  return Q38A_OK;
}

q38a_qk_norm_rope_params append_params(const q38a_runner* r, int layer, int row0) {
  const int nq = r->opt.num_q_heads;
  q38a_qk_norm_rope_params p{};
  p.proj = r->proj + size_t(layer) * size_t(r->rows) * r->ld + size_t(row0) * r->ld;
  p.ld_proj = r->ld;
  p.q_norm = r->opt.q_norm + size_t(layer) * kHeadDim;
  p.k_norm = r->opt.k_norm + size_t(layer) * kHeadDim;
  p.eps = r->opt.eps;
  p.rope_theta = float(r->opt.rope_theta);
  p.num_q_heads = nq;
  p.num_kv_heads = r->opt.num_kv_heads;
  p.q_out = r->q16 + size_t(row0) * nq * kHeadDim;
  p.attn_layer = layer;
  p.rope_cos_sin = r->rope;
  p.rope_rows = r->opt.max_context;
  return p;
}

q38a_attention_params attention_params(const q38a_runner* r, int layer, int row0) {
  const int nq = r->opt.num_q_heads;
  const uint16_t* proj = r->proj + size_t(layer) * size_t(r->rows) * r->ld + size_t(row0) * r->ld;
  q38a_attention_params p{};
  p.q = r->q16 + size_t(row0) * nq * kHeadDim;
  p.gate = proj + size_t(nq) * kHeadDim;
  p.ld_gate = r->ld;
  p.out = r->out + size_t(layer) * size_t(r->rows) * nq * kHeadDim + size_t(row0) * nq * kHeadDim;
  p.num_q_heads = nq;
  p.num_kv_heads = r->opt.num_kv_heads;
  p.attn_layer = layer;
  p.split_scratch = r->scratch;
  p.max_splits = r->opt.max_splits;
  return p;
}

enum class Kind { Decode, Prefill, Mixed };

// The per-layer launches of one step whose metadata is already on (or queued to) the device.
int launch_layers(q38a_runner* r, Kind kind, int row0, const q38a_batch_desc& b, hipStream_t s) {
  q38a_kv_cache_desc kvd{};
  if (int rc = q38a_kv_cache_desc_get(r->kv, &kvd)) return rc;
  for (int layer = 0; layer < r->opt.attn_layers; ++layer) {
    const q38a_qk_norm_rope_params ap = append_params(r, layer, row0);
    if (int rc = q38a_qk_norm_rope_append(&ap, &b, &kvd, s)) return rc;
    const q38a_attention_params p = attention_params(r, layer, row0);
    int rc = Q38A_OK;
    // A prefill chunk of two or more tokens goes through the ragged launch, which also splits a
    // row tile's keys over several workgroups (the prefill launch does not): 0.15 vs 0.42 ms for a
    // 512-token chunk on a 9,290-token prefix, the same on a 2,048-token chunk. The batch has no
    // decode row, so the launch is bit-reproducible. A one-token chunk would be a decode row there.
    if (kind == Kind::Decode) rc = q38a_attention_decode(&p, &b, &kvd, s);
    else if (kind == Kind::Prefill && b.num_tokens == 1) rc = q38a_attention_prefill(&p, &b, &kvd, s);
    else {
      q38a_attention_params pr = p;
      pr.split_scratch = r->rscratch;
      rc = q38a_attention_ragged(&pr, &b, &kvd, s);
    }
    if (rc) return rc;
  }
  return Q38A_OK;
}

int capture_decode_graph(q38a_runner* r, int bucket, hipStream_t s, hipGraphExec_t* out) {
  if (int rc = check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "runner: begin capture")) return rc;
  int rc = upload_meta(r, s);
  if (!rc) rc = launch_layers(r, Kind::Decode, 0, r->batch(bucket, bucket, 1), s);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(s, &g);
  if (!rc) rc = check_hip(e, "runner: end capture");
  if (!rc) rc = check_hip(hipGraphInstantiate(out, g, nullptr, nullptr, 0), "runner: graph instantiate");
  if (g) (void)hipGraphDestroy(g);
  return rc;
}

}  // namespace

extern "C" {

int q38a_runner_bucket_for(int n, int max_batch) {
  for (int b : kBuckets)
    if (b >= n && b <= max_batch) return b;
  return max_batch;
}

int q38a_runner_create(const q38a_runner_options* opt, q38a_runner** out) {
  clear_error();
  if (!opt || !out) return set_error(Q38A_ERR_INVALID, "runner_create: null argument");
  *out = nullptr;
  const q38a_runner_options& o = *opt;
  if (o.num_q_heads <= 0 || o.num_kv_heads <= 0 || o.num_q_heads % o.num_kv_heads || o.attn_layers <= 0 ||
      o.num_pages <= 1 || o.max_batch <= 0 || o.max_chunk <= 0 || o.max_context <= 0 || o.max_splits <= 0 ||
      o.max_splits > 512 || !o.q_norm || !o.k_norm || !(o.rope_theta > 0))
    return set_error(Q38A_ERR_INVALID, "runner_create: bad options");
  auto* r = new (std::nothrow) q38a_runner();
  if (!r) return set_error(Q38A_ERR_INVALID, "runner_create: out of host memory");
  r->opt = o;
  r->ld = 2 * (o.num_q_heads + o.num_kv_heads) * kHeadDim;
  r->prefill_row = o.max_batch + 1;
  r->rows = r->prefill_row + o.max_chunk;
  r->dummy_slot = o.max_batch;
  r->meta = MetaLayout(r->rows);
  const int max_pages = (o.max_context + kPageTokens - 1) / kPageTokens;
  int rc = q38a_kv_cache_create(o.kv_dtype, o.num_kv_heads, o.attn_layers, o.num_pages, o.max_batch + 1, max_pages,
                                &r->kv);
  int ok = 0;
  if (!rc) rc = q38a_kv_cache_ensure(r->kv, r->dummy_slot, 1, &ok);
  if (!rc && !ok) rc = set_error(Q38A_ERR_CAPACITY, "runner_create: no page for the dummy slot");
  const size_t nq = size_t(o.num_q_heads);
  const size_t proj_elems = size_t(o.attn_layers) * size_t(r->rows) * size_t(r->ld);
  const size_t out_elems = size_t(o.attn_layers) * size_t(r->rows) * nq * kHeadDim;
  const size_t scratch = q38a_split_scratch_floats(o.max_batch + 1, o.num_q_heads, o.max_splits);
  const size_t rscratch = q38a_ragged_scratch_floats(o.max_batch + 1, r->rows, std::max(o.max_chunk, 2), o.num_q_heads,
                                                     o.num_kv_heads, o.max_splits);
  auto dmalloc = [&](void** p, size_t bytes, const char* what) {
    if (!rc) rc = check_hip(hipMalloc(p, bytes), what);
    if (!rc) rc = check_hip(hipMemset(*p, 0, bytes), what);
  };
  dmalloc(reinterpret_cast<void**>(&r->proj), proj_elems * 2, "runner_create: proj");
  dmalloc(reinterpret_cast<void**>(&r->out), out_elems * 2, "runner_create: out");
  dmalloc(reinterpret_cast<void**>(&r->q16), size_t(r->rows) * nq * kHeadDim * 2, "runner_create: q16");
  dmalloc(reinterpret_cast<void**>(&r->scratch), scratch * sizeof(float), "runner_create: scratch");
  dmalloc(reinterpret_cast<void**>(&r->rscratch), rscratch * sizeof(float), "runner_create: ragged scratch");
  dmalloc(reinterpret_cast<void**>(&r->meta_dev), r->meta.bytes, "runner_create: metadata");
  dmalloc(reinterpret_cast<void**>(&r->rope), size_t(o.max_context) * kRotaryDim * sizeof(float), "runner_create: rope");
  if (!rc) rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&r->meta_host), r->meta.bytes, 0), "runner_create: pinned metadata");
  if (!rc) rc = check_hip(hipEventCreateWithFlags(&r->meta_done, hipEventDisableTiming), "runner_create: event");
  if (!rc) rc = check_hip(hipStreamCreateWithFlags(&r->capture_stream, hipStreamNonBlocking), "runner_create: stream");
  if (!rc) {
    // RoPE table of every position, computed once on the host with the reference's libm calls
    std::vector<float> table(size_t(o.max_context) * kRotaryDim);
    rc = q38a_rope_table_fill(table.data(), 0, o.max_context, o.rope_theta, kRotaryDim);
    if (!rc) rc = check_hip(hipMemcpy(r->rope, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice),
                            "runner_create: rope upload");
  }
  if (!rc) rc = check_hip(hipDeviceSynchronize(), "runner_create: sync");
  if (rc) {
    delete r;
    return rc;
  }
  *out = r;
  return Q38A_OK;
}

void q38a_runner_destroy(q38a_runner* r) {
  if (r && r->meta_pending) (void)hipEventSynchronize(r->meta_done);
  delete r;
}

int q38a_runner_get_buffers(const q38a_runner* r, q38a_runner_buffers* out) {
  clear_error();
  if (!r || !out) return set_error(Q38A_ERR_INVALID, "runner_get_buffers: null argument");
  const size_t nq = size_t(r->opt.num_q_heads);
  *out = q38a_runner_buffers{r->proj, r->ld, size_t(r->rows) * r->ld, r->out, size_t(r->rows) * nq * kHeadDim,
                             r->q16, r->rows, r->prefill_row};
  return Q38A_OK;
}

q38a_kv_cache* q38a_runner_kv(q38a_runner* r) { return r ? r->kv : nullptr; }

int q38a_runner_num_slots(const q38a_runner* r) { return r ? r->opt.max_batch : 0; }

int q38a_runner_set_graphs(q38a_runner* r, int on) {
  clear_error();
  if (!r) return set_error(Q38A_ERR_INVALID, "runner_set_graphs: null runner");
  r->opt.use_graphs = on;
  return Q38A_OK;
}

int q38a_runner_graph_buckets(const q38a_runner* r, int* buckets, int cap) {
  if (!r) return 0;
  int n = 0;
  for (const auto& g : r->graphs) {
    if (buckets && n < cap) buckets[n] = g.first;
    ++n;
  }
  return n;
}

int q38a_runner_decode(q38a_runner* r, const q38a_step_seq* rows, int n, void* stream) {
  clear_error();
  if (!r) return set_error(Q38A_ERR_INVALID, "runner_decode: null runner");
  if (n <= 0 || n > r->opt.max_batch)
    return set_error(Q38A_ERR_INVALID, "runner_decode: %d rows (max %d)", n, r->opt.max_batch);
  if (int rc = check_seqs(r, rows, n, r->opt.max_batch - 1)) return rc;
  for (int i = 0; i < n; ++i)
    if (rows[i].n != 1) return set_error(Q38A_ERR_INVALID, "runner_decode: row %d has %d tokens", i, rows[i].n);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool graphs = r->opt.use_graphs != 0;
  const int bucket = graphs ? q38a_runner_bucket_for(n, r->opt.max_batch) : n;
  if (int rc = q38a_kv_cache_sync(r->kv, stream)) return rc;
  std::vector<q38a_step_seq> padded(size_t(bucket), q38a_step_seq{r->dummy_slot, 0, 1});
  if (graphs && !r->graphs.count(bucket)) {
    // warm-up outside capture on the dummy slot only (lazy module loading, cached device queries)
    if (int rc = wait_meta(r)) return rc;
    fill_meta(r, padded.data(), bucket);
    if (int rc = upload_meta(r, s)) return rc;
    if (int rc = launch_layers(r, Kind::Decode, 0, r->batch(bucket, bucket, 1), s)) return rc;
    if (int rc = check_hip(hipStreamSynchronize(s), "runner: warm-up")) return rc;
    hipGraphExec_t exec = nullptr;
    if (int rc = capture_decode_graph(r, bucket, r->capture_stream, &exec)) return rc;
    r->graphs[bucket] = exec;
  }
  std::copy(rows, rows + n, padded.begin());
  if (int rc = wait_meta(r)) return rc;
  fill_meta(r, padded.data(), bucket);
  if (graphs) {
    if (int rc = check_hip(hipGraphLaunch(r->graphs[bucket], s), "runner: graph launch")) return rc;
  } else {
    if (int rc = upload_meta(r, s)) return rc;
    if (int rc = launch_layers(r, Kind::Decode, 0, r->batch(bucket, bucket, 1), s)) return rc;
  }
  return mark_meta(r, s);
}

int q38a_runner_prefill(q38a_runner* r, int slot, int pos0, int n, void* stream) {
  clear_error();
  if (!r) return set_error(Q38A_ERR_INVALID, "runner_prefill: null runner");
  if (n > r->opt.max_chunk) return set_error(Q38A_ERR_INVALID, "runner_prefill: %d tokens (max %d)", n, r->opt.max_chunk);
  const q38a_step_seq q{slot, pos0, n};
  if (int rc = check_seqs(r, &q, 1, r->opt.max_batch - 1)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = q38a_kv_cache_sync(r->kv, stream)) return rc;
  if (int rc = wait_meta(r)) return rc;
  fill_meta(r, &q, 1);
  if (int rc = upload_meta(r, s)) return rc;
  if (int rc = launch_layers(r, Kind::Prefill, r->prefill_row, r->batch(1, n, n), s)) return rc;
  return mark_meta(r, s);
}

int q38a_runner_step(q38a_runner* r, const q38a_step_seq* seqs, int num_seqs, void* stream) {
  clear_error();
  if (!r) return set_error(Q38A_ERR_INVALID, "runner_step: null runner");
  if (int rc = check_seqs(r, seqs, num_seqs, r->opt.max_batch - 1)) return rc;
  int tokens = 0, max_run = 0;
  for (int b = 0; b < num_seqs; ++b) {
    tokens += seqs[b].n;
    max_run = std::max(max_run, seqs[b].n);
  }
  if (num_seqs > r->opt.max_batch + 1 || tokens > r->rows || max_run > std::max(r->opt.max_chunk, 1))
    return set_error(Q38A_ERR_INVALID, "runner_step: %d sequences / %d tokens exceed the runner's buffers", num_seqs,
                     tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = q38a_kv_cache_sync(r->kv, stream)) return rc;
  if (int rc = wait_meta(r)) return rc;
  fill_meta(r, seqs, num_seqs);
  if (int rc = upload_meta(r, s)) return rc;
  if (int rc = launch_layers(r, Kind::Mixed, 0, r->batch(num_seqs, tokens, max_run), s)) return rc;
  return mark_meta(r, s);
}

}  // extern "C"
