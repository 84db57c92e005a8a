/*
 * q38a runtime — the host side around the attention kernels of include/q38a.h: the launch
 * interface of the reference ModelRunner for the full-attention layers (step metadata upload,
 * per-layer append + attention, one hipGraph per decode batch-size bucket) and the reference
 * Engine's continuous-batching scheduler (admission with whole-request KV reservation, at most one
 * prefill chunk per iteration, one decode batch), plus a mixed policy that packs the chunk and the
 * decode rows into one ragged launch.
 *
 * Plain C ABI: opaque handles, POD structs, int status (Q38A_OK = 0, q38a_last_error() for the
 * message). Single-threaded like the reference (engine.h:43): one runner is driven by one thread
 * and one stream.
 */
#ifndef Q38A_RUNTIME_H
#define Q38A_RUNTIME_H

#include "q38a.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runner (reference include/qwen38/model_runner.h:33-121, src/model_runner.cpp) --------- */

typedef struct q38a_runner q38a_runner;

/* Mirrors the attention-relevant part of reference RunnerOptions (model_runner.h:33-45). */
typedef struct q38a_runner_options {
  int kv_dtype;          /* Q38A_KV_INT8 / Q38A_KV_BF16 */
  int num_q_heads;       /* 24 */
  int num_kv_heads;      /* 4 */
  int attn_layers;       /* full-attention layers sharing the page ids (16) */
  int num_pages;         /* KV pool pages per layer */
  int max_batch;         /* sequence slots; one more (dummy) slot pads graph buckets */
  int max_chunk;         /* tokens of one prefill chunk (reference prefill_chunk) */
  int max_context;       /* positions per sequence */
  int max_splits;        /* decode split bound, <= 512 */
  float eps;             /* RMSNorm epsilon (1e-6) */
  double rope_theta;     /* 1e7 */
  const float* q_norm;   /* device fp32 [attn_layers][256], stored 1 + w */
  const float* k_norm;   /* device fp32 [attn_layers][256] */
  int use_graphs;        /* decode steps replay one hipGraph per bucket */
} q38a_runner_options;

/* Runner-owned device buffers. Row r of a step is token r of the packed batch: decode rows use
 * rows [0, n), a prefill chunk alone uses rows [prefill_row, prefill_row + n), a mixed step uses
 * rows [0, tokens) in the order of its sequences. */
typedef struct q38a_runner_buffers {
  uint16_t* proj;            /* bf16 [attn_layers][rows][ld_proj]: q | gate | k | v per row */
  int ld_proj;
  size_t proj_layer_stride;  /* elements */
  uint16_t* out;             /* bf16 [attn_layers][rows][nq * 256] gated attention output */
  size_t out_layer_stride;   /* elements */
  uint16_t* q16;             /* fp16 [rows][nq][256], q of the last layer run */
  int rows;                  /* max_batch + 1 + max_chunk */
  int prefill_row;           /* max_batch + 1 */
} q38a_runner_buffers;

/* One sequence of a step: positions [pos0, pos0 + n) of the sequence in `slot`. */
typedef struct q38a_step_seq {
  int slot;
  int pos0;
  int n;
} q38a_step_seq;

int q38a_runner_create(const q38a_runner_options* opt, q38a_runner** out);
void q38a_runner_destroy(q38a_runner* r);
int q38a_runner_get_buffers(const q38a_runner* r, q38a_runner_buffers* out);
/* The runner's page allocator (slots [0, max_batch) are the caller's). */
q38a_kv_cache* q38a_runner_kv(q38a_runner* r);
int q38a_runner_num_slots(const q38a_runner* r);

/* Bucketed batch size of a decode step (reference src/model_runner.cpp:28-33):
 * the first of {1, 2, 4, 8, 12, 16, 24, 32, 48, 64} >= n and <= max_batch, else max_batch. */
int q38a_runner_bucket_for(int n, int max_batch);

/* One decode step of every attention layer: rows[i] = {slot, position, 1}; the pages of every
 * position must be reserved. Rows are padded to the bucket with the dummy slot at position 0; with
 * graphs on, the step (metadata upload + append + decode per layer) is one replayed graph
 * (reference ModelRunner::decode, src/model_runner.cpp:488-532). */
int q38a_runner_decode(q38a_runner* r, const q38a_step_seq* rows, int n, void* stream);

/* One prefill chunk of every attention layer (reference ModelRunner::prefill, eager). Chunks of two
 * or more tokens use the ragged attention launch (it splits long key ranges over workgroups), a
 * one-token chunk the prefill launch. */
int q38a_runner_prefill(q38a_runner* r, int slot, int pos0, int n, void* stream);

/* One mixed step: any sequences (n == 1 decode rows, n > 1 chunks), one ragged attention launch
 * per layer. No counterpart in the reference. */
int q38a_runner_step(q38a_runner* r, const q38a_step_seq* seqs, int num_seqs, void* stream);

int q38a_runner_set_graphs(q38a_runner* r, int on);
/* Buckets whose decode graph has been captured (ascending); returns the count. */
int q38a_runner_graph_buckets(const q38a_runner* r, int* buckets, int cap);

/* ---- engine (reference include/qwen38/engine.h, src/engine.cpp) ---------------------------- */

typedef struct q38a_engine q38a_engine;

typedef struct q38a_engine_options {
  int prefill_chunk;  /* tokens per prefill chunk, <= the runner's max_chunk */
  int mixed;          /* 0: reference policy (prefill launch, then a decode launch that already
                         includes a sequence whose prompt just completed); 1: the chunk and the
                         decode rows of earlier iterations in one ragged launch */
} q38a_engine_options;

/* One planned sequence of the next iteration and the runner rows its tokens occupy. */
typedef struct q38a_plan_entry {
  int request_id;
  int slot;
  int pos0;
  int n;
  int row;  /* first proj/out row of the tokens */
} q38a_plan_entry;

typedef struct q38a_engine_stats {
  long long iterations, launches, prefill_tokens, decode_tokens, requests_done, requests_failed;
} q38a_engine_stats;

int q38a_engine_create(q38a_runner* runner, const q38a_engine_options* opt, q38a_engine** out);
void q38a_engine_destroy(q38a_engine* e);
/* Queue a request of `prompt_tokens` prompt tokens generating `max_new_tokens`; returns its id
 * (>= 0) or a negative status. Requests are admitted in order when a slot and the pages of the
 * whole request are free (reference Engine::admit, src/engine.cpp:62-91). */
int q38a_engine_submit(q38a_engine* e, int prompt_tokens, int max_new_tokens);
/* Admit and plan the next iteration; *n = planned sequences (0: nothing runnable). The caller
 * fills the planned rows of the runner's proj buffer before q38a_engine_execute. */
int q38a_engine_plan(q38a_engine* e, q38a_plan_entry* entries, int cap, int* n);
/* Run the planned iteration on `stream` and advance every sequence (reference Engine::step,
 * src/engine.cpp:110-184). */
int q38a_engine_execute(q38a_engine* e, void* stream);
int q38a_engine_idle(const q38a_engine* e);
int q38a_engine_get_stats(const q38a_engine* e, q38a_engine_stats* out);
/* Ids of requests finished since the last call (negative id = failed, as -1 - id). */
int q38a_engine_take_finished(q38a_engine* e, int* ids, int cap, int* n);
/* Next position to write of a running request, or -1. */
int q38a_engine_position(const q38a_engine* e, int request_id);

#ifdef __cplusplus
}
#endif

#endif /* Q38A_RUNTIME_H */
