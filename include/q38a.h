/*
 * q38a — MI355X (gfx950) ragged paged-KV attention step for the 16 full-attention layers of
 * Qwen3.8-27B. C ABI of the hand-written HIP kernels and of the host-side page allocator and
 * step runner that call them.
 *
 * Every entry point mirrors one function of the reference engine's kernel launch API
 * (reference src/kernels/kernels.h) or its host classes (include/qwen38/kv_cache.h,
 * src/model_runner.cpp); the citation is on each declaration. Differences from the C++
 * reference are confined to what a C ABI needs:
 *   - fp16 / bf16 tensors are passed as uint16_t bit patterns, streams as void* (hipStream_t);
 *   - errors are an int status (Q38A_OK = 0) plus q38a_last_error(), a thread-local message,
 *     instead of the reference's qwen38::Error exceptions;
 *   - q38a_qk_norm_rope_params carries a RoPE cos/sin table (q38a_rope_table_fill) computed on
 *     the host with the same libm calls as the reference CPU path, so appended int8 bytes match
 *     it bit for bit.
 * Conventions (reference kernels.h:1-6): all pointers are device pointers unless stated, every
 * launcher is asynchronous on `stream`, allocates nothing, never synchronises the host, and is
 * safe to capture into a hipGraph (data-dependent sizes are read from device memory).
 */
#ifndef Q38A_H
#define Q38A_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q38A_PAGE_TOKENS 64 /* reference kernels.h:38 kPageTokens */
#define Q38A_HEAD_DIM 256   /* reference kernels.h:39 kHeadDim */

/* KV page formats. INT8 and BF16 are the reference's (kernels.h:36 KvDtype). INT8_VT is the
 * "tensor-core decode" variant of the int8 format (reference docs/OPTIMIZATION_PLAN.md:199-201):
 * the same bytes per page, K codes and K scales laid out as in INT8, but the V codes stored
 * transposed within each 16-token quarter of the page, [kvh][4 quarters][256 dims][16 tokens]
 * (a dim's 16 tokens contiguous, consecutive dims adjacent), and the V scales group-major,
 * [kvh][4 groups][64 tokens] f16.
 * INT8_VT is EXPERIMENTAL: every kernel supports it and it is parity-tested like INT8, but it is
 * slower than INT8 on every measured workload (decode, long-context decode, prefill and the mixed
 * step), so INT8 is the format to use. */
enum { Q38A_KV_INT8 = 0, Q38A_KV_BF16 = 1, Q38A_KV_INT8_VT = 2 };

/* Status codes. */
enum {
  Q38A_OK = 0,
  Q38A_ERR_INVALID = 1,     /* bad argument: null pointer, size, geometry */
  Q38A_ERR_UNSUPPORTED = 2, /* head_dim / GQA group / head count the kernels do not implement */
  Q38A_ERR_HIP = 3,         /* a HIP runtime call or kernel launch failed */
  Q38A_ERR_CAPACITY = 4     /* KV pool exhausted or a per-sequence page limit exceeded */
};

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* q38a_last_error(void);

/* ---- batch and cache descriptors --------------------------------------------------------- */

/* One engine step: M tokens from B sequences, each a contiguous run (a prefill chunk or one
 * decode token). Mirrors reference kernels.h:22-31 BatchDesc. */
typedef struct q38a_batch_desc {
  int num_seqs;           /* B (host value; fixed per captured graph) */
  int num_tokens;         /* M (host value; fixed per captured graph) */
  int max_tokens_per_seq; /* upper bound of any sequence's run length (host value) */
  const int32_t* seq_start; /* [B + 1] cu_seqlens: token offsets of each sequence */
  const int32_t* seq_slot;  /* [B] block-table row */
  const int32_t* seq_pos0;  /* [B] position of the sequence's first token in this step */
  const int32_t* tok_pos;   /* [M] absolute position of every token */
  const int32_t* tok_seq;   /* [M] sequence index of every token */
} q38a_batch_desc;

/* Paged KV cache of all attention layers (reference kernels.h:41-70 KvCacheDesc and
 * docs/FORMAT.md 3.1). Per (layer, page), int8: K [kvh][64][256] i8 | V same |
 * K scales [kvh][64][4] f16 | V scales same; bf16: K [kvh][64][256] bf16 | V same. */
typedef struct q38a_kv_cache_desc {
  uint8_t* pool;             /* base of the pool: [layers][num_pages][page_bytes] */
  int dtype;                 /* Q38A_KV_INT8 or Q38A_KV_BF16 */
  int kv_heads;
  int num_pages;
  size_t page_bytes;         /* bytes per (layer, page) */
  size_t layer_stride;       /* num_pages * page_bytes */
  const int32_t* block_table; /* [slots][max_pages_per_seq] page ids */
  int max_pages_per_seq;
} q38a_kv_cache_desc;

/* Bytes of one (layer, page) block (reference kernels.h:66-69 page_bytes_for). */
size_t q38a_kv_page_bytes(int dtype, int kv_heads);

/* Byte offsets inside one (layer, page) block (reference kernels.h:53-65):
 * out[0] K row, out[1] V row, out[2] K scales, out[3] V scales (scales: int8 formats only).
 * INT8_VT: out[1] is the V code of (head, dim 0, tok) (dim d at + 16 d) and out[3] the V scale of
 * (head, group 0, tok) (group g at + 128 g). */
int q38a_kv_offsets(int dtype, int kv_heads, int head, int tok, size_t out[4]);

/* ---- fused q/k RMSNorm + RoPE + KV append ------------------------------------------------- */

/* Mirrors reference kernels.h:142-153 QkNormRopeParams, plus the RoPE table. */
typedef struct q38a_qk_norm_rope_params {
  const uint16_t* proj;   /* [M][ld_proj] bf16: [q nq*256 | gate nq*256 | k nkv*256 | v nkv*256] */
  int ld_proj;
  const float* q_norm;    /* [256], already 1 + w */
  const float* k_norm;    /* [256], already 1 + w */
  float eps;
  float rope_theta;       /* informational: the table below already encodes theta */
  int num_q_heads;
  int num_kv_heads;
  uint16_t* q_out;        /* [M][nq][256] fp16 */
  int attn_layer;         /* index among attention layers */
  const float* rope_cos_sin; /* [rope_rows][64]: per position [cos 0..31 | sin 0..31] */
  int rope_rows;          /* positions covered by the table; every tok_pos must be below it */
} q38a_qk_norm_rope_params;

/* Host-side RoPE table for positions [pos_begin, pos_begin + count): out[count][rotary_dim],
 * each row [cos(pos*inv_i) | sin(pos*inv_i)], inv_i = 1 / powf(theta, 2i / rotary_dim), through
 * the same libm calls as reference src/ref/ops.cpp:101-111. `out` is host memory. */
int q38a_rope_table_fill(float* out, int pos_begin, int count, double theta, int rotary_dim);

/* Per token: offset-RMSNorm of q and k heads, partial RoPE (dims 0..63, pairs (i, i+32)), q -> fp16,
 * k and v -> paged cache (int8 per 64-dim group with an fp16 scale, or bf16).
 * Replaces reference kernels.h:154-155 qk_norm_rope_append (src/kernels/qk_norm_rope.cu:94-100). */
int q38a_qk_norm_rope_append(const q38a_qk_norm_rope_params* p, const q38a_batch_desc* batch,
                             const q38a_kv_cache_desc* kv, void* stream);

/* ---- attention ---------------------------------------------------------------------------- */

/* Mirrors reference kernels.h:157-168 AttentionParams. */
typedef struct q38a_attention_params {
  const uint16_t* q;      /* [M][nq][256] fp16 */
  const uint16_t* gate;   /* bf16, row stride ld_gate (normally proj + nq*256) */
  int ld_gate;
  uint16_t* out;          /* [M][nq*256] bf16 */
  int num_q_heads;
  int num_kv_heads;
  int attn_layer;
  float* split_scratch;   /* decode partials: [B][nq][max_splits][256 + 2] floats */
  int max_splits;
} q38a_attention_params;

/* Upper bound of the splits per sequence the decode launchers use; size split_scratch with
 * q38a_split_scratch_floats(B, nq, this). Replaces reference kernels.h:172
 * attention_decode_splits (src/kernels/attention_decode.cu:272-277). */
int q38a_attention_decode_splits(int batch_seqs, int kv_heads, int num_sms, int max_splits);

/* Floats of split scratch for `rows` decode rows. */
size_t q38a_split_scratch_floats(int rows, int num_q_heads, int max_splits);

/* Decode: one token per sequence (M == B), keys [0, seq_pos0 + 1) of each sequence; split-KV
 * flash-decoding on MFMA, sigmoid(gate) applied in the merge. Replaces reference
 * kernels.h:173-174 attention_decode (src/kernels/attention_decode.cu:279-296). */
int q38a_attention_decode(const q38a_attention_params* p, const q38a_batch_desc* batch,
                          const q38a_kv_cache_desc* kv, void* stream);

/* The split kernel of q38a_attention_decode alone: the partials go to p->split_scratch and p->out
 * is not written. Their consumer is q38a_qgemm_merge_oproj (include/q38a_gemm.h), which merges
 * them inside the o-projection. No counterpart in the reference (its decode launch always runs the
 * combine kernel, src/kernels/attention_decode.cu:279-296). */
int q38a_attention_decode_partials(const q38a_attention_params* p, const q38a_batch_desc* batch,
                                   const q38a_kv_cache_desc* kv, void* stream);

/* q38a_attention_decode without caller scratch: the split partials go to a static device array
 * of q38a_noalloc_scratch_floats() floats (32 MiB, one per GPU, held until the process ends) and
 * p->split_scratch is ignored; the call allocates nothing (no hipMalloc, no library allocation).
 * Fails with Q38A_ERR_INVALID when num_seqs * num_q_heads * max_splits * 258 exceeds the array.
 * Every call on one GPU shares the array: calls that overlap in time on one GPU race.
 * No counterpart in the reference; for callers that cannot allocate (code under hipGraph
 * capture, tight serving loops, harnesses that forbid allocation). */
int q38a_attention_decode_noalloc(const q38a_attention_params* p, const q38a_batch_desc* batch,
                                  const q38a_kv_cache_desc* kv, void* stream);
size_t q38a_noalloc_scratch_floats(void);

/* Prefill: causal attention of each sequence's new tokens over its cached prefix and themselves
 * (the chunk's K/V must already be appended); fp16 MFMA, gate in the epilogue. Replaces
 * reference kernels.h:178-179 attention_prefill (src/kernels/attention_prefill.cu:317-335). */
int q38a_attention_prefill(const q38a_attention_params* p, const q38a_batch_desc* batch,
                           const q38a_kv_cache_desc* kv, void* stream);

/* Floats of split_scratch q38a_attention_ragged needs for a batch of these host sizes (the
 * BatchDesc host fields, num_seqs/num_tokens/max_tokens_per_seq, of every launch it serves must
 * not exceed them). No counterpart in the reference; 0 for invalid arguments. */
size_t q38a_ragged_scratch_floats(int num_seqs, int num_tokens, int max_tokens_per_seq, int num_q_heads,
                                  int num_kv_heads, int max_splits);

/* Zeroes the counters at the front of a ragged scratch buffer (asynchronous on `stream`). Call it
 * once after allocating the buffer, unless it was allocated zeroed; every q38a_attention_ragged
 * launch leaves the counters zero again. No counterpart in the reference. */
int q38a_ragged_scratch_init(float* split_scratch, void* stream);

/* Mixed continuous-batching step: sequences with one token (decode rows) and with several
 * (prefill chunks) in one ragged batch, scheduled by one attention launch plus the split merge;
 * split_scratch holds q38a_ragged_scratch_floats(...) floats.
 * No counterpart in the reference (its Engine::step, src/engine.cpp:133-182, runs prefill and
 * decode as separate launches); semantics are those of attention_decode / attention_prefill
 * applied to each sequence. The decode rows' key blocks are handed out dynamically, so the
 * blocks a wave sums, and the fp16 rounding of its probabilities, can differ from run to run: a
 * decode row's outputs move by up to ~2^-11 of the V magnitude (inside the parity tolerance);
 * prefill rows, and the decode and prefill launches, are bit-reproducible. The launch's work counters (decode item queue and
 * block claims) live at the front of split_scratch: launches with separate scratch buffers are
 * independent and may run concurrently on different streams; one scratch buffer serves one
 * launch at a time. */
int q38a_attention_ragged(const q38a_attention_params* p, const q38a_batch_desc* batch,
                          const q38a_kv_cache_desc* kv, void* stream);

/* ---- host-side page allocator (reference include/qwen38/kv_cache.h:19-51) ----------------- */

typedef struct q38a_kv_cache q38a_kv_cache; /* opaque; owns the device pool and block table */

/* Allocates and zeroes a pool of num_pages pages for `layers` attention layers and a
 * [num_slots][max_pages_per_seq] block table (reference src/kv_cache.cpp:14-38). */
int q38a_kv_cache_create(int dtype, int kv_heads, int layers, int num_pages, int num_slots,
                         int max_pages_per_seq, q38a_kv_cache** out);
void q38a_kv_cache_destroy(q38a_kv_cache* c);
/* Descriptor of the cache (reference kv_cache.cpp:40-51). */
int q38a_kv_cache_desc_get(const q38a_kv_cache* c, q38a_kv_cache_desc* out);
/* Reserve pages for positions [0, tokens) of `slot`; *ok = 0 (and nothing changes) when the pool
 * cannot provide them (reference kv_cache.cpp:53-70). Returns Q38A_ERR_CAPACITY if `tokens`
 * exceeds the per-sequence limit. */
int q38a_kv_cache_ensure(q38a_kv_cache* c, int slot, int tokens, int* ok);
/* Return the slot's pages to the free list (reference kv_cache.cpp:72-76). */
int q38a_kv_cache_release(q38a_kv_cache* c, int slot);
/* Upload modified block-table rows asynchronously (reference kv_cache.cpp:78-88). */
int q38a_kv_cache_sync(q38a_kv_cache* c, void* stream);
int q38a_kv_cache_free_pages(const q38a_kv_cache* c);
int q38a_kv_cache_pages_of(const q38a_kv_cache* c, int slot);
/* Host copy of a slot's page list (up to `cap` entries); returns the count in *n. */
int q38a_kv_cache_page_list(const q38a_kv_cache* c, int slot, int32_t* pages, int cap, int* n);

#ifdef __cplusplus
}
#endif

#endif /* Q38A_H */
