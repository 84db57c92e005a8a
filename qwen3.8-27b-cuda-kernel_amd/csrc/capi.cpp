// C ABI of the q38a library: argument validation, error reporting, the host RoPE table and the
// kernel launchers' entry points. Exceptions never cross this boundary; every function returns a
// status and leaves a thread-local message for q38a_last_error().
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace q38a {

int launch_qk_norm_rope_append(const q38a_qk_norm_rope_params& p, const q38a_batch_desc& b,
                               const q38a_kv_cache_desc& kv, hipStream_t stream);
int launch_attention_decode(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream);
int launch_attention_decode_partials(const q38a_attention_params& p, const q38a_batch_desc& b,
                                     const q38a_kv_cache_desc& kv, hipStream_t stream);
int launch_attention_prefill(const q38a_attention_params& p, const q38a_batch_desc& b,
                             const q38a_kv_cache_desc& kv, hipStream_t stream);
int launch_attention_ragged(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream);
int ragged_scratch_init(float* scratch, hipStream_t stream);
int launch_attention_decode_noalloc(const q38a_attention_params& p, const q38a_batch_desc& b,
                                    const q38a_kv_cache_desc& kv, hipStream_t stream);
size_t noalloc_scratch_floats();
int max_group();
size_t ragged_scratch_floats(int num_seqs, int num_tokens, int max_tokens_per_seq, int nq, int nkv, int max_splits);

namespace {
thread_local std::string g_error;
}

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

void clear_error() { g_error.clear(); }

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return Q38A_OK;
  return set_error(Q38A_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int device_cu_count(int* out) {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lock(mu);
  if (int(cache.size()) <= dev) cache.resize(size_t(dev) + 1, 0);
  if (cache[size_t(dev)] == 0) {
    int cus = 0;
    if (int rc = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
                           "hipDeviceGetAttribute"))
      return rc;
    cache[size_t(dev)] = cus;
  }
  *out = cache[size_t(dev)];
  return Q38A_OK;
}

int validate_batch(const q38a_batch_desc* b, bool need_tok) {
  if (!b) return set_error(Q38A_ERR_INVALID, "batch descriptor is null");
  if (b->num_seqs < 0 || b->num_tokens < 0 || b->max_tokens_per_seq < 0)
    return set_error(Q38A_ERR_INVALID, "batch: negative size");
  if (b->num_seqs > 0 && (!b->seq_start || !b->seq_slot || !b->seq_pos0))
    return set_error(Q38A_ERR_INVALID, "batch: seq_start/seq_slot/seq_pos0 must be set");
  if (need_tok && b->num_tokens > 0 && (!b->tok_pos || !b->tok_seq))
    return set_error(Q38A_ERR_INVALID, "batch: tok_pos/tok_seq must be set");
  return Q38A_OK;
}

int validate_kv(const q38a_kv_cache_desc* k) {
  if (!k) return set_error(Q38A_ERR_INVALID, "KV descriptor is null");
  if (!k->pool || !k->block_table) return set_error(Q38A_ERR_INVALID, "KV: pool and block_table must be set");
  if (k->dtype != Q38A_KV_INT8 && k->dtype != Q38A_KV_BF16 && k->dtype != Q38A_KV_INT8_VT)
    return set_error(Q38A_ERR_INVALID, "KV: unknown dtype %d", k->dtype);
  if (k->kv_heads <= 0 || k->num_pages <= 0 || k->max_pages_per_seq <= 0)
    return set_error(Q38A_ERR_INVALID, "KV: kv_heads, num_pages and max_pages_per_seq must be positive");
  if (k->page_bytes != q38a_kv_page_bytes(k->dtype, k->kv_heads))
    return set_error(Q38A_ERR_INVALID, "KV: page_bytes %zu does not match the layout (%zu)", k->page_bytes,
                     q38a_kv_page_bytes(k->dtype, k->kv_heads));
  if (k->layer_stride < size_t(k->num_pages) * k->page_bytes)
    return set_error(Q38A_ERR_INVALID, "KV: layer_stride smaller than num_pages * page_bytes");
  return Q38A_OK;
}

namespace {

int validate_heads(int nq, int nkv) {
  if (nq <= 0 || nkv <= 0 || nq % nkv != 0)
    return set_error(Q38A_ERR_UNSUPPORTED, "attention: %d q heads are not a multiple of %d kv heads", nq, nkv);
  if (nq / nkv > max_group())
    return set_error(Q38A_ERR_UNSUPPORTED, "attention: GQA group %d exceeds %d", nq / nkv, max_group());
  return Q38A_OK;
}

int validate_attention(const q38a_attention_params* p, const q38a_batch_desc* b, const q38a_kv_cache_desc* kv,
                       bool need_scratch) {
  if (!p) return set_error(Q38A_ERR_INVALID, "attention params are null");
  if (int rc = validate_batch(b, false)) return rc;
  if (int rc = validate_kv(kv)) return rc;
  if (int rc = validate_heads(p->num_q_heads, p->num_kv_heads)) return rc;
  if (p->num_kv_heads != kv->kv_heads)
    return set_error(Q38A_ERR_INVALID, "attention: %d kv heads but the cache has %d", p->num_kv_heads, kv->kv_heads);
  if (!p->q || !p->gate || !p->out) return set_error(Q38A_ERR_INVALID, "attention: q, gate and out must be set");
  if (p->ld_gate < p->num_q_heads * kHeadDim)
    return set_error(Q38A_ERR_INVALID, "attention: ld_gate %d < nq*256", p->ld_gate);
  if (p->attn_layer < 0) return set_error(Q38A_ERR_INVALID, "attention: negative layer");
  if (need_scratch && (!p->split_scratch || p->max_splits <= 0))
    return set_error(Q38A_ERR_INVALID, "attention: split scratch and max_splits must be set");
  return Q38A_OK;
}

}  // namespace
}  // namespace q38a

using namespace q38a;

extern "C" {

const char* q38a_last_error(void) { return g_error.c_str(); }

size_t q38a_kv_page_bytes(int dtype, int kv_heads) {
  if (kv_heads <= 0 || (dtype != Q38A_KV_INT8 && dtype != Q38A_KV_BF16 && dtype != Q38A_KV_INT8_VT)) return 0;
  return PageLayout{kv_heads, dtype}.page_bytes();
}

int q38a_kv_offsets(int dtype, int kv_heads, int head, int tok, size_t out[4]) {
  clear_error();
  if (!out || kv_heads <= 0 || head < 0 || head >= kv_heads || tok < 0 || tok >= kPageTokens ||
      (dtype != Q38A_KV_INT8 && dtype != Q38A_KV_BF16 && dtype != Q38A_KV_INT8_VT))
    return set_error(Q38A_ERR_INVALID, "kv_offsets: bad arguments");
  const PageLayout L{kv_heads, dtype};
  out[0] = L.k_row(head, tok);
  out[1] = dtype == Q38A_KV_INT8_VT ? L.vt_code(head, 0, tok) : L.v_row(head, tok);
  out[2] = L.int8() ? L.k_scales(head, tok) : 0;
  out[3] = dtype == Q38A_KV_INT8_VT ? L.vt_scale(head, 0, tok) : (L.int8() ? L.v_scales(head, tok) : 0);
  return Q38A_OK;
}

int q38a_rope_table_fill(float* out, int pos_begin, int count, double theta, int rotary_dim) {
  clear_error();
  if (!out || count < 0 || pos_begin < 0 || rotary_dim != kRotaryDim || !(theta > 0))
    return set_error(Q38A_ERR_INVALID, "rope_table_fill: bad arguments (rotary_dim must be 64)");
  // Same float operations and libm calls as the reference CPU path (src/ref/ops.cpp:101-111):
  // inv = 1 / powf(theta, 2i / 64), angle = pos * inv, then cosf / sinf of the float angle.
  const int half = rotary_dim / 2;
  float inv[kRotaryDim / 2];
  for (int i = 0; i < half; ++i) {
    const volatile float expo = float(2 * i) / float(rotary_dim);
    inv[i] = 1.0f / std::pow(float(theta), float(expo));
  }
  for (int p = 0; p < count; ++p) {
    float* row = out + size_t(p) * rotary_dim;
    const float fpos = float(pos_begin + p);
    for (int i = 0; i < half; ++i) {
      const volatile float angle = fpos * inv[i];
      row[i] = std::cos(float(angle));
      row[half + i] = std::sin(float(angle));
    }
  }
  return Q38A_OK;
}

int q38a_qk_norm_rope_append(const q38a_qk_norm_rope_params* p, const q38a_batch_desc* batch,
                             const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (!p) return set_error(Q38A_ERR_INVALID, "qk_norm_rope params are null");
  if (int rc = validate_batch(batch, true)) return rc;
  if (int rc = validate_kv(kv)) return rc;
  if (p->num_q_heads <= 0 || p->num_kv_heads <= 0 || p->num_kv_heads != kv->kv_heads)
    return set_error(Q38A_ERR_INVALID, "qk_norm_rope: head counts (%d q, %d kv, cache %d)", p->num_q_heads,
                     p->num_kv_heads, kv->kv_heads);
  if (!p->proj || !p->q_norm || !p->k_norm || !p->q_out)
    return set_error(Q38A_ERR_INVALID, "qk_norm_rope: proj, q_norm, k_norm and q_out must be set");
  if (p->ld_proj < 2 * (p->num_q_heads + p->num_kv_heads) * kHeadDim || p->ld_proj % 4 != 0)
    return set_error(Q38A_ERR_INVALID, "qk_norm_rope: ld_proj %d too small or not a multiple of 4", p->ld_proj);
  if (!p->rope_cos_sin || p->rope_rows <= 0)
    return set_error(Q38A_ERR_INVALID, "qk_norm_rope: rope_cos_sin table (q38a_rope_table_fill) is required");
  if (p->attn_layer < 0) return set_error(Q38A_ERR_INVALID, "qk_norm_rope: negative layer");
  return launch_qk_norm_rope_append(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

int q38a_attention_decode_splits(int batch_seqs, int kv_heads, int num_sms, int max_splits) {
  (void)batch_seqs;
  (void)kv_heads;
  (void)num_sms;
  // Splits are chosen per sequence on the device (balanced by pages); max_splits bounds them and
  // the launchers accept at most 512.
  return max_splits < 1 ? 1 : (max_splits > 512 ? 512 : max_splits);
}

size_t q38a_split_scratch_floats(int rows, int num_q_heads, int max_splits) {
  if (rows <= 0 || num_q_heads <= 0 || max_splits <= 0) return 0;
  return size_t(rows) * size_t(num_q_heads) * size_t(max_splits) * (kHeadDim + 2);
}

size_t q38a_ragged_scratch_floats(int num_seqs, int num_tokens, int max_tokens_per_seq, int num_q_heads,
                                  int num_kv_heads, int max_splits) {
  if (num_seqs <= 0 || num_tokens <= 0 || max_tokens_per_seq <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || max_splits <= 0)
    return 0;
  return ragged_scratch_floats(num_seqs, num_tokens, max_tokens_per_seq, num_q_heads, num_kv_heads, max_splits);
}

int q38a_attention_decode(const q38a_attention_params* p, const q38a_batch_desc* batch,
                          const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_attention(p, batch, kv, true)) return rc;
  if (batch->num_tokens != batch->num_seqs)
    return set_error(Q38A_ERR_INVALID, "attention_decode: one token per sequence required (M %d, B %d)",
                     batch->num_tokens, batch->num_seqs);
  return launch_attention_decode(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

int q38a_attention_decode_partials(const q38a_attention_params* p, const q38a_batch_desc* batch,
                                   const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_attention(p, batch, kv, true)) return rc;
  if (batch->num_tokens != batch->num_seqs)
    return set_error(Q38A_ERR_INVALID, "attention_decode_partials: one token per sequence required (M %d, B %d)",
                     batch->num_tokens, batch->num_seqs);
  return launch_attention_decode_partials(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

int q38a_attention_decode_noalloc(const q38a_attention_params* p, const q38a_batch_desc* batch,
                                  const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_attention(p, batch, kv, false)) return rc;
  if (p->max_splits <= 0) return set_error(Q38A_ERR_INVALID, "attention_decode_noalloc: max_splits must be positive");
  if (batch->num_tokens != batch->num_seqs)
    return set_error(Q38A_ERR_INVALID, "attention_decode_noalloc: one token per sequence required (M %d, B %d)",
                     batch->num_tokens, batch->num_seqs);
  return launch_attention_decode_noalloc(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

size_t q38a_noalloc_scratch_floats(void) { return noalloc_scratch_floats(); }

int q38a_attention_prefill(const q38a_attention_params* p, const q38a_batch_desc* batch,
                           const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_attention(p, batch, kv, false)) return rc;
  return launch_attention_prefill(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

int q38a_ragged_scratch_init(float* split_scratch, void* stream) {
  clear_error();
  if (!split_scratch) return set_error(Q38A_ERR_INVALID, "ragged_scratch_init: scratch is null");
  return ragged_scratch_init(split_scratch, static_cast<hipStream_t>(stream));
}

int q38a_attention_ragged(const q38a_attention_params* p, const q38a_batch_desc* batch,
                          const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_attention(p, batch, kv, true)) return rc;
  return launch_attention_ragged(*p, *batch, *kv, static_cast<hipStream_t>(stream));
}

}  // extern "C"
