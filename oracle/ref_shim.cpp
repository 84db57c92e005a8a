// extern "C" entry points over the reference's own CPU implementation of the attention step
// (reference src/ref/ops.cpp:79-171, compiled from /root/reference by oracle/Makefile into
// oracle/_ref/). Used only by the tests (to pin the oracle restatement) and by the benchmark's
// CPU-baseline leg; nothing on the product path loads it.
#include <cstring>

#include "ref/ops.h"

using qwen38::ModelConfig;
namespace ref = qwen38::ref;

namespace {
ModelConfig make_cfg(int nq, int nkv, int rotary_dim, double theta, float eps) {
  ModelConfig c;
  c.num_attention_heads = nq;
  c.num_key_value_heads = nkv;
  c.head_dim = 256;
  c.rotary_dim = rotary_dim;
  c.rope_theta = theta;
  c.rms_norm_eps = eps;
  return c;
}
}  // namespace

extern "C" {

// kv_dtype: 0 int8, 1 bf16, 2 f32. Writes q [nq][256], k/v rows [nkv][256] as the reference
// KvStore holds them (dequantized floats).
void refx_qk_norm_rope_append_token(int nq, int nkv, int rotary_dim, double theta, float eps, const float* proj_row,
                                    int pos, const float* q_norm, const float* k_norm, float* q_out, float* k_out,
                                    float* v_out, int kv_dtype, int exact) {
  const ModelConfig cfg = make_cfg(nq, nkv, rotary_dim, theta, eps);
  // The reference store is indexed by position; keep one (grown on demand) instead of zeroing a
  // position-sized store on every call.
  static ref::KvStore st;
  if (st.kv_heads != nkv || st.capacity <= pos) st.resize(nkv, 256, pos + 1 > st.capacity ? pos + 1 : st.capacity);
  const ref::KvDtype d = kv_dtype == 0 ? ref::KvDtype::Int8 : kv_dtype == 1 ? ref::KvDtype::BF16 : ref::KvDtype::F32;
  ref::qk_norm_rope_append(cfg, proj_row, pos, q_norm, k_norm, q_out, st, d, exact != 0);
  for (int h = 0; h < nkv; ++h) {
    std::memcpy(k_out + size_t(h) * 256, st.k_at(h, pos), 256 * sizeof(float));
    std::memcpy(v_out + size_t(h) * 256, st.v_at(h, pos), 256 * sizeof(float));
  }
}

void refx_int8_group_roundtrip(float* x, int n) { ref::int8_group_roundtrip(x, n); }

// Persistent KvStore handles (so timing loops do not copy the cache).
void* refx_store_new(int nkv, int cap) {
  auto* st = new ref::KvStore();
  st->resize(nkv, 256, cap);
  return st;
}
void refx_store_free(void* h) { delete static_cast<ref::KvStore*>(h); }
float* refx_store_k(void* h) { return static_cast<ref::KvStore*>(h)->k.data(); }
float* refx_store_v(void* h) { return static_cast<ref::KvStore*>(h)->v.data(); }

// ref::attention_token over a store: q [nq][256], gate [nq*256], out [nq*256] (bf16-rounded).
void refx_attention_token(void* store, int nq, int nkv, const float* q, const float* gate, int pos, float* out,
                          int exact) {
  const ModelConfig cfg = make_cfg(nq, nkv, 64, 1e7, 1e-6f);
  ref::attention_token(cfg, q, gate, pos, *static_cast<ref::KvStore*>(store), out, exact != 0);
}

}  // extern "C"
