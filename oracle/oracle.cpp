// CPU oracle for the ragged paged-KV attention step (test infrastructure only).
//
// This file restates, in plain C++, the reference engine's CPU implementation of the
// full-attention step of Qwen3.8 so that the HIP kernels can be checked against it:
//   - fp16 / bf16 round-to-nearest-even conversions      reference include/qwen38/common.h:38-80
//   - int8 per-64-group quantizer (fp16 scale, RNE, ±127) reference src/ref/ops.cpp:79-90
//   - offset RMSNorm with a double sum of squares         reference src/ref/ops.cpp:94-99
//   - partial rotate-half RoPE through libm powf/cosf/sinf reference src/ref/ops.cpp:101-111
//   - q/k norm + RoPE + KV append for one token           reference src/ref/ops.cpp:125-142
//   - exact (double) softmax attention + sigmoid gate     reference src/ref/ops.cpp:144-171
//   - paged KV byte layout (K, V, K scales, V scales)     reference src/kernels/kernels.h:41-70,
//                                                          docs/FORMAT.md:185-196
// Unlike the reference KvStore (src/ref/ops.h:54-62), which keeps dequantized floats, this
// restatement emits the int8 code bytes and fp16 scale bits, written into a page pool with the
// reference byte layout, so that the device cache can be compared byte for byte.
//
// Only the test suite, the smoke check and the benchmark's CPU-baseline leg load this library;
// the product path never does. Build: `make -C oracle` (compiled with -ffp-contract=off so that
// no multiply-add is fused, matching the reference's x86-64 build, which has no FMA).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

constexpr int kHeadDim = 256;
constexpr int kPageTokens = 64;

uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// ---- 16-bit formats (common.h:38-80) ------------------------------------------------------------
float bf16_to_f32(uint16_t b) { return u2f(uint32_t(b) << 16); }

uint16_t f32_to_bf16(float f) {
  const uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = std::ldexp(float(m), -24);
    return m == 0 ? u2f(sign) : (sign ? -v : v);
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return uint16_t(sign | 0x7e00u);
  if (a >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
  if (a < 0x38800000u) return uint16_t(sign | uint32_t(std::nearbyint(u2f(a) * 16777216.0f)));
  const uint32_t v = (a + 0xfffu + ((a >> 13) & 1u)) >> 13;
  return uint16_t(sign | (v - (112u << 10)));
}

float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
float sigmoidf_ref(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// ---- per-token math (ops.cpp:79-111) ----------------------------------------------------------
// One 64-element group: returns the fp16 scale bits and writes the int8 codes.
uint16_t quantize_group(const float* x, int8_t* codes) {
  float amax = 0.0f;
  for (int i = 0; i < 64; ++i) amax = std::max(amax, std::fabs(x[i]));
  const uint16_t sbits = f32_to_f16(amax / 127.0f);
  const float scale = f16_to_f32(sbits);
  for (int i = 0; i < 64; ++i) {
    float q = 0.0f;
    if (scale > 0.0f) q = std::min(std::max(std::nearbyint(x[i] / scale), -127.0f), 127.0f);
    codes[i] = int8_t(q);
  }
  return sbits;
}

void rms_offset_norm(const float* x, int n, const float* w, float eps, float* y) {
  double ss = 0;
  for (int i = 0; i < n; ++i) ss += double(x[i]) * x[i];
  const float r = 1.0f / std::sqrt(float(ss / n) + eps);
  for (int i = 0; i < n; ++i) y[i] = x[i] * r * w[i];
}

void rope_cos_sin(int pos, double theta, int rotary_dim, float* cs) {
  const int half = rotary_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float inv = 1.0f / std::pow(float(theta), float(2 * i) / float(rotary_dim));
    const float angle = float(pos) * inv;
    cs[i] = std::cos(angle);
    cs[half + i] = std::sin(angle);
  }
}

void rope_apply(float* y, int rotary_dim, const float* cs) {
  const int half = rotary_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float c = cs[i], s = cs[half + i];
    const float x1 = y[i], x2 = y[i + half];
    y[i] = x1 * c - x2 * s;
    y[i + half] = x2 * c + x1 * s;
  }
}

// ---- paged layout (kernels.h:41-70) -----------------------------------------------------------
// dtype 0: int8 (reference), 1: bf16 (reference), 2: int8 with V transposed per page (this
// library's variant of the int8 format: the same codes and scales at other offsets, V^T
// [kvh][4 quarters][256][16 tokens], V scales [kvh][4][64]; K and its scales as in dtype 0).
struct Layout {
  int kv_heads;
  int dtype;
  bool int8() const { return dtype != 1; }
  size_t elem() const { return int8() ? 1 : 2; }
  size_t k_off(int h, int t) const { return (size_t(h) * kPageTokens + t) * kHeadDim * elem(); }
  size_t v_off(int h, int t) const { return size_t(kv_heads) * kPageTokens * kHeadDim * elem() + k_off(h, t); }
  size_t ks_off(int h, int t) const {
    return 2 * size_t(kv_heads) * kPageTokens * kHeadDim + (size_t(h) * kPageTokens + t) * 8;
  }
  size_t vs_off(int h, int t) const { return ks_off(h, t) + size_t(kv_heads) * kPageTokens * 8; }
  // dtype 2: V code of (h, dim d, token t) and V scale of (h, group g, token t)
  size_t vt_code_off(int h, int d, int t) const {
    return size_t(kv_heads) * kPageTokens * kHeadDim + ((size_t(h) * 4 + t / 16) * kHeadDim + d) * 16 + t % 16;
  }
  size_t vt_scale_off(int h, int g, int t) const {
    return 2 * size_t(kv_heads) * kPageTokens * kHeadDim + size_t(kv_heads) * kPageTokens * 8 +
           ((size_t(h) * 4 + g) * kPageTokens + t) * 2;
  }
  size_t page_bytes() const {
    return int8() ? 2 * size_t(kv_heads) * kPageTokens * (kHeadDim + 8)
                  : 2 * size_t(kv_heads) * kPageTokens * kHeadDim * 2;
  }
};

void store_row(uint8_t* page, const Layout& L, bool is_v, int h, int t, const float* y) {
  if (L.dtype == 1) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(page + (is_v ? L.v_off(h, t) : L.k_off(h, t)));
    for (int d = 0; d < kHeadDim; ++d) dst[d] = f32_to_bf16(y[d]);
    return;
  }
  if (L.dtype == 2 && is_v) {  // same quantisation, codes scattered down the V^T columns
    int8_t codes[kHeadDim];
    for (int g = 0; g < 4; ++g) {
      const uint16_t s = quantize_group(y + 64 * g, codes + 64 * g);
      std::memcpy(page + L.vt_scale_off(h, g, t), &s, 2);
    }
    for (int d = 0; d < kHeadDim; ++d) page[L.vt_code_off(h, d, t)] = uint8_t(codes[d]);
    return;
  }
  int8_t* dst = reinterpret_cast<int8_t*>(page + (is_v ? L.v_off(h, t) : L.k_off(h, t)));
  uint16_t* sc = reinterpret_cast<uint16_t*>(page + (is_v ? L.vs_off(h, t) : L.ks_off(h, t)));
  for (int g = 0; g < 4; ++g) sc[g] = quantize_group(y + 64 * g, dst + 64 * g);
}

void load_row(const uint8_t* page, const Layout& L, bool is_v, int h, int t, float* out) {
  if (L.dtype == 1) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(page + (is_v ? L.v_off(h, t) : L.k_off(h, t)));
    for (int d = 0; d < kHeadDim; ++d) out[d] = bf16_to_f32(src[d]);
    return;
  }
  if (L.dtype == 2 && is_v) {
    for (int d = 0; d < kHeadDim; ++d) {
      uint16_t s;
      std::memcpy(&s, page + L.vt_scale_off(h, d / 64, t), 2);
      out[d] = float(int8_t(page[L.vt_code_off(h, d, t)])) * f16_to_f32(s);
    }
    return;
  }
  const int8_t* src = reinterpret_cast<const int8_t*>(page + (is_v ? L.v_off(h, t) : L.k_off(h, t)));
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(page + (is_v ? L.vs_off(h, t) : L.ks_off(h, t)));
  for (int d = 0; d < kHeadDim; ++d) out[d] = float(src[d]) * f16_to_f32(sc[d / 64]);
}

}  // namespace

extern "C" {

// Scalar conversions, exported for the exhaustive format tests.
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_f32_to_bf16(float f) { return f32_to_bf16(f); }
float orc_bf16_to_f32(uint16_t b) { return bf16_to_f32(b); }

// Bulk f32 -> f16 bits (exhaustive tests over bit patterns).
void orc_f32_to_f16_n(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}
void orc_f32_to_bf16_n(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(x[i]);
}

// int8 quantizer over n (multiple of 64) floats: codes[n], scale bits[n/64] (ops.cpp:79-90).
void orc_quantize_int8(const float* x, int n, int8_t* codes, uint16_t* scales) {
  for (int g = 0; g < n / 64; ++g) scales[g] = quantize_group(x + 64 * g, codes + 64 * g);
}

// RoPE cos/sin for positions [pos_begin, pos_begin + count): out[count][rotary_dim] laid out
// as [cos(0..half) | sin(0..half)] per position (ops.cpp:101-111).
void orc_rope_table(int pos_begin, int count, double theta, int rotary_dim, float* out) {
  for (int p = 0; p < count; ++p) rope_cos_sin(pos_begin + p, theta, rotary_dim, out + size_t(p) * rotary_dim);
}

// Offset RMSNorm of one row (ops.cpp:94-99).
void orc_rms_offset_norm(const float* x, int n, const float* w, float eps, float* y) { rms_offset_norm(x, n, w, eps, y); }

// q/k norm + RoPE + KV append for the tokens of a ragged batch (ops.cpp:125-142 per token).
//   proj      [M][ld_proj] bf16 bits: [q nq*256 | gate nq*256 | k nkv*256 | v nkv*256]
//   tok_pos   [M], tok_seq [M], seq_slot [B]
//   q_out     [M][nq][256] fp16 bits
//   pool      one attention layer of the page pool (num_pages * page_bytes), updated in place
//   block_table [slots][max_pages]
void orc_qk_norm_rope_append(const uint16_t* proj, int ld_proj, int m_tokens, const int* tok_pos, const int* tok_seq,
                             const int* seq_slot, const float* q_norm, const float* k_norm, float eps, double theta,
                             int rotary_dim, int nq, int nkv, uint16_t* q_out, uint8_t* pool, int kv_dtype,
                             const int* block_table, int max_pages) {
  const Layout L{nkv, kv_dtype};
  std::vector<float> x(kHeadDim), y(kHeadDim), cs(rotary_dim);
  for (int m = 0; m < m_tokens; ++m) {
    const uint16_t* row = proj + size_t(m) * ld_proj;
    const int pos = tok_pos[m];
    rope_cos_sin(pos, theta, rotary_dim, cs.data());
    for (int h = 0; h < nq; ++h) {
      for (int d = 0; d < kHeadDim; ++d) x[d] = bf16_to_f32(row[h * kHeadDim + d]);
      rms_offset_norm(x.data(), kHeadDim, q_norm, eps, y.data());
      rope_apply(y.data(), rotary_dim, cs.data());
      for (int d = 0; d < kHeadDim; ++d) q_out[(size_t(m) * nq + h) * kHeadDim + d] = f32_to_f16(y[d]);
    }
    const int slot = seq_slot[tok_seq[m]];
    const int page = block_table[size_t(slot) * max_pages + pos / kPageTokens];
    uint8_t* pg = pool + size_t(page) * L.page_bytes();
    const int t = pos % kPageTokens;
    for (int h = 0; h < nkv; ++h) {
      const uint16_t* kr = row + size_t(2 * nq + h) * kHeadDim;
      const uint16_t* vr = row + size_t(2 * nq + nkv + h) * kHeadDim;
      for (int d = 0; d < kHeadDim; ++d) x[d] = bf16_to_f32(kr[d]);
      rms_offset_norm(x.data(), kHeadDim, k_norm, eps, y.data());
      rope_apply(y.data(), rotary_dim, cs.data());
      store_row(pg, L, false, h, t, y.data());
      for (int d = 0; d < kHeadDim; ++d) x[d] = bf16_to_f32(vr[d]);
      store_row(pg, L, true, h, t, x.data());
    }
  }
}

// Quantize/convert raw K or V rows straight into the pool (no norm, no RoPE): used to build
// synthetic prior context "with the reference quantizer".
//   rows [n][nkv][256] float; positions pos0.. pos0+n-1 of `slot`.
void orc_fill_rows(const float* k_rows, const float* v_rows, int n, int pos0, int slot, int nkv, uint8_t* pool,
                   int kv_dtype, const int* block_table, int max_pages) {
  const Layout L{nkv, kv_dtype};
  for (int i = 0; i < n; ++i) {
    const int pos = pos0 + i;
    uint8_t* pg = pool + size_t(block_table[size_t(slot) * max_pages + pos / kPageTokens]) * L.page_bytes();
    for (int h = 0; h < nkv; ++h) {
      store_row(pg, L, false, h, pos % kPageTokens, k_rows + (size_t(i) * nkv + h) * kHeadDim);
      store_row(pg, L, true, h, pos % kPageTokens, v_rows + (size_t(i) * nkv + h) * kHeadDim);
    }
  }
}

// Dequantized cache of one sequence: k/v [nkv][len][256] floats (what the kernels see).
void orc_read_back(const uint8_t* pool, int kv_dtype, int nkv, const int* block_table, int max_pages, int slot,
                   int len, float* k, float* v) {
  const Layout L{nkv, kv_dtype};
  for (int pos = 0; pos < len; ++pos) {
    const uint8_t* pg = pool + size_t(block_table[size_t(slot) * max_pages + pos / kPageTokens]) * L.page_bytes();
    for (int h = 0; h < nkv; ++h) {
      load_row(pg, L, false, h, pos % kPageTokens, k + (size_t(h) * len + pos) * kHeadDim);
      load_row(pg, L, true, h, pos % kPageTokens, v + (size_t(h) * len + pos) * kHeadDim);
    }
  }
}

// Exact attention of one query token at `pos` over k/v[0..pos] (ops.cpp:144-171).
//   q [nq][256] floats (fp16-exact values), gate [nq*256] floats (bf16-exact), k/v [nkv][cap][256]
//   out [nq*256] floats, bf16-rounded.
void orc_attention_token(int nq, int nkv, const float* q, const float* gate, int pos, const float* k, const float* v,
                         int cap, float* out) {
  const int group = nq / nkv;
  const double scale = 1.0 / std::sqrt(double(kHeadDim));
  std::vector<double> s(size_t(pos) + 1);
  for (int h = 0; h < nq; ++h) {
    const int kvh = h / group;
    double mx = -1e300;
    for (int j = 0; j <= pos; ++j) {
      const float* kr = k + (size_t(kvh) * cap + j) * kHeadDim;
      double dot = 0;
      for (int d = 0; d < kHeadDim; ++d) dot += double(q[size_t(h) * kHeadDim + d]) * kr[d];
      s[j] = dot * scale;
      mx = std::max(mx, s[j]);
    }
    double l = 0;
    for (int j = 0; j <= pos; ++j) {
      s[j] = std::exp(s[j] - mx);
      l += s[j];
    }
    for (int d = 0; d < kHeadDim; ++d) {
      double o = 0;
      for (int j = 0; j <= pos; ++j) o += s[j] * v[(size_t(kvh) * cap + j) * kHeadDim + d];
      const float val = float(o / l) * sigmoidf_ref(gate[size_t(h) * kHeadDim + d]);
      out[size_t(h) * kHeadDim + d] = round_bf16(val);
    }
  }
}

// Ragged batch attention straight from the page pool: every token m of sequence b attends to
// positions [0, tok_pos[m]] of its slot (decode rows and prefill chunks alike).
//   q [M][nq][256] fp16 bits, gate rows at proj-like stride ld_gate (bf16 bits), out [M][nq*256] bf16 bits.
void orc_attention_ragged(int nq, int nkv, int num_seqs, const int* seq_start, const int* seq_slot, const int* tok_pos,
                          const uint16_t* q16, const uint16_t* gate, int ld_gate, const uint8_t* pool, int kv_dtype,
                          const int* block_table, int max_pages, uint16_t* out) {
  std::vector<float> qf(size_t(nq) * kHeadDim), gf(size_t(nq) * kHeadDim), of(size_t(nq) * kHeadDim);
  for (int b = 0; b < num_seqs; ++b) {
    int len = 0;
    for (int m = seq_start[b]; m < seq_start[b + 1]; ++m) len = std::max(len, tok_pos[m] + 1);
    if (len == 0) continue;
    std::vector<float> k(size_t(nkv) * len * kHeadDim), v(k.size());
    orc_read_back(pool, kv_dtype, nkv, block_table, max_pages, seq_slot[b], len, k.data(), v.data());
    for (int m = seq_start[b]; m < seq_start[b + 1]; ++m) {
      for (size_t e = 0; e < qf.size(); ++e) qf[e] = f16_to_f32(q16[size_t(m) * nq * kHeadDim + e]);
      for (size_t e = 0; e < gf.size(); ++e) gf[e] = bf16_to_f32(gate[size_t(m) * ld_gate + e]);
      orc_attention_token(nq, nkv, qf.data(), gf.data(), tok_pos[m], k.data(), v.data(), len, of.data());
      for (size_t e = 0; e < of.size(); ++e) out[size_t(m) * nq * kHeadDim + e] = f32_to_bf16(of[e]);
    }
  }
}

// ---- BQ weights and the projection GEMMs (reference docs/FORMAT.md 2, src/bq_host.cpp,
//      src/kernels/qgemm.cu:285-384) --------------------------------------------------------------
// The file layout, stated from the format description: slab (kb, nb) = 16 k x 64 n, stored
// nb-major; lane 4g + t owns column 64 nb + 8 j + g (j < 8) and rows 16 kb + 2t + {0, 1, 8, 9};
// pair q = 2j + h holds rows 16 kb + 2t + 8h + {0, 1}; lo word q / 4 carries the first element's
// nibble at bit 4 (q % 4) and the second's at bit 16 + 4 (q % 4); bq5 hi word: bit q / bit 16 + q;
// bq6 hi words q / 8: bits 2 (q % 8) / 16 + 2 (q % 8); scales: 64-column blocks per (nb, group),
// column 8j + g at entry 8g + j.

// Writes the file planes of W (codes c in [-2^(b-1), 2^(b-1)) [n][k], bf16 scale bits [n][k/64]).
void orc_bq_pack_file(int bits, int n, int k, const int8_t* codes, const uint16_t* scales, uint8_t* lo, uint8_t* hi,
                      uint16_t* sc) {
  const int slabs_k = k / 16;
  const size_t hb = bits == 5 ? 128 : bits == 6 ? 256 : 0;
  std::memset(lo, 0, size_t(n) * k / 2);
  if (hb) std::memset(hi, 0, size_t(n / 64) * slabs_k * hb);
  for (int row = 0; row < n; ++row)
    for (int col = 0; col < k; ++col) {
      const unsigned u = unsigned(int(codes[size_t(row) * k + col]) + (1 << (bits - 1)));
      const int nb = row / 64, nl = row % 64, j = nl / 8, g = nl % 8;
      const int kb = col / 16, kl = col % 16, h = kl / 8, t = (kl % 8) / 2, e = kl % 2;
      const size_t slab = size_t(nb) * slabs_k + kb;
      const int lane = 4 * g + t, q = 2 * j + h;
      uint32_t* w = reinterpret_cast<uint32_t*>(lo + slab * 512 + lane * 16) + q / 4;
      *w |= uint32_t(u & 15u) << (e ? 16 + 4 * (q % 4) : 4 * (q % 4));
      if (bits == 5) *reinterpret_cast<uint32_t*>(hi + slab * 128 + lane * 4) |= uint32_t((u >> 4) & 1u) << (e ? 16 + q : q);
      if (bits == 6)
        reinterpret_cast<uint32_t*>(hi + slab * 256 + lane * 8)[q / 8] |= uint32_t((u >> 4) & 3u) << (e ? 16 + 2 * (q % 8) : 2 * (q % 8));
    }
  for (int row = 0; row < n; ++row)
    for (int gr = 0; gr < k / 64; ++gr) {
      const int nb = row / 64, nl = row % 64;
      sc[(size_t(nb) * (k / 64) + gr) * 64 + (nl % 8) * 8 + nl / 8] = scales[size_t(row) * (k / 64) + gr];
    }
}

// Dequantised weights W[n][k] = bf16(code * scale) from the file planes (BQView::weight).
void orc_bq_file_weight(int bits, int n, int k, const uint8_t* lo, const uint8_t* hi, const uint16_t* sc, float* w) {
  const int slabs_k = k / 16;
  for (int row = 0; row < n; ++row)
    for (int col = 0; col < k; ++col) {
      const int nb = row / 64, nl = row % 64, j = nl / 8, g = nl % 8;
      const int kb = col / 16, kl = col % 16, h = kl / 8, t = (kl % 8) / 2, e = kl % 2;
      const size_t slab = size_t(nb) * slabs_k + kb;
      const int lane = 4 * g + t, q = 2 * j + h;
      uint32_t word;
      std::memcpy(&word, lo + slab * 512 + lane * 16 + 4 * (q / 4), 4);
      unsigned u = (word >> (e ? 16 + 4 * (q % 4) : 4 * (q % 4))) & 15u;
      if (bits == 5) {
        std::memcpy(&word, hi + slab * 128 + lane * 4, 4);
        u |= ((word >> (e ? 16 + q : q)) & 1u) << 4;
      } else if (bits == 6) {
        std::memcpy(&word, hi + slab * 256 + lane * 8 + 4 * (q / 8), 4);
        u |= ((word >> (e ? 16 + 2 * (q % 8) : 2 * (q % 8))) & 3u) << 4;
      }
      const int c = int(u) - (1 << (bits - 1));
      const float s = bf16_to_f32(sc[(size_t(nb) * (k / 64) + col / 64) * 64 + g * 8 + j]);
      w[size_t(row) * k + col] = round_bf16(float(c) * s);
    }
}

// C = A W^T in double over the reference's bf16 weights, then an epilogue (qgemm.cu:285-384):
//   kind 0 StoreBF16: out bf16 [m][ldo] = bf16(float(C) * rs), rs from partials_in (or 1);
//   kind 3 StoreF32:  out fp32 [m][ldo] = float(C) * rs;
//   kind 2 Residual:  residual[m][n] += float(C); xbf = bf16(residual); partials_out[m][n/128] =
//                     sum of squares (double) of the new residual over each 128 columns.
// a: bf16 bits [m][k]; w: fp32 [n][k].
void orc_qgemm(const uint16_t* a, int m, const float* w, int n, int k, int kind, void* out, int ldo, int n_store,
               const float* partials_in, int hidden, float eps, float* residual, uint16_t* xbf, float* partials_out) {
  std::vector<double> arow(static_cast<size_t>(k));
  for (int row = 0; row < m; ++row) {
    for (int i = 0; i < k; ++i) arow[size_t(i)] = bf16_to_f32(a[size_t(row) * k + i]);
    float rs = 1.0f;
    if (partials_in) {
      float ssum = 0.0f;
      for (int b = 0; b < hidden / 128; ++b) ssum += partials_in[size_t(row) * (hidden / 128) + b];
      rs = 1.0f / std::sqrt(ssum / float(hidden) + eps);
    }
    for (int col = 0; col < n; ++col) {
      const float* wr = w + size_t(col) * k;
      double c = 0.0;
      for (int i = 0; i < k; ++i) c += arow[size_t(i)] * wr[i];
      if (kind == 2) {
        float& r = residual[size_t(row) * n + col];
        r = r + float(c);
        xbf[size_t(row) * n + col] = f32_to_bf16(r);
      } else if (col < n_store) {
        const float y = float(c) * rs;
        if (kind == 3) static_cast<float*>(out)[size_t(row) * ldo + col] = y;
        else static_cast<uint16_t*>(out)[size_t(row) * ldo + col] = f32_to_bf16(y);
      }
    }
    if (kind == 2)
      for (int b = 0; b < n / 128; ++b) {
        double ss = 0.0;
        for (int col = 128 * b; col < 128 * b + 128; ++col) {
          const double x = residual[size_t(row) * n + col];
          ss += x * x;
        }
        partials_out[size_t(row) * (n / 128) + b] = float(ss);
      }
  }
}

}  // extern "C"
