// Device code of the fused q/k offset-RMSNorm + partial RoPE + KV append, shared by the append
// launch (append.hip) and the in-projection GEMM's fused epilogue (qgemm.hip). See append.hip for
// the semantics and the exactness argument.
#pragma once

#include "common.hpp"

// No multiply-add fusion in this code: every product and sum rounds on its own, as in the
// reference's x86-64 build. (Restored to the default at the end of this header.)
#pragma clang fp contract(off)


namespace q38a {
namespace {

// Correctly rounded binary32 division and square root, as the reference's IEEE single-precision
// code computes them: HIP compiles fp32 division and sqrtf to correctly rounded sequences
// (-fhip-fp32-correctly-rounded-divide-sqrt, clang's default, which the build keeps), at a
// fraction of the cost of the binary64 operations (the quantiser divides every element).
#ifdef __FAST_MATH__
#error "the append must round division and square root correctly: build without fast-math"
#endif
__device__ inline float div_rn(float a, float b) { return a / b; }
__device__ inline float sqrt_rn(float a) { return __builtin_sqrtf(a); }

constexpr int kWavesPerBlock = 4;

// Position of the lowest set bit of a nonzero float: x = odd * 2^lowest_bit_of(x).
__device__ inline int lowest_bit_of(float x) {
  const uint32_t b = as_u32(x) & 0x7fffffffu;
  const uint32_t e = b >> 23, m = b & 0x7fffffu;
  return e == 0 ? -149 + __builtin_ctz(m) : int(e) - 150 + __builtin_ctz(m | 0x800000u);
}

// floor(log2 x) for a positive normal double
__device__ inline int exponent_of_f64(double x) {
  return int((__builtin_bit_cast(uint64_t, x) >> 52) & 0x7ff) - 1023;
}

// Sum over the wave in double, in a fixed tree order (the callers use it only where every order
// gives the same, exact, sum).
__device__ inline double wave_sum(double v) {
  auto add = [](double x, uint32_t lo, uint32_t hi) {
    return x + __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
  };
  auto lo = [](double x) { return uint32_t(__builtin_bit_cast(uint64_t, x)); };
  auto hi = [](double x) { return uint32_t(__builtin_bit_cast(uint64_t, x) >> 32); };
  v = add(v, dpp_move<kDppXor1>(lo(v)), dpp_move<kDppXor1>(hi(v)));
  v = add(v, dpp_move<kDppXor2>(lo(v)), dpp_move<kDppXor2>(hi(v)));
  v = add(v, dpp_move<kDppHalfMirror>(lo(v)), dpp_move<kDppHalfMirror>(hi(v)));
  v = add(v, dpp_move<kDppMirror>(lo(v)), dpp_move<kDppMirror>(hi(v)));
  {
    const auto a = __builtin_amdgcn_permlane16_swap(lo(v), lo(v), false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(hi(v), hi(v), false, false);
    v = __builtin_bit_cast(double, (uint64_t(b[0]) << 32) | a[0]) + __builtin_bit_cast(double, (uint64_t(b[1]) << 32) | a[1]);
  }
  {
    const auto a = __builtin_amdgcn_permlane32_swap(lo(v), lo(v), false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(hi(v), hi(v), false, false);
    v = __builtin_bit_cast(double, (uint64_t(b[0]) << 32) | a[0]) + __builtin_bit_cast(double, (uint64_t(b[1]) << 32) | a[1]);
  }
  return v;
}

// max over each 16-lane row (a 64-dim quantisation group), the result in every lane of the row
__device__ inline float row16_max(float x) {
  auto mx = [](float a, uint32_t b) { return fmaxf(a, __uint_as_float(b)); };
  x = mx(x, dpp_move<kDppRor8>(__float_as_uint(x)));
  x = mx(x, dpp_move<kDppRor4>(__float_as_uint(x)));
  x = mx(x, dpp_move<kDppXor2>(__float_as_uint(x)));
  return mx(x, dpp_move<kDppXor1>(__float_as_uint(x)));
}

struct AppendArgs {
  const uint16_t* proj;
  int ld_proj;
  const float* q_norm;
  const float* k_norm;
  float eps;
  int nq, nkv;
  uint16_t* q_out;
  int attn_layer;
  const float* rope;  // [rope_rows][64]
  int rope_rows;
};

// Per-row loads, issued for all of a wave's rows before any row is computed (each row's chain is
// proj + position, then the RoPE row, then tok_seq -> seq_slot -> block_table for a k or v row).
struct RowLoads {
  int m, r, pos;
  uint2 raw;
  float4 c4, s4;
  int page;
  bool store_ok;
};

// Offset-RMSNorm and partial RoPE of one q or k row in place: lane l holds dims 4l .. 4l + 3.
// wv: this lane's four norm weights (q_norm or k_norm, already 1 + w).
__device__ inline void norm_rope_row(const AppendArgs& p, double* stage, int lane, bool pos_ok, const float4& wv,
                                     const float4& c4, const float4& s4, float (&x)[4]) {
  // ---- sum of squares, bit-identical to the left-to-right double sum ----------------------------
  int lmin = 1 << 20;
  double part = 0.0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    part += double(x[e]) * double(x[e]);
    if (x[e] != 0.0f) lmin = min(lmin, lowest_bit_of(x[e]));
  }
  lmin = wave_min_i32(lmin);
  // The tree sum equals the left-to-right sum when every partial sum of either order is exact: all
  // partial sums, multiples of 2^(2 lmin) no larger than the total (< 2^(H + 1)), fit in 53 bits,
  // H + 1 - 2 lmin <= 53, with H from the tree sum itself and one bit of margin for its own
  // rounding (a zero total: every square is zero). A second test, nonzero magnitudes within 14
  // binades, admitted no N(0,1) row that this one rejects (0.6% of rows fall back either way), and
  // cost two more wave reductions per row.
  const double tree = wave_sum(part);
  double ss;
  if (tree == 0.0 || exponent_of_f64(tree) + 2 - 2 * lmin <= 53) {
    ss = tree;  // exact in any order
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) stage[4 * lane + e] = double(x[e]);  // converted off the serial chain
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    double seq = 0.0;
    if (lane == 0) {
      // fma(v, v, seq) = fl(seq + v * v) = fl(seq + fl(v * v)): v is a bf16 value, so v * v is exact
      // in double and the single rounding is the reference's; one instruction less per element.
      // The loads go out 16 at a time ahead of their part of the chain (one LDS round trip per 16
      // elements instead of per element).
      for (int i0 = 0; i0 < kHeadDim; i0 += 16) {
        double v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = stage[i0 + j];
#pragma unroll
        for (int j = 0; j < 16; ++j) seq = __builtin_fma(v[j], v[j], seq);
      }
    }
    ss = __shfl(seq, 0, 64);
  }
  const float mean = float(ss / double(kHeadDim));
  const float rs = div_rn(1.0f, sqrt_rn(mean + p.eps));
  const float wl[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = (x[e] * rs) * wl[e];

  // ---- partial RoPE: lanes 0-7 own dims 0-31, lanes 8-15 own dims 32-63 -------------------------
  float partner[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) partner[e] = __uint_as_float(dpp_move<kDppRor8>(__float_as_uint(x[e])));
  if (lane < 16 && pos_ok) {
    const float c[4] = {c4.x, c4.y, c4.z, c4.w}, s[4] = {s4.x, s4.y, s4.z, s4.w};
    if (lane < 8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = x[e] * c[e] - partner[e] * s[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = x[e] * c[e] + partner[e] * s[e];
    }
  }
}

// q as stored: fp16 (RNE) of this lane's four dims; NaN when the position has no RoPE row.
__device__ inline uint2 q_row_bits(const float (&x)[4], bool pos_ok) {
  uint16_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = pos_ok ? f16_bits(x[e]) : uint16_t(0x7e00u);  // NaN flags a bad position
  return uint2{uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
}

// int8 quantisation of a 256-dim row: the group g = lane / 16 covers dims [64g, 64g + 64); returns
// this lane's four codes (byte e = dim 4 lane + e) and the group's fp16 scale bits in *sbits.
__device__ inline uint32_t quantize_row_int8(const float (&x)[4], uint16_t* sbits) {
  const float amax = row16_max(fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
  *sbits = f16_bits(div_rn(amax, 127.0f));
  const float scale = f16_value(*sbits);
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float q = 0.0f;
    if (scale > 0.0f) q = fminf(fmaxf(__builtin_rintf(div_rn(x[e], scale)), -127.0f), 127.0f);
    packed |= (uint32_t(int32_t(q)) & 0xffu) << (8 * e);
  }
  return packed;
}

// An int8 K or V row of (page, head, token in page) into the cache (int8 pages, not VT).
__device__ inline void store_row_int8(const KvArgs& kv, int attn_layer, int page, int head, int tok, bool is_k,
                                      int lane, uint32_t packed, uint16_t sbits) {
  uint8_t* base = kv.pool + size_t(attn_layer) * kv.layer_stride + size_t(page) * kv.page_bytes;
  const size_t row = is_k ? kv.layout.k_row(head, tok) : kv.layout.v_row(head, tok);
  *reinterpret_cast<uint32_t*>(base + row + 4 * lane) = packed;
  if ((lane & 15) == 0) {
    const size_t so = is_k ? kv.layout.k_scales(head, tok) : kv.layout.v_scales(head, tok);
    reinterpret_cast<uint16_t*>(base + so)[lane >> 4] = sbits;
  }
}

// One (token, head row): norm, RoPE, then the q store or the page-row store, from its loads.
__device__ inline void append_row(const AppendArgs& p, const KvArgs& kv, double* stage, int lane, const RowLoads& L) {
  const int m = L.m, r = L.r, pos = L.pos, page = L.page;
  const bool store_ok = L.store_ok;
  const uint2 raw = L.raw;
  const bool is_q = r < p.nq, is_k = !is_q && r < p.nq + p.nkv;
  const bool pos_ok = pos >= 0 && pos < p.rope_rows;
  float x[4] = {bf16_value(uint16_t(raw.x)), bf16_value(uint16_t(raw.x >> 16)), bf16_value(uint16_t(raw.y)),
                bf16_value(uint16_t(raw.y >> 16))};

  if (is_q || is_k) {
    const float4 wv = *reinterpret_cast<const float4*>((is_q ? p.q_norm : p.k_norm) + 4 * lane);
    norm_rope_row(p, stage, lane, pos_ok, wv, L.c4, L.s4, x);
  }

  if (is_q) {
    *reinterpret_cast<uint2*>(p.q_out + (size_t(m) * p.nq + r) * kHeadDim + 4 * lane) = q_row_bits(x, pos_ok);
    return;
  }

  const int head = is_k ? r - p.nq : r - p.nq - p.nkv;
  if (!store_ok) return;
  const int tok = pos % kPageTokens;
  uint8_t* base = kv.pool + size_t(p.attn_layer) * kv.layer_stride + size_t(page) * kv.page_bytes;
  const bool vt = !is_k && kv.layout.dtype == Q38A_KV_INT8_VT;  // V codes transposed, scales group-major

  if (kv.layout.dtype == Q38A_KV_BF16) {
    const size_t row = is_k ? kv.layout.k_row(head, tok) : kv.layout.v_row(head, tok);
    uint2 out;
    out.x = uint32_t(bf16_bits(x[0])) | (uint32_t(bf16_bits(x[1])) << 16);
    out.y = uint32_t(bf16_bits(x[2])) | (uint32_t(bf16_bits(x[3])) << 16);
    *reinterpret_cast<uint2*>(base + row + 8 * lane) = out;
    return;
  }

  uint16_t sbits;
  const uint32_t packed = quantize_row_int8(x, &sbits);
  if (vt) {
    // dim 4 lane + e of this token: byte `tok` of V^T row (head, dim)
#pragma unroll
    for (int e = 0; e < 4; ++e) base[kv.layout.vt_code(head, 4 * lane + e, tok)] = uint8_t(packed >> (8 * e));
    if ((lane & 15) == 0) *reinterpret_cast<uint16_t*>(base + kv.layout.vt_scale(head, lane >> 4, tok)) = sbits;
    return;
  }
  store_row_int8(kv, p.attn_layer, page, head, tok, is_k, lane, packed, sbits);
}

// The dependent loads of one (token m, head row r) job: its proj slice (raw, 4 bf16 of this lane's
// dims, given by the caller), position, RoPE row, and for k and v rows the cache page.
__device__ inline void row_meta(const AppendArgs& p, const BatchArgs& batch, const KvArgs& kv, int lane, RowLoads& L) {
  // a k or v row's block-table row (tok_seq -> seq_slot) does not depend on the position, so its two
  // loads go out before the position has returned: three dependent round trips to the page id
  // instead of four
  int slot = 0;
  if (L.r >= p.nq) slot = batch.seq_slot[batch.tok_seq[L.m]];
  const int pos = L.pos;
  const bool pos_ok = pos >= 0 && pos < p.rope_rows;
  L.c4 = float4{1.f, 1.f, 1.f, 1.f};
  L.s4 = float4{0.f, 0.f, 0.f, 0.f};
  if (L.r < p.nq + p.nkv && lane < 16 && pos_ok) {  // q and k rows: cos/sin of this lane's dims
    const float* cs = p.rope + size_t(pos) * kRotaryDim + 4 * (lane & 7);
    L.c4 = *reinterpret_cast<const float4*>(cs);
    L.s4 = *reinterpret_cast<const float4*>(cs + 32);
  }
  const int page_idx = pos / kPageTokens;
  L.store_ok = L.r >= p.nq && pos_ok && page_idx < kv.max_pages_per_seq;
  L.page = 0;
  if (L.store_ok) L.page = kv.block_table[size_t(slot) * kv.max_pages_per_seq + page_idx];
}

}  // namespace
}  // namespace q38a

// the default contraction again for the code of the including file
#pragma clang fp contract(fast)
