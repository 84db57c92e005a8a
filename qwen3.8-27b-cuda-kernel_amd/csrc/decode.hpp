// Split-KV flash-decoding over the paged KV cache on gfx950 MFMA, plus the gated split merge.
//
// Semantics follow reference src/kernels/attention_decode.cu:97-257 (and the exact CPU form
// src/ref/ops.cpp:144-171): for decode row b and q head hq (kv head hq / group), softmax over keys
// [0, seq_pos0[b] + 1) of q.k / 16, weighted sum of V, then out = (acc / l) * sigmoid(gate) in bf16.
//
// MI355X design. Decode is HBM-bound (each KV byte is used once); with GQA 6 and int8 KV it needs
// ~12 flop/byte, which at 8 TB/s is more than the non-packed fp32 VALU can issue alongside the
// int8 widening, so both products run on MFMA and the VALU only widens codes and runs the softmax:
//   * one workgroup = 4 waves (8 in the ragged launch) works on one item (sequence, kv head, run of
//     whole pages, see plan.hpp); each wave takes 16-token blocks of the item's pages in turn;
//   * S^T[16 tok][16 heads] = K[16 tok][256] . Q^T with v_mfma_f32_16x16x32_f16: K codes enter the
//     MFMA exactly (int8 -> fp16 by a byte permute and one packed add), Q as stored (fp16), and the
//     per-(token, 64-dim group) K scale multiplies the four group partials in fp32 afterwards;
//   * O[16 heads][256] += P'[16 heads][16 tok] . V[16 tok][256] with v_mfma_f32_16x16x16_f16:
//     V codes are exact in fp16 and the V scale is folded into P' = p * v_scale per group, rounded
//     once to fp16 (relative error <= 2^-11, a twentieth of the output tolerance);
//   * each wave keeps the next block's loads in flight while it computes the current one;
//   * the S^T accumulator layout (lane = head, 4 tokens) is exactly the A-operand layout of the
//     PV product, so probabilities never leave registers;
//   * K rows are read as 4 x 16-byte loads per lane (a 16-lane group covers 64 contiguous bytes of
//     a row), V rows as 16 x 4-byte loads (16 lanes cover 64 contiguous bytes);
//   * the waves' (max, sum, acc) are merged in LDS and written once per item as a partial;
//     attn_merge_kernel combines partials with the log-sum-exp rule and applies sigmoid(gate).
// bf16 KV pages use the same schedule with bf16 MFMAs for both products; q (fp16) is split exactly
// into two bf16 operands and P likewise into hi + lo.
#pragma once

#include "plan.hpp"

namespace q38a {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxGroup = 8;
constexpr int kMaxMergeSplits = 512;  // max_splits accepted by the launchers
constexpr int kTeam = 8;            // workgroups (splits) per claim team: consecutive ones sit on 8 XCDs
constexpr int kClaimSlots = 4096;   // teams whose first item index is larger use the static schedule
constexpr int kClaimStride = 32;    // ints per counter (one 128-byte line)

struct DecodeArgs {
  const uint16_t* q;
  int nq, nkv, group;
  int attn_layer;
  float* scratch;
  int max_splits;
  int target_items;
  const uint16_t* gate;  // bf16, row stride ld_gate
  int ld_gate;
  uint16_t* out;         // [M][nq * 256] bf16
  // Dynamic block claims (decode_items): balances the decode items against whatever else runs on
  // the CUs (the ragged launch's prefill units), at the price of run-to-run bit reproducibility:
  // which wave sums which block changes the fp32 summation order. Off: a fixed schedule.
  bool dynamic_claims;
  // Items handed out by a launch-wide counter (*queue) instead of a fixed stride: workgroups
  // that start late (behind other work on their CUs) take fewer items.
  bool item_queue;
  // Counters of the two dynamic schedules, in the caller's scratch (one 128-byte line each); they
  // must be zero when the launch starts, and the launch's merge kernel zeroes them again.
  int* claims;  // [kClaimSlots][kClaimStride]
  int* queue;
};


typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
// 16-byte register vector (a native vector type, so copies never go through memory)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Four int8 codes -> two fp16 pairs, exactly: byte b -> fp16 bits 0x64 | (b ^ 0x80) = 1024 + (c + 128),
// then subtract 1152. One XOR per word, one byte permute and one packed add per pair.
__device__ inline void codes4_to_half(uint32_t w, half2_t& lo, half2_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [b0, 64, b1, 64]
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [b2, 64, b3, 64]
  const half2_t bias = {_Float16(1152.0f), _Float16(1152.0f)};
  lo = __builtin_bit_cast(half2_t, a) - bias;
  hi = __builtin_bit_cast(half2_t, b) - bias;
}

__device__ inline half8_t codes16_to_half8(uint32_t w0, uint32_t w1) {
  half2_t a, b, c, d;
  codes4_to_half(w0, a, b);
  codes4_to_half(w1, c, d);
  return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Byte i of two words (codes of tokens r and r + 1 at one dim) -> fp16 pair, exactly.
__device__ inline half2_t code_pair_to_half(uint32_t w_r0, uint32_t w_r1, int i) {
  const uint32_t sel = 0x0C000C00u | (uint32_t(4 + i) << 16) | uint32_t(i);  // [b_r0, 0, b_r1, 0]
  const uint32_t x = __builtin_amdgcn_perm(w_r1, w_r0, sel) ^ 0x64806480u;
  const half2_t bias = {_Float16(1152.0f), _Float16(1152.0f)};
  return __builtin_bit_cast(half2_t, x) - bias;
}

__device__ inline float half_lo(uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w))); }
__device__ inline float half_hi(uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16))); }

__device__ inline short bf16_short(float f) { return short(bf16_bits(f)); }

// x = hi + lo with hi = bf16(x) and lo = bf16(x - hi): a 16-bit significand carried by two bf16
// MFMA operands (relative error ~2^-17 instead of bf16's 2^-9), with fp32's exponent range.
__device__ inline void split_bf16(float x, short& hi, short& lo) {
  const uint16_t h = bf16_bits(x);
  hi = short(h);
  lo = short(bf16_bits(x - bf16_value(h)));
}

// Max over the 4 rows of 16 lanes (lanes l, l ^ 16, l ^ 32, l ^ 48) with VALU lane swaps: each
// v_permlane*_swap exchanges half of its two operands' rows, so the max of its two results is the
// max over each pair of rows.
__device__ inline float max_over_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

constexpr float kDecodeSlack = 8.0f;  // log2 units the running max may lag behind the true max

// Online-softmax state update shared by both page formats. S holds this lane's 4 raw scores
// (head n16, tokens 4 j4 + r); returns p[4] and rescales O when the running max moves. The running
// max only moves when a block's max exceeds it by more than kDecodeSlack, so p <= 2^kDecodeSlack
// and O is rarely rescaled after the first block.
__device__ inline void softmax_step(const float (&S)[4], const bool (&valid)[4], float& m_run, float& l_run,
                                    float (&p)[4], float4_t (&O)[16], int j4) {
  float s2[4], bmax = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    s2[r] = valid[r] ? S[r] : -INFINITY;
    bmax = fmaxf(bmax, s2[r]);
  }
  bmax = max_over_rows(bmax) * kScoreScale;  // kScoreScale > 0 commutes with the max
  const bool bump = bmax > m_run + kDecodeSlack;
  float corr = 1.0f;
  if (__any(bump)) {
    const float mnew = bump ? bmax : m_run;
    corr = __builtin_amdgcn_exp2f(m_run - mnew);  // m_run = -inf gives 0
    const bool empty = m_run == -INFINITY;       // nothing accumulated yet: O rows are zero
    m_run = mnew;
    if (!__all(empty)) {
      // O rows are heads 4 j4 + r; their correction factors live in lanes 4 j4 + r (quad 0)
      float cr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr, 4 * j4 + r, 64);
#pragma unroll
      for (int k = 0; k < 16; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[k][r] *= cr[r];
    }
  }
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s2[r], kScoreScale, -m_run));
    psum += p[r];
  }
  l_run = l_run * corr + psum;
}

// scale of (token r, group g) from a 32-byte fp16 block, [token][group] (int8 pages) or
// [group][token] (V scales of int8 VT pages)
template <bool GroupMajor = false>
__device__ inline float scale_at(const u32x4 (&sc)[2], int r, int g) {
  const int idx = GroupMajor ? g * 4 + r : r * 4 + g;
  const u32x4 w = sc[idx >> 3];
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  const uint32_t word = ws[(idx & 7) >> 1];
  return (idx & 1) ? half_hi(word) : half_lo(word);
}

struct Int8Block {
  u32x4 k[4];         // K codes of token t0 + n16, dims 64g + 16 j4 + [0, 16), g = 0..3
  u32x4 ks[2];        // K scales of tokens t0 + 4 j4 + [0, 4): [token][group] fp16
  uint32_t v[4][4];   // int8: [r][w]: V codes of token t0 + 4 j4 + r, dims 16 n16 + 4 w + [0, 4)
                      // VT:   [g][w]: V codes of dim 64 g + lane, tokens t0 + 4 w + [0, 4)
  u32x4 vs[2];        // V scales of tokens t0 + 4 j4 + [0, 4): [token][group] (int8), [group][token] (VT)
};

// Per-lane byte offsets of a block's loads, relative to the block's uniform bases (page + 256 *
// first token for rows, page + 8 * first token for scales); fixed for the whole item.
struct Int8Offsets {
  uint32_t k, ks, v, vs;
};

template <bool VT>
__device__ inline Int8Offsets int8_offsets(const PageLayout& L, int kvh, int n16, int j4) {
  Int8Offsets o;
  o.k = uint32_t(L.k_row(kvh, n16)) + 16 * j4;
  o.ks = uint32_t(L.k_scales(kvh, 4 * j4));
  if constexpr (VT) {
    o.v = uint32_t(L.vt_code(kvh, n16 + 16 * j4, 0));  // dim = lane; + 1,024 B per 64 dims
    o.vs = uint32_t(L.vt_scale(kvh, 0, 4 * j4));
  } else {
    o.v = uint32_t(L.v_row(kvh, 4 * j4)) + 16 * n16;
    o.vs = uint32_t(L.v_scales(kvh, 4 * j4));
  }
  return o;
}

// pg: the page; in0: the block's first token within it (a multiple of 16). K rows, int8 V rows and
// VT V^T quarters advance by 256 bytes per token, K and int8 V scales by 8, VT V scales by 2.
template <bool VT>
__device__ inline void load_int8_block(Int8Block& d, const uint8_t* pg, int in0, const Int8Offsets& o,
                                       int live_bytes) {
  if constexpr (VT) {
    // K and its scales as for int8 pages. V: a block's V^T quarter is 256 dims x 16 tokens, 4 KB
    // contiguous, so lane l reads the 16 tokens of dims 64 q + l (four 16-byte loads, the wave's
    // loads 1 KB contiguous each); a 4 x 4 word transpose across the four 16-lane rows (two
    // permlane32 and two permlane16 swaps per four words) then leaves lane (n16, j4) with tokens
    // 4 j4 + [0, 4) of dims 64 q + 16 i + n16, the layout the PV MFMAs take.
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pg), short(0), live_bytes, 0x00020000);
    const int srow = kHeadDim * in0, ssc = 8 * in0;  // 16 tokens further = 4,096 B, for K and V^T
    constexpr int kNT = 2;  // cache policy: non-temporal
#pragma unroll
    for (int g = 0; g < 4; ++g)
      d.k[g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.k + 64 * g, srow, kNT));
    d.ks[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.ks, ssc, kNT));
    d.ks[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.ks + 16, ssc, kNT));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.v + 1024 * q, srow, kNT));
      d.v[q][0] = w.x;
      d.v[q][1] = w.y;
      d.v[q][2] = w.z;
      d.v[q][3] = w.w;
    }
    // V scales, group-major: group g's 4 tokens are 8 contiguous bytes, groups 128 B apart
    uint32_t sv[4][2];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, o.vs + 2 * kPageTokens * g, 2 * in0, kNT);
      sv[g][0] = x[0];
      sv[g][1] = x[1];
    }
    d.vs[0] = u32x4{sv[0][0], sv[0][1], sv[1][0], sv[1][1]};
    d.vs[1] = u32x4{sv[2][0], sv[2][1], sv[3][0], sv[3][1]};
  } else {
    // every load is 16 bytes per lane and non-temporal (the bytes are read once): on this page
    // pattern that streams ~7% faster than ordinary loads with 4-byte V words (a read-pattern probe
    // of the decode launch's loads, 432 MB per launch: 6.28 vs 5.88 TB/s). The loads go through a
    // buffer resource over the page whose size is `live_bytes`: 0 turns every load into one that
    // returns zeros without touching memory, so a wave's last iteration keeps the loop's single
    // path without fetching a block again (non-temporal bytes are not kept in the L2, so a repeat
    // is another HBM read).
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pg), short(0), live_bytes, 0x00020000);
    const int srow = kHeadDim * in0, ssc = 8 * in0;
    constexpr int kNT = 2;  // cache policy: non-temporal
#pragma unroll
    for (int g = 0; g < 4; ++g)
      d.k[g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.k + 64 * g, srow, kNT));
    d.ks[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.ks, ssc, kNT));
    d.ks[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.ks + 16, ssc, kNT));
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const u32x4 w =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.v + kHeadDim * rr, srow, kNT));
      d.v[rr][0] = w.x;
      d.v[rr][1] = w.y;
      d.v[rr][2] = w.z;
      d.v[rr][3] = w.w;
    }
    d.vs[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.vs, ssc, kNT));
    d.vs[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o.vs + 16, ssc, kNT));
  }
}

// 4 x 4 transpose of 32-bit words across the four 16-lane rows of a wave: afterwards register i
// of a lane in row j holds what register j held in the lane of row i with the same position in
// its row (two permlane32 swaps exchange the rows 0-1 / 2-3 halves, two permlane16 swaps the odd
// and even rows).
__device__ inline void row_transpose4(uint32_t& a0, uint32_t& a1, uint32_t& a2, uint32_t& a3) {
  auto r = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
  a0 = r[0];
  a2 = r[1];
  r = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
  a1 = r[0];
  a3 = r[1];
  r = __builtin_amdgcn_permlane16_swap(a0, a1, false, false);
  a0 = r[0];
  a1 = r[1];
  r = __builtin_amdgcn_permlane16_swap(a2, a3, false, false);
  a2 = r[0];
  a3 = r[1];
}

// One 16-token block of int8 pages for this lane: S^T = K . Q^T per 64-dim group on fp16 MFMAs
// (codes exact in fp16, q as stored), the group's K scale applied to the fp32 partial; then
// O += P' V with P' = p * v_scale per group rounded once to fp16 (relative error <= 2^-11; V codes
// are exact). Tail: the block may reach past the item's last key (masked).
template <bool Tail, bool VT = false>
__device__ inline void compute_block(const Int8Block& d, const half8_t (&qf)[4][2], int t0, int t_end, float& m_run,
                                     float& l_run, float4_t (&O)[16], int j4) {
  bool valid[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) valid[r] = !Tail || t0 + 4 * j4 + r < t_end;
  float S[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const half8_t q0 = qf[g][0];
    const half8_t q1 = qf[g][1];
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes16_to_half8(d.k[g].x, d.k[g].y), q0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes16_to_half8(d.k[g].z, d.k[g].w), q1, acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) S[r] += acc[r] * scale_at(d.ks, r, g);
  }
  float p[4];
  softmax_step(S, valid, m_run, l_run, p, O, j4);
  if constexpr (VT) {
    // O += P' V, P' = p * v_scale per group rounded once to fp16, V codes exact. The block holds
    // lane l's dims 64 g + l (16 tokens each); the transpose gives lane (n16, j4) tokens
    // 4 j4 + [0, 4) of dims 64 g + 16 i + n16 in v[g][i].
    uint32_t v[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t a0 = d.v[g][0], a1 = d.v[g][1], a2 = d.v[g][2], a3 = d.v[g][3];
      row_transpose4(a0, a1, a2, a3);
      v[g][0] = a0;
      v[g][1] = a1;
      v[g][2] = a2;
      v[g][3] = a3;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      half4_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) pa[r] = _Float16(valid[r] ? p[r] * scale_at<true>(d.vs, r, g) : 0.f);
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // the word already holds tokens 0..3 of the lane's dim
        half2_t lo, hi;
        codes4_to_half(v[g][i], lo, hi);
        O[4 * g + i] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, half4_t{lo[0], lo[1], hi[0], hi[1]}, O[4 * g + i], 0, 0,
                                                            0);
      }
    }
  } else {
    // O += P V', P = p in fp16, V' = code * v_scale rounded once to fp16 (relative error <= 2^-11 on
    // either side). MFMA m: column n16 is dim 16 n16 + m, so the 16 columns of one MFMA span all four
    // scale groups and the scale goes with V; the lane's dims 16 n16 + [0, 16) are all in group
    // n16 / 4, so it needs one scale per token.
    half4_t pa;
#pragma unroll
    for (int r = 0; r < 4; ++r) pa[r] = _Float16(valid[r] ? p[r] : 0.f);
    const int gv = (threadIdx.x & 15) >> 2;
    const half2_t s01 = {_Float16(scale_at(d.vs, 0, gv)), _Float16(scale_at(d.vs, 1, gv))};
    const half2_t s23 = {_Float16(scale_at(d.vs, 2, gv)), _Float16(scale_at(d.vs, 3, gv))};
#pragma unroll
    for (int m = 0; m < 16; ++m) {  // byte m % 4 of word m / 4 of the four tokens
      const half2_t v01 = code_pair_to_half(d.v[0][m >> 2], d.v[1][m >> 2], m & 3) * s01;
      const half2_t v23 = code_pair_to_half(d.v[2][m >> 2], d.v[3][m >> 2], m & 3) * s23;
      O[m] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, half4_t{v01[0], v01[1], v23[0], v23[1]}, O[m], 0, 0, 0);
    }
  }
}

// The 16-token blocks a wave works through. Static: blocks first, first + stride, ... of [tb, te).
// Dynamic (ctr != nullptr): the wave starts with block `first`, then claims blocks from a counter
// shared by a team of workgroups (a claim returning c means block base + c), so waves on faster CUs
// or XCDs take more of the team's blocks and the team finishes together.
struct BlockSource {
  int tb, te;   // tokens [tb, te); tb is page aligned
  int nblk;     // 16-token blocks in [tb, te)
  int first;    // this wave's first block
  int stride;   // static schedule step
  int base;     // dynamic: first claimable block (the team's waves start with blocks [0, base))
  int* ctr;     // dynamic: the team's claim counter
};

// int8 pages: the blocks of `src`; the next block's loads are in flight while the current one is
// computed, and with a claim counter the claim after that is in flight too. Block indices, pages
// and block-table reads are wave-uniform; blocks past te are masked. The waves of a workgroup do
// not synchronise here: each loads its q operand straight from global memory.
// kQBuf: q through a bounds-checked buffer load (no select on its values); the ragged launch keeps
// the select form, which measured faster there.
template <bool VT, bool kQBuf = false>
__device__ void decode_item_int8(const DecodeArgs& a, const KvArgs& kv, const int* bt, int kvh, int q_row,
                                 const BlockSource& src, float& m_run, float& l_run, float4_t (&O)[16]) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, j4 = lane >> 4;
  if (src.first >= src.nblk) return;
  // Q^T operand (rows past the group are zero): lane (head n16, k-group j4) holds dims
  // 64g + 16 j4 + 8h + [0, 8) for group g, half h. Issued before the K/V loads, so waiting for it
  // does not wait for them.
  half8_t qf[4][2];
  {
    if constexpr (kQBuf) {
      // a buffer over the group's q rows: lanes of rows past the group read past its end and get
      // zeros from the bounds check, so no select on the loaded values makes anything wait for q
      // before the first K/V loads go out
      const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(a.q + (size_t(q_row) * a.nq + kvh * a.group) * kHeadDim), short(0),
          a.group * kHeadDim * 2, 0x00020000);
      const int qoff = n16 < a.group ? n16 * kHeadDim * 2 + 32 * j4 : 0x7ffffff0;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          qf[g][h] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(qr, qoff, 128 * g + 16 * h, 0));
    } else {
      const bool real = n16 < a.group;
      const uint16_t* qlane = a.q + (size_t(q_row) * a.nq + kvh * a.group + (real ? n16 : 0)) * kHeadDim + 16 * j4;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          half8_t x = *reinterpret_cast<const half8_t*>(qlane + 64 * g + 8 * h);
          qf[g][h] = real ? x : half8_t{};
        }
    }
  }
  const uint8_t* layer = kv.pool + size_t(a.attn_layer) * kv.layer_stride;
  const Int8Offsets off = int8_offsets<VT>(kv.layout, kvh, n16, j4);
  // the block table is read-only during the launch: through the constant address space its
  // wave-uniform entries become scalar loads, which do not wait behind the vector loads in flight
  const __attribute__((address_space(4))) int* btc = (const __attribute__((address_space(4))) int*)(bt);
  auto load = [&](Int8Block& d, int idx, bool live) {
    const int t0 = src.tb + 16 * idx;
    const uint8_t* pg = layer + size_t(btc[t0 / kPageTokens]) * kv.page_bytes;
    load_int8_block<VT>(d, pg, t0 % kPageTokens, off, live ? int(kv.page_bytes) : 0);
  };
  // one lane claims; the value is read (readfirstlane) only when the next block is chosen
  auto claim = [&]() {
    int c = 0;
    if (lane == 0) c = __hip_atomic_fetch_add(src.ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return c;
  };
  // Each claim is issued before the loads of the block it follows, so resolving it (a wait on the
  // vector memory counter) never waits for K/V data: the next block's loads always go out before
  // the current block's data is awaited.
  const bool dynamic = src.ctr != nullptr;
  int idx = src.first;
  int pending = dynamic ? claim() : 0;
  Int8Block cur, nxt;
  load(cur, idx, true);
  for (;;) {
    // the empty asm pins the claim's use here: without it the compiler reads the claim right after
    // issuing it, which waits for every load in flight
    if (dynamic) asm volatile("" : "+v"(pending));
    const int c = __builtin_amdgcn_readfirstlane(pending);
    const int nidx = dynamic ? src.base + c : idx + src.stride;
    const bool more = nidx < src.nblk;  // uniform
    if (more && dynamic) pending = claim();
    // unconditional (on the last iteration, loads of the current block's page that read nothing):
    // with a single path the compiler's wait for the current block does not also cover the next
    // block's loads
    load(nxt, more ? nidx : idx, more);
    compute_block<true, VT>(cur, qf, src.tb + 16 * idx, src.te, m_run, l_run, O, j4);
    if (!more) break;
    cur = nxt;
    idx = nidx;
  }
}

// bf16 pages: keys [t_begin, t_end), each wave takes 16-token blocks in turn from global memory.
template <int W>
__device__ void decode_item_bf16(const DecodeArgs& a, const KvArgs& kv, const int* bt, int kvh, int q_row,
                                 int t_begin, int t_end, float& m_run, float& l_run, float4_t (&O)[16]) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, j4 = lane >> 4;
  const int G = a.group;
  const bool real = n16 < G;
  const uint16_t* qrow = a.q + (size_t(q_row) * a.nq + kvh * G + (real ? n16 : 0)) * kHeadDim;
  const uint8_t* layer = kv.pool + size_t(a.attn_layer) * kv.layer_stride;
  const int nblk = (t_end - t_begin + 15) >> 4;
  // bf16 pages: q (fp16) = hi + lo exactly, both bf16; P likewise split into hi + lo
  bf16x8_t qb[4][2], qb_lo[4][2];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 w = *reinterpret_cast<const u32x4*>(qrow + 64 * g + 16 * j4 + 8 * h);
      if (!real) w = u32x4{0u, 0u, 0u, 0u};
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
      bf16x8_t v, vl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (e & 1) ? half_hi(ws[e >> 1]) : half_lo(ws[e >> 1]);
        short hi, lo;
        split_bf16(x, hi, lo);
        v[e] = __builtin_bit_cast(__bf16, hi);
        vl[e] = __builtin_bit_cast(__bf16, lo);
      }
      qb[g][h] = v;
      qb_lo[g][h] = vl;
    }
  // The next block's K loads go out as soon as QK^T has consumed this block's K, and its V loads as
  // soon as PV has consumed this block's V (the same registers), so each wave keeps a block's
  // loads in flight while it computes. Past the wave's last block the loads go to an empty buffer
  // resource (they read nothing), which keeps the loop a single path. Config 5c 162.2 -> 160.0 us,
  // config 2 on bf16 pages 87.2 -> 86.1 us (three alternating runs of each build).
  if (wave >= nblk) return;
  const __attribute__((address_space(4))) int* btc = (const __attribute__((address_space(4))) int*)(bt);
  // per-lane byte offsets within a page, relative to the block's first row (row = 512 bytes):
  // K: token n16, dims 64 g + 16 j4 + 8 h + [0, 8); V: tokens 4 j4 + r, dims 16 n16 + [0, 16)
  const uint32_t koff = uint32_t(kv.layout.k_row(kvh, n16)) + 32 * j4;
  const uint32_t voff = uint32_t(kv.layout.v_row(kvh, 4 * j4)) + 32 * n16;
  constexpr int kRowBytes = 2 * kHeadDim;
  auto page_of = [&](int blk, bool live) {
    const uint8_t* pg = layer + size_t(btc[(t_begin + 16 * blk) / kPageTokens]) * kv.page_bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pg), short(0), live ? int(kv.page_bytes) : 0,
                                             0x00020000);
  };
  auto load_k = [&](u32x4 (&kw)[4][2], __amdgpu_buffer_rsrc_t pg, int srow) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        kw[g][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, koff + 128 * g + 16 * h, srow, 0));
  };
  // V: tile k, column n16 <-> dim 16 n16 + k; lane reads 32 contiguous bytes of each of 4 rows
  auto load_v = [&](u32x4 (&vw)[4][2], __amdgpu_buffer_rsrc_t pg, int srow) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        vw[r][i] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, voff + kRowBytes * r + 16 * i, srow, 0));
  };
  int blk = wave;
  u32x4 kw[4][2], vw[4][2];
  {
    const auto pg = page_of(blk, true);
    const int srow = ((16 * blk) % kPageTokens) * kRowBytes;  // t_begin is page aligned
    load_k(kw, pg, srow);
    load_v(vw, pg, srow);
  }
  for (;;) {
    const int t0 = t_begin + 16 * blk;
    const int nb = blk + W;
    const bool more = nb < nblk;  // uniform
    const auto npg = page_of(more ? nb : blk, more);
    const int nsrow = ((16 * (more ? nb : blk)) % kPageTokens) * kRowBytes;
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) valid[r] = t0 + 4 * j4 + r < t_end;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bf16x8_t kb = __builtin_bit_cast(bf16x8_t, kw[g][h]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qb[g][h], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qb_lo[g][h], acc, 0, 0, 0);
      }
    __builtin_amdgcn_sched_barrier(0);
    load_k(kw, npg, nsrow);
    __builtin_amdgcn_sched_barrier(0);
    const float S[4] = {acc[0], acc[1], acc[2], acc[3]};
    float p[4];
    softmax_step(S, valid, m_run, l_run, p, O, j4);
    short4_t pa_hi, pa_lo;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      short hi, lo;
      split_bf16(p[r], hi, lo);
      pa_hi[r] = hi;
      pa_lo[r] = lo;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      short4_t vb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const u32x4 w = vw[r][k >> 3];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        const uint32_t word = ws[(k & 7) >> 1];
        vb[r] = valid[r] ? short((k & 1) ? (word >> 16) : (word & 0xffffu)) : short(0);
      }
      O[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_hi, vb, O[k], 0, 0, 0);
      O[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_lo, vb, O[k], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_v(vw, npg, nsrow);
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
    blk = nb;
  }
}

// Dim held by accumulator tile k in column n (depends on how V was mapped onto MFMA columns): dim
// 16 n + k for int8 and bf16 pages, 64 (k / 4) + 16 (k % 4) + n for int8 VT pages. For int8 and
// bf16 pages tiles 4 k4 .. 4 k4 + 3 of a column are consecutive dims starting at tile_dim4.
__device__ inline int tile_dim4(int k4, int n) { return 16 * n + 4 * k4; }

template <int W>
struct alignas(16) WaveMerge {
  float o[W][kMaxGroup][kHeadDim];
  float m[W][kMaxGroup];
  float l[W][kMaxGroup];
};

template <int W = kWaves>
struct alignas(16) DecodeShared {
  WaveMerge<W> merge;  // the W waves' state at the end of an item
  int next_item;       // the item the workgroup takes next (item queue)
};

// Merges the W waves' (m, l, O) of an item in LDS and writes the item's partial to scratch.
template <int DT, int W>
__device__ void finish_item(const DecodeArgs& a, WaveMerge<W>& sm, int b, int kvh, int split, float m_run, float l_run,
                            const float4_t (&O)[16]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = a.group;
  l_run = xor16_sum(l_run);  // l over the 4 quads of each head lane
  l_run = xor32_sum(l_run);
  if (lane < G) {
    sm.m[wave][lane] = m_run;
    sm.l[wave][lane] = l_run;
  }
  const int n16 = lane & 15, j4 = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int head = 4 * j4 + r;
    if (head < G) {
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        if constexpr (DT == Q38A_KV_INT8_VT) {
#pragma unroll
          for (int i = 0; i < 4; ++i) sm.o[wave][head][64 * k4 + 16 * i + n16] = O[4 * k4 + i][r];
        } else {
          *reinterpret_cast<float4_t*>(&sm.o[wave][head][tile_dim4(k4, n16)]) =
              float4_t{O[4 * k4][r], O[4 * k4 + 1][r], O[4 * k4 + 2][r], O[4 * k4 + 3][r]};
        }
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 64 * W) {
    const int g = idx / kHeadDim, d = idx % kHeadDim;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, sm.m[w][g]);
    float acc = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = sm.m[w][g] == -INFINITY ? 0.f : exp2f(sm.m[w][g] - M);
      acc += f * sm.o[w][g][d];
      lsum += f * sm.l[w][g];
    }
    float* dst = a.scratch + ((size_t(b) * a.nq + kvh * G + g) * a.max_splits + split) * (kHeadDim + 2);
    dst[d] = acc;
    if (d == 0) {
      dst[kHeadDim] = M;
      dst[kHeadDim + 1] = lsum;
    }
  }
  __syncthreads();
}

// Claim counters of the dynamic block schedule (DecodeArgs::claims), one per team of up to kTeam
// consecutive splits of a (decode row, kv head), in the slot of the team's first item, one 128-byte
// line each (claims on one line serialise). The item queue (DecodeArgs::queue) holds the next item
// of the launch. Both live in the caller's scratch, so launches with their own scratch never
// interact; the merge kernel that follows a launch zeroes every counter the launch used.

// Persistent loop over the decode items of a launch: this workgroup is number `wg` of `nwg` that
// stride over items of pl.cp pages (wave_decode_plan). The items of a decode row are ordered
// (kv head, split), so the splits of one (row, kv head) are consecutive workgroups, i.e. spread
// over the XCDs; teams of kTeam of them share a claim counter over their pages (int8 pages; the
// items of one row are consecutive, so a team's items are items slot .. slot + members - 1).
// Partials go to a.scratch.
template <int DT, int W = kWaves>
__device__ __attribute__((always_inline)) inline void decode_items(const DecodeArgs& a, const BatchArgs& batch,
                                                                   const KvArgs& kv, const DecodePlan& pl,
                                                                   DecodeShared<W>& sh, int wg, int nwg) {
  const int cp = pl.cp;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // sh.next_item is written before the first barrier of the grab and read after it; the previous
  // item's finish_item ends with a barrier, so no wave still reads the old value
  auto grab = [&]() {
    if (threadIdx.x == 0) {
      sh.next_item = __hip_atomic_fetch_add(a.queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(sh.next_item);
  };
  for (int item = a.item_queue ? grab() : wg;; item = a.item_queue ? grab() : item + nwg) {
    const ItemSpot at = wave_locate(batch, a.nkv, pl, item);
    if (at.seq < 0) break;
    const int b = at.seq;
    // the row's metadata and block-table slot in one round trip: scalar loads in the decode launch
    // (through the constant address space; the launch metadata is read-only), vector loads in the
    // ragged launch (where the scalar form measured 2% slower on config 4)
    int slot, q_row, q_end, pos0;
    if constexpr (W == kWaves) {
      scalar_load4(batch.seq_slot, b, batch.seq_start, b, batch.seq_start, b + 1, batch.seq_pos0, b, slot, q_row, q_end,
                   pos0);
    } else {
      slot = batch.seq_slot[b];
      q_row = batch.seq_start[b];
      q_end = batch.seq_start[b + 1];
      pos0 = batch.seq_pos0[b];
    }
    const int L = q_end - q_row == 1 ? pos0 + 1 : 0;
    const int nsplit = ceil_div_i(ceil_div_i(L, kPageTokens), cp);
    const int kvh = at.local / nsplit, split = at.local % nsplit;
    const int span = cp * kPageTokens;  // tokens per split
    const int* bt = kv.block_table + size_t(slot) * kv.max_pages_per_seq;
    float m_run = -INFINITY, l_run = 0.f;
    float4_t O[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) O[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (DT != Q38A_KV_BF16) {
      BlockSource src;
      const int team = split / kTeam, member = split % kTeam;
      const int slot = item - member;  // the team's first item
      if (a.dynamic_claims && slot < kClaimSlots) {
        const int members = min(kTeam, nsplit - team * kTeam);
        src.tb = team * kTeam * span;
        src.te = min(L, src.tb + members * span);
        src.first = member * W + wave;
        src.base = members * W;
        src.ctr = a.claims + size_t(slot) * kClaimStride;
      } else {
        src.tb = split * span;
        src.te = min(L, src.tb + span);
        src.first = wave;
        src.ctr = nullptr;
      }
      src.nblk = ceil_div_i(src.te - src.tb, 16);
      src.stride = W;
      decode_item_int8<DT == Q38A_KV_INT8_VT, W == kWaves>(a, kv, bt, kvh, q_row, src, m_run, l_run, O);
    } else {
      const int t_begin = split * span;
      decode_item_bf16<W>(a, kv, bt, kvh, q_row, t_begin, min(L, t_begin + span), m_run, l_run, O);
    }
    finish_item<DT, W>(a, sh.merge, b, kvh, split, m_run, l_run, O);
  }
}

constexpr int kMergeWaves = 4;
constexpr int kMergeThreads = 64 * kMergeWaves;
constexpr int kMergeBatch = 16;  // splits a lane loads at once

__device__ inline float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

__device__ inline float sigmoid_gate(uint16_t g) { return fast_sigmoid(bf16_value(g)); }

// Gated merge of one (row, q head)'s split partials (reference attention_decode.cu:241-257):
// M = max_s m_s, a = sum_s 2^(m_s - M) acc_s, l = sum_s 2^(m_s - M) l_s, y = (a / l) * sigmoid(gate).
// The merge kernels fold the splits in kMergeWaves interleaved running states (state w: splits w,
// w + kMergeWaves, ...) and combine the states; the o-projection's A staging (qgemm.hip) replays
// the same steps in one thread. Every multiply-add below is an explicit fmaf, so the result does
// not depend on the call site's contraction and both produce the same bits.

// Folds the splits s = first, first + step, ... (< splits) of one (row, q head) into a running
// log-sum-exp state (M, lsum, acc[4] of dims d..d+3), kMergeBatch splits in flight per lane.
// Split s sits at src + s * stride: acc[256], m, l; m = -inf marks an empty split.
__device__ inline void fold_splits(const float* src, int first, int step, int splits, size_t stride, int d, float& M,
                                   float& lsum, float (&acc)[4]) {
  for (int s0 = first; s0 < splits; s0 += step * kMergeBatch) {
    float2 v[kMergeBatch][2], ml[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int s = min(s0 + step * u, splits - 1);
      const float* p = src + s * stride;
      v[u][0] = *reinterpret_cast<const float2*>(p + d);
      v[u][1] = *reinterpret_cast<const float2*>(p + d + 2);
      ml[u] = *reinterpret_cast<const float2*>(p + kHeadDim);
      if (s0 + step * u >= splits) ml[u].x = -INFINITY;
    }
    float bm = M;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) bm = fmaxf(bm, ml[u].x);
    if (bm == -INFINITY) continue;  // uniform: (m, l) are the same in every lane
    const float c = __builtin_amdgcn_exp2f(M - bm);  // M = -inf gives 0
    M = bm;
    lsum *= c;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= c;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float w = __builtin_amdgcn_exp2f(ml[u].x - M);  // empty split: 0
      lsum = __builtin_fmaf(w, ml[u].y, lsum);
      acc[0] = __builtin_fmaf(w, v[u][0].x, acc[0]);
      acc[1] = __builtin_fmaf(w, v[u][0].y, acc[1]);
      acc[2] = __builtin_fmaf(w, v[u][1].x, acc[2]);
      acc[3] = __builtin_fmaf(w, v[u][1].y, acc[3]);
    }
  }
}

// Combines the kMergeWaves states of one dim into the gated bf16 output.
__device__ inline uint16_t merge_combine(const float (&m)[kMergeWaves], const float (&l)[kMergeWaves],
                                         const float (&acc)[kMergeWaves], uint16_t gate) {
  float Mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kMergeWaves; ++w) Mx = fmaxf(Mx, m[w]);
  float a = 0.f, lsum = 0.f;
#pragma unroll
  for (int w = 0; w < kMergeWaves; ++w) {
    const float f = __builtin_amdgcn_exp2f(m[w] - Mx);  // empty state: 0
    a = __builtin_fmaf(f, acc[w], a);
    lsum = __builtin_fmaf(f, l[w], lsum);
  }
  return bf16_bits((a / lsum) * sigmoid_gate(gate));
}

struct alignas(16) MergeShared {
  float m[kMergeWaves], l[kMergeWaves];
  float acc[kMergeWaves][kHeadDim];
};

// The whole workgroup (kMergeWaves waves) merges one (row, q head): wave w folds splits w, w + 4,
// ..., the waves' states are combined in LDS, and thread t finishes dim t.
__device__ inline void merge_row_wg(const float* src, int splits, size_t stride, const uint16_t* gate_row,
                                    uint16_t* out_row, MergeShared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = 4 * lane;
  // the gate is read before the partials, so its load is not a second round trip after theirs
  const uint16_t gate = gate_row[threadIdx.x];
  float M = -INFINITY, lsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  fold_splits(src, wave, kMergeWaves, splits, stride, d, M, lsum, acc);
  if (lane == 0) {
    sh.m[wave] = M;
    sh.l[wave] = lsum;
  }
  *reinterpret_cast<float4_t*>(&sh.acc[wave][d]) = float4_t{acc[0], acc[1], acc[2], acc[3]};
  __syncthreads();
  const int t = threadIdx.x;
  float m[kMergeWaves], l[kMergeWaves], at[kMergeWaves];
#pragma unroll
  for (int w = 0; w < kMergeWaves; ++w) {
    m[w] = sh.m[w];
    l[w] = sh.l[w];
    at[w] = sh.acc[w][t];
  }
  out_row[t] = merge_combine(m, l, at, gate);
}

// The same merge for dims d..d+3 in one thread (the kMergeWaves folds one after the other).
__device__ inline void merge_quad(const float* src, int splits, size_t stride, int d, const uint16_t* gate4,
                                  uint16_t (&y)[4]) {
  const uint2 g = *reinterpret_cast<const uint2*>(gate4);  // before the partials' loads
  float m[kMergeWaves], l[kMergeWaves], acc[kMergeWaves][4];
#pragma unroll
  for (int w = 0; w < kMergeWaves; ++w) {
    m[w] = -INFINITY;
    l[w] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[w][i] = 0.f;
    fold_splits(src, w, kMergeWaves, splits, stride, d, m[w], l[w], acc[w]);
  }
  const uint16_t gv[4] = {uint16_t(g.x), uint16_t(g.x >> 16), uint16_t(g.y), uint16_t(g.y >> 16)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float at[kMergeWaves];
#pragma unroll
    for (int w = 0; w < kMergeWaves; ++w) at[w] = acc[w][i];
    y[i] = merge_combine(m, l, at, gv[i]);
  }
}

// merge_row for prefill partial rows (kPartialRowFloats: O / l in fp16, then m, l): split s weighs
// 2^(m_s - M) l_s. One wave; lane l owns dims 4l + [0, 4).
template <int kBatch>
__device__ inline void merge_row_h16_b(const float* src, int splits, size_t stride, const uint16_t* gate_row,
                                       uint16_t* out_row) {
  const int d = 4 * (threadIdx.x & 63);
  const uint2 g = *reinterpret_cast<const uint2*>(gate_row + d);  // before the partials' loads
  float M = -INFINITY, wsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += kBatch) {
    uint2 v[kBatch];
    float2 ml[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int s = min(s0 + u, splits - 1);
      const float* p = src + s * stride;
      v[u] = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + d);
      ml[u] = *reinterpret_cast<const float2*>(p + kHeadDim / 2);
      if (s0 + u >= splits) ml[u] = float2{-INFINITY, 0.f};
    }
    float bm = M;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) bm = fmaxf(bm, ml[u].x);
    if (bm == -INFINITY) continue;  // uniform
    const float c = __builtin_amdgcn_exp2f(M - bm);
    M = bm;
    wsum *= c;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= c;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float w = __builtin_amdgcn_exp2f(ml[u].x - M) * ml[u].y;  // empty split: 0
      const half2_t a = __builtin_bit_cast(half2_t, v[u].x), b = __builtin_bit_cast(half2_t, v[u].y);
      wsum += w;
      acc[0] += w * float(a[0]);
      acc[1] += w * float(a[1]);
      acc[2] += w * float(b[0]);
      acc[3] += w * float(b[1]);
    }
  }
  const uint16_t gv[4] = {uint16_t(g.x), uint16_t(g.x >> 16), uint16_t(g.y), uint16_t(g.y >> 16)};
  uint16_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = bf16_bits((wsum > 0.f ? acc[i] / wsum : 0.f) * sigmoid_gate(gv[i]));
  *reinterpret_cast<uint2*>(out_row + d) = uint2{uint32_t(o[0]) | (uint32_t(o[1]) << 16), uint32_t(o[2]) | (uint32_t(o[3]) << 16)};
}

// The split loads of one batch are issued together; the batch follows the split count so that a
// row with few splits does not issue (clamped, repeated) loads for splits it does not have.
__device__ inline void merge_row_h16(const float* src, int splits, size_t stride, const uint16_t* gate_row,
                                     uint16_t* out_row) {
  if (splits <= 4) merge_row_h16_b<4>(src, splits, stride, gate_row, out_row);
  else if (splits <= 8) merge_row_h16_b<8>(src, splits, stride, gate_row, out_row);
  else merge_row_h16_b<kMergeBatch>(src, splits, stride, gate_row, out_row);
}



}  // namespace
}  // namespace q38a
