// Split-KV flash-decoding over the paged KV cache on gfx950 MFMA, plus the gated split merge.
//
// Semantics follow reference src/kernels/attention_decode.cu:97-257 (and the exact CPU form
// src/ref/ops.cpp:144-171): for decode row b and q head hq (kv head hq / group), softmax over keys
// [0, seq_pos0[b] + 1) of q.k / 16, weighted sum of V, then out = (acc / l) * sigmoid(gate) in bf16.
//
// MI355X design. Decode is HBM-bound (each KV byte is used once); with GQA 6 and int8 KV it needs
// ~12 flop/byte, which at 8 TB/s is more than the non-packed fp32 VALU can issue alongside the
// int8 widening, so both products run on MFMA and the VALU only widens codes and runs the softmax:
//   * one workgroup = 4 waves works on one item (sequence, kv head, run of whole pages, see
//     plan.hpp); each wave takes 16-token blocks of the item's pages in turn;
//   * S^T[16 tok][16 heads] = K[16 tok][256] . Q^T with v_mfma_f32_16x16x32_f16: K codes enter the
//     MFMA exactly (int8 is exact in fp16), Q as stored (fp16), and the per-(token, 64-dim group)
//     K scale multiplies the four group partials in fp32 afterwards;
//   * O[16 heads][256] += P'[16 heads][16 tok] . V[16 tok][256] with v_mfma_f32_16x16x16_bf16:
//     V codes are exact in bf16 and the V scale is folded into P' = p * v_scale per group, so no
//     dequantised value is ever rounded and no fp16 range limit applies to V; P' enters as a
//     hi + lo pair of bf16 operands (two MFMAs), i.e. with a 16-bit significand;
//   * the S^T accumulator layout (lane = head, 4 tokens) is exactly the A-operand layout of the
//     PV product, so probabilities never leave registers;
//   * K rows are read as 4 x 16-byte loads per lane (a 16-lane group covers 64 contiguous bytes of
//     a row), V rows as 16 x 4-byte loads (16 lanes cover 64 contiguous bytes);
//   * the 4 waves' (max, sum, acc) are merged in LDS and written once per item as a partial;
//     attn_merge_kernel combines partials with the log-sum-exp rule and applies sigmoid(gate).
// bf16 KV pages use the same schedule with bf16 MFMAs for both products; q (fp16) is split exactly
// into two bf16 operands and P likewise into hi + lo.
#include "plan.hpp"

namespace q38a {

int max_group() { return 8; }

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxGroup = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kScoreScale = kLog2e / 16.0f;  // 1/sqrt(256) folded into the exp2 domain

struct DecodeArgs {
  const uint16_t* q;
  int nq, nkv, group;
  int attn_layer;
  float* scratch;
  int max_splits;
  int target_items;
};

__device__ inline half8_t codes_to_half8(uint32_t lo, uint32_t hi) {
  half8_t r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = _Float16(float(int8_t(lo >> (8 * e))));
    r[4 + e] = _Float16(float(int8_t(hi >> (8 * e))));
  }
  return r;
}

__device__ inline short bf16_short(float f) { return short(bf16_bits(f)); }

// x = hi + lo with hi = bf16(x) and lo = bf16(x - hi): a 16-bit significand carried by two bf16
// MFMA operands (relative error ~2^-17 instead of bf16's 2^-9), with fp32's exponent range.
__device__ inline void split_bf16(float x, short& hi, short& lo) {
  const uint16_t h = bf16_bits(x);
  hi = short(h);
  lo = short(bf16_bits(x - bf16_value(h)));
}

// Keys [t_begin, t_end) of one (sequence, kv head) for the GROUP q heads of that kv head.
// Writes the wave's (m, l, O) for the caller's LDS merge.
template <int DT>
__device__ void decode_item(const DecodeArgs& a, const KvArgs& kv, const int* bt, int kvh, int q_row, int t_begin,
                            int t_end, float& m_run, float& l_run, float4_t (&O)[16]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n16 = lane & 15, j4 = lane >> 4;  // MFMA lane coordinates
  const int G = a.group;

  // Q^T operand: lane (head n16, k-group j4); group g, half h covers dims 64g + 16 j4 + 8h + [0, 8)
  half8_t qf[4][2];
  bf16x8_t qb[4][2], qb_lo[4][2];  // bf16 pages: q (fp16) = hi + lo exactly, both bf16
  {
    const bool real = n16 < G;
    const uint16_t* qrow = a.q + (size_t(q_row) * a.nq + kvh * G + (real ? n16 : 0)) * kHeadDim;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint4 w = *reinterpret_cast<const uint4*>(qrow + 64 * g + 16 * j4 + 8 * h);
        if (!real) w = make_uint4(0, 0, 0, 0);
        if constexpr (DT == Q38A_KV_INT8) {
          qf[g][h] = __builtin_bit_cast(half8_t, w);
        } else {
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
          bf16x8_t v, vl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = f16_value(uint16_t(ws[e >> 1] >> (16 * (e & 1))));
            short hi, lo;
            split_bf16(x, hi, lo);
            v[e] = __builtin_bit_cast(__bf16, hi);
            vl[e] = __builtin_bit_cast(__bf16, lo);
          }
          qb[g][h] = v;
          qb_lo[g][h] = vl;
        }
      }
    }
  }

  const uint8_t* layer = kv.pool + size_t(a.attn_layer) * kv.layer_stride;
  const int nblk = (t_end - t_begin + 15) >> 4;
  for (int blk = wave; blk < nblk; blk += kWaves) {
    const int t0 = t_begin + 16 * blk;
    const uint8_t* pg = layer + size_t(bt[t0 / kPageTokens]) * kv.page_bytes;
    const int in0 = t0 % kPageTokens;
    // token validity for this lane's 4 score / probability slots (tokens 4 j4 + r)
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) valid[r] = t0 + 4 * j4 + r < t_end;

    float S[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (DT == Q38A_KV_INT8) {
      const uint8_t* krow = pg + kv.layout.k_row(kvh, in0 + n16);
      uint4 kr[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) kr[g] = *reinterpret_cast<const uint4*>(krow + 64 * g + 16 * j4);
      const uint4* ksp = reinterpret_cast<const uint4*>(pg + kv.layout.k_scales(kvh, in0 + 4 * j4));
      const uint4 ks0 = ksp[0], ks1 = ksp[1];
      const uint32_t ksw[8] = {ks0.x, ks0.y, ks0.z, ks0.w, ks1.x, ks1.y, ks1.z, ks1.w};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_half8(kr[g].x, kr[g].y), qf[g][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_half8(kr[g].z, kr[g].w), qf[g][1], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int idx = r * 4 + g;  // token r, group g: half index in the 32-byte scale block
          const float sc = f16_value(uint16_t(ksw[idx >> 1] >> (16 * (idx & 1))));
          S[r] += acc[r] * sc;
        }
      }
    } else {
      const uint8_t* krow = pg + kv.layout.k_row(kvh, in0 + n16);
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 w = *reinterpret_cast<const uint4*>(krow + 2 * (64 * g + 16 * j4 + 8 * h));
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w), qb[g][h], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w), qb_lo[g][h], acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) S[r] = acc[r];
    }

    // ---- online softmax (log2 domain); lane (head n16, quad j4) holds tokens 4 j4 + r -------------
    float s2[4], bmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s2[r] = valid[r] ? S[r] * kScoreScale : -INFINITY;
      bmax = fmaxf(bmax, s2[r]);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(m_run, bmax);
    const float corr = exp2f(m_run - mnew);
    float p[4], psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = exp2f(s2[r] - mnew);
      psum += p[r];
    }
    l_run = l_run * corr + psum;
    m_run = mnew;
    // O rows are heads 4 j4 + r; their correction factors live in lanes 4 j4 + r (quad 0)
    float cr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr, 4 * j4 + r, 64);
#pragma unroll
    for (int k = 0; k < 16; ++k)
#pragma unroll
      for (int r = 0; r < 4; ++r) O[k][r] *= cr[r];

    // ---- O += P' V ---------------------------------------------------------------------------------
    if constexpr (DT == Q38A_KV_INT8) {
      uint32_t vr[4][4];  // [group][token r]: dims 64g + 4 n16 + [0, 4) of token 4 j4 + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint8_t* vrow = pg + kv.layout.v_row(kvh, in0 + 4 * j4 + r);
#pragma unroll
        for (int g = 0; g < 4; ++g) vr[g][r] = *reinterpret_cast<const uint32_t*>(vrow + 64 * g + 4 * n16);
      }
      const uint4* vsp = reinterpret_cast<const uint4*>(pg + kv.layout.v_scales(kvh, in0 + 4 * j4));
      const uint4 vs0 = vsp[0], vs1 = vsp[1];
      const uint32_t vsw[8] = {vs0.x, vs0.y, vs0.z, vs0.w, vs1.x, vs1.y, vs1.z, vs1.w};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        short4_t pa_hi, pa_lo;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int idx = r * 4 + g;
          const float vs = valid[r] ? f16_value(uint16_t(vsw[idx >> 1] >> (16 * (idx & 1)))) : 0.f;
          short hi, lo;
          split_bf16(p[r] * vs, hi, lo);
          pa_hi[r] = hi;
          pa_lo[r] = lo;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          short4_t vb;
#pragma unroll
          for (int r = 0; r < 4; ++r) vb[r] = bf16_short(float(int8_t(vr[g][r] >> (8 * i))));
          O[4 * g + i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_hi, vb, O[4 * g + i], 0, 0, 0);
          O[4 * g + i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_lo, vb, O[4 * g + i], 0, 0, 0);
        }
      }
    } else {
      short4_t pa_hi, pa_lo;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        short hi, lo;
        split_bf16(p[r], hi, lo);
        pa_hi[r] = hi;
        pa_lo[r] = lo;
      }
      // tile k, column n16 <-> dim 16 n16 + k; lane reads 32 contiguous bytes of each of 4 rows
      uint4 vw[4][2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint8_t* vrow = pg + kv.layout.v_row(kvh, in0 + 4 * j4 + r);
        vw[r][0] = *reinterpret_cast<const uint4*>(vrow + 32 * n16);
        vw[r][1] = *reinterpret_cast<const uint4*>(vrow + 32 * n16 + 16);
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        short4_t vb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint4 w = vw[r][k >> 3];
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
          const uint32_t word = ws[(k & 7) >> 1];
          vb[r] = valid[r] ? short((k & 1) ? (word >> 16) : (word & 0xffffu)) : short(0);
        }
        O[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_hi, vb, O[k], 0, 0, 0);
        O[k] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa_lo, vb, O[k], 0, 0, 0);
      }
    }
  }
}

// Dim of accumulator tile k, column n (depends on how V rows were mapped onto MFMA columns).
template <int DT>
__device__ inline int tile_dim(int k, int n) {
  if constexpr (DT == Q38A_KV_INT8) return 64 * (k >> 2) + 4 * n + (k & 3);
  else return 16 * n + k;
}

struct DecodeShared {
  PlanShared plan;
  float m[kWaves][kMaxGroup];
  float l[kWaves][kMaxGroup];
  float o[kWaves][kMaxGroup][kHeadDim];
};

template <int DT>
__global__ void __launch_bounds__(kThreads) attn_decode_kernel(DecodeArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ DecodeShared sh;
  build_plan(batch, a.nkv, a.max_splits, a.target_items, sh.plan);
  const int B = batch.num_seqs;
  const int total = sh.plan.prefix[B];
  const int cp = sh.plan.chunk_pages;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = a.group;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = find_seq(sh.plan, B, item);
    const int local = item - sh.plan.prefix[b];
    const int split = local / a.nkv, kvh = local % a.nkv;
    const int L = decode_len(batch, b);
    const int t_begin = split * cp * kPageTokens;
    const int t_end = min(L, t_begin + cp * kPageTokens);
    const int* bt = kv.block_table + size_t(batch.seq_slot[b]) * kv.max_pages_per_seq;
    const int q_row = batch.seq_start[b];

    float m_run = -INFINITY, l_run = 0.f;
    float4_t O[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) O[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    decode_item<DT>(a, kv, bt, kvh, q_row, t_begin, t_end, m_run, l_run, O);

    // wave totals: l over the 4 quads of each head lane
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (lane < G) {
      sh.m[wave][lane] = m_run;
      sh.l[wave][lane] = l_run;
    }
    const int n16 = lane & 15, j4 = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = 4 * j4 + r;
      if (head < G) {
#pragma unroll
        for (int k = 0; k < 16; ++k) sh.o[wave][head][tile_dim<DT>(k, n16)] = O[k][r];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += kThreads) {
      const int g = idx / kHeadDim, d = idx % kHeadDim;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh.m[w][g]);
      float acc = 0.f, lsum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = sh.m[w][g] == -INFINITY ? 0.f : exp2f(sh.m[w][g] - M);
        acc += f * sh.o[w][g][d];
        lsum += f * sh.l[w][g];
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
}

struct MergeArgs {
  const uint16_t* gate;
  int ld_gate;
  uint16_t* out;
  int nq, nkv;
  const float* scratch;
  int max_splits;
  int target_items;
};

// grid (nq, B): combine the item partials of (decode row b, q head), normalise, apply the gate.
__global__ void __launch_bounds__(kPlanThreads) attn_merge_kernel(MergeArgs a, BatchArgs batch) {
  __shared__ PlanShared plan;
  build_plan(batch, a.nkv, a.max_splits, a.target_items, plan);
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int L = decode_len(batch, b);
  if (L == 0) return;
  const int splits = ceil_div_i(ceil_div_i(L, kPageTokens), plan.chunk_pages);
  const float* src = a.scratch + (size_t(b) * a.nq + hq) * a.max_splits * (kHeadDim + 2);
  float M = -INFINITY;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, src[s * (kHeadDim + 2) + kHeadDim]);
  float acc = 0.f, lsum = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float ms = src[s * (kHeadDim + 2) + kHeadDim];
    const float f = ms == -INFINITY ? 0.f : exp2f(ms - M);
    acc += f * src[s * (kHeadDim + 2) + d];
    lsum += f * src[s * (kHeadDim + 2) + kHeadDim + 1];
  }
  const int row = batch.seq_start[b];
  const float g = bf16_value(a.gate[size_t(row) * a.ld_gate + hq * kHeadDim + d]);
  const float y = (acc / lsum) * (1.0f / (1.0f + expf(-g)));
  a.out[(size_t(row) * a.nq + hq) * kHeadDim + d] = bf16_bits(y);
}

constexpr int kBlocksPerCu = 2;
constexpr int kItemsPerBlock = 4;

}  // namespace

// Shared with the ragged launcher: decode grid size and the merge launch.
int decode_grid(int* grid, int* target_items) {
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  *grid = cus * kBlocksPerCu;
  *target_items = *grid * kItemsPerBlock;
  return Q38A_OK;
}

int launch_merge(const q38a_attention_params& p, const q38a_batch_desc& b, int target_items, hipStream_t stream) {
  MergeArgs m{p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, p.split_scratch, p.max_splits, target_items};
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.num_q_heads, b.num_seqs), dim3(kPlanThreads), 0, stream, m,
                     to_args(b));
  return check_hip(hipGetLastError(), "attention merge launch");
}

int launch_attention_decode(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream) {
  if (b.num_seqs == 0) return Q38A_OK;
  if (b.num_seqs >= kMaxSeqs) return set_error(Q38A_ERR_INVALID, "attention_decode: at most %d sequences", kMaxSeqs - 1);
  int grid = 0, target = 0;
  if (int rc = decode_grid(&grid, &target)) return rc;
  DecodeArgs a{p.q, p.num_q_heads, p.num_kv_heads, p.num_q_heads / p.num_kv_heads, p.attn_layer,
               p.split_scratch, p.max_splits, target};
  if (kv.dtype == Q38A_KV_INT8)
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_INT8>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  else
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_BF16>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  if (int rc = check_hip(hipGetLastError(), "attention_decode launch")) return rc;
  return launch_merge(p, b, target, stream);
}

}  // namespace q38a
