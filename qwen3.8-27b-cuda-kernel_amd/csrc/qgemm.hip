// BQ-weight GEMM for gfx950 (q38a_qgemm) and the attention in-projection with the q/k norm, RoPE
// and KV append fused into its epilogue (q38a_qgemm_qkv_append).
//
// Semantics follow reference src/kernels/qgemm.cu:285-384 (epilogues) and :573-616 (launcher):
// C[M][N] = A[M][K] . W^T, W[n][k] = code * scale[n][k / 64], A bf16, fp32 accumulation; StoreBF16
// stores bf16(C * rs) with the folded-RMSNorm row scale rs, Residual adds C into the fp32 residual
// stream and refreshes its bf16 copy and its per-128-column sums of squares.
//
// MI355X design:
//   * v_mfma_f32_32x32x16_bf16 with the activations as the A operand and the weights as B. A lane
//     of the B operand holds eight consecutive k of one column; the repacked weights
//     (bq_repack.cpp) give it those codes as one 16-byte word per 64-k group (+ the high bits).
//   * The codes enter the MFMA as the exact bf16 values 128 + u (u = the stored unsigned code, two
//     bit operations per pair), so no conversion arithmetic is spent on them; the offset and the
//     per-(column, group) scale are applied once per group in fp32:
//       C += scale[n][g] * (T_g - (128 + 2^(b-1)) * S_g),  T_g = sum_{k in g} a[m][k] (128 + u),
//     where S_g = sum_{k in g} a[m][k] comes from one more MFMA against a ones operand (its output
//     lands in the same registers as T's rows). T carries at most ~8 bits of cancellation; the
//     result keeps ~16 significant bits, far below the bf16 output's rounding.
//   * A workgroup is four waves over a 32 MB-row x 256-column tile (a wave: 64 columns, two MFMA
//     column blocks); the K loop walks 64-wide groups with the next group's loads in flight.
//   * Small M leaves too few tiles to pull the weights at HBM speed, so K is split over several
//     workgroups: each writes its fp32 partial tile (rows < M only) with write-through stores,
//     counts its arrival on a per-tile counter, and the last to arrive sums the slices in slice
//     order (deterministic) and runs the epilogue, then resets the counter.
//   * The fused in-projection tiles are exactly one 256-column head: a q, k or v tile is rounded to
//     bf16 into LDS and the append's per-row code (append.hpp) runs on it, so q/k/v never make the
//     round trip through proj; gate tiles are stored to proj, where attention reads them.
#include <type_traits>

#include "append.hpp"
#include "decode.hpp"
#include "q38a_gemm.h"

namespace q38a {

int decode_grid(int* grid, int* target_items);
int launch_attention_merge(const q38a_attention_params& p, const q38a_batch_desc& b, hipStream_t stream);
int launch_qk_norm_rope_append(const q38a_qk_norm_rope_params& p, const q38a_batch_desc& b,
                               const q38a_kv_cache_desc& kv, hipStream_t stream);

namespace {

// A workgroup covers 256 columns: 8 waves of one 32-column block for one row block (small M: more
// waves, each with fewer registers, keep more weight bytes in flight), 4 waves of two blocks for two
// row blocks (more reuse of each A operand).
constexpr int kTileN = 256;
constexpr int kMaxWaves = 8;
__host__ __device__ constexpr int nb_of(int mb) { return mb == 1 ? 1 : 2; }      // 32-column blocks per wave
__host__ __device__ constexpr int waves_of(int mb) { return kTileN / (32 * nb_of(mb)); }
// K parts of a workgroup's slice: one row block runs two sets of 8 waves, each over half the slice's
// groups (twice the weight bytes in flight per CU), their sums added through LDS
__host__ __device__ constexpr int kparts_of(int mb) { return mb == 1 ? 2 : 1; }
__host__ __device__ constexpr int threads_of(int mb) { return 64 * waves_of(mb) * kparts_of(mb); }
constexpr int kEpiFused = 100;  // epilogue kind of the fused in-projection

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const uint16_t* a;
  int m, n, k;
  const uint8_t* lo;
  const uint8_t* hi;
  const uint16_t* scales;
  int kind;
  void* out;
  int ldo, n_store;
  float* residual;
  uint16_t* xbf;
  float* partials_out;
  const float* partials_in;
  int norm_blocks;
  float inv_hidden, eps;
  int tiles_n, splits;
  float* ws_partials;
  int* counters;
};

// The o-projection's A from decode split partials (q38a_qgemm_merge_oproj): A[row][256 h + d] is the
// gated merge of (decode row, q head h), as the decode launch's merge kernel computes it.
struct MergeIn {
  const float* scratch;
  const uint16_t* gate;
  int ld_gate, nq, nkv, max_splits, target_items;
};

// One lane's share of one (32-column block, group) of weights: 32 low nibbles, their high bits, and
// the column's scale.
struct BWords {
  u32x4 lo;
  u32x2 hi;
  uint32_t scale;  // bf16 bits in the low half (converted where used, so the load is not awaited early)
};

// A wave-uniform address kept in scalar registers (a buffer resource built from an address the
// compiler computed in vector registers would otherwise be legalised lane by lane).
template <class T>
__device__ inline T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(v)));
  const uint64_t hi = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(v >> 32)));
  return reinterpret_cast<T*>(lo | (hi << 32));
}

// Buffer resources over the three weight planes: the per-group offsets are wave-uniform (scalar
// offsets), the lane's part a fixed vector offset, so no per-load 64-bit address arithmetic.
struct BPlanes {
  __amdgpu_buffer_rsrc_t lo, hi, sc;
};

template <int BITS>
__device__ inline BPlanes make_bplanes(const GemmArgs& a) {
  const int units = (a.n / 32) * (a.k / 64);
  constexpr int hb = BITS == 4 ? 0 : BITS == 5 ? 4 : 8;
  BPlanes p;
  p.lo = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.lo), short(0), units * 1024, 0x00020000);
  p.hi = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(BITS == 4 ? a.lo : a.hi), short(0), units * 64 * hb,
                                           0x00020000);
  p.sc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.scales), short(0), units * 64, 0x00020000);
  return p;
}

// Cache policy of a buffer load: non-temporal (data read once).
constexpr int kNonTemporal = 2;

template <int BITS, int CPOL = 0>
__device__ inline void load_bwords(BWords& b, const BPlanes& p, int nb, int g, int G, int lane) {
  const int unit = nb * G + g;
  b.lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(p.lo, lane * 16, unit * 1024, CPOL));
  if constexpr (BITS == 5) b.hi = u32x2{__builtin_amdgcn_raw_buffer_load_b32(p.hi, lane * 4, unit * 256, CPOL), 0u};
  else if constexpr (BITS == 6)
    b.hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(p.hi, lane * 8, unit * 512, CPOL));
  else b.hi = u32x2{0u, 0u};
  b.scale = __builtin_amdgcn_raw_buffer_load_b16(p.sc, (lane & 31) * 2, unit * 64, CPOL);
}

// (x & m) | c: one v_and_or_b32. Plain code, not inline assembly: an MFMA reading a register that an
// inline-assembly instruction wrote gets no hazard wait states from the compiler (it does not count
// the assembly as a VALU write), and then reads stale values.
__device__ inline uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

// Shift right by a signed constant (left when negative).
template <int R>
__device__ inline uint32_t shr(uint32_t x) {
  if constexpr (R > 0) return x >> R;
  else if constexpr (R < 0) return x << (-R);
  else return x;
}

// Pair P of step S of the B operand: two bf16 values 128 + u, exact: the low nibbles masked into
// the magic 0x4300 (one shift and one and-or; no shift at P = 0), the high bits masked in at bit 4.
template <int BITS, int S, int P>
__device__ inline uint32_t b_pair(const BWords& b, uint32_t magic) {
  constexpr int q = 4 * S + P;
  uint32_t w = and_or(shr<4 * P>(b.lo[S]), 0x000F000Fu, magic);
  if constexpr (BITS == 5) w = and_or(shr<q - 4>(b.hi.x), 0x00100010u, w);
  if constexpr (BITS == 6) w = and_or(shr<2 * (q & 7) - 4>(q < 8 ? b.hi.x : b.hi.y), 0x00300030u, w);
  return w;
}

template <int BITS, int S>
__device__ inline bf16x8_t b_operand(const BWords& b, uint32_t magic) {
  const u32x4 v{b_pair<BITS, S, 0>(b, magic), b_pair<BITS, S, 1>(b, magic), b_pair<BITS, S, 2>(b, magic),
                b_pair<BITS, S, 3>(b, magic)};
  return __builtin_bit_cast(bf16x8_t, v);
}

// Row scale of the folded RMSNorm (reference qgemm.cu:288-297): 64 partials of the row in flight
// per round (loads past the row's end re-read its last block and are not added), summed in block
// order.
__device__ inline float row_scale(const GemmArgs& a, int row) {
  if (!a.partials_in || row >= a.m) return 1.0f;
  const float* pr = a.partials_in + size_t(row) * a.norm_blocks;
  const int last = a.norm_blocks - 1;
  float s = 0.0f;
  for (int b = 0; b < a.norm_blocks; b += 64) {
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = pr[b + i < last ? b + i : last];
#pragma unroll
    for (int i = 0; i < 64; ++i) s = b + i <= last ? s + v[i] : s;
  }
  return 1.0f / __builtin_sqrtf(s * a.inv_hidden + a.eps);
}

struct alignas(16) GemmShared {
  union {
    uint16_t tile[64][kTileN + 8];  // fused epilogue: the bf16 head tile (rows x 256)
    float resid_ss[kMaxWaves][64];  // residual epilogue: per-wave sums of squares of its columns
    float kpart[kMaxWaves][16][64];  // the second K part's sums (one row block, one column block)
  };
  double stage[kMaxWaves][kHeadDim];  // the append's sequential-sum fallback
  float rs[64];                       // row scales of the folded RMSNorm (1 without partials_in)
  int last;
};

// The tile's end, shared by both kernels: split-K slices summed by the last workgroup to arrive,
// then the epilogue. C element e of (row block mb, column block j) in this lane: row
// 32 mb + 8 (e / 4) + 4 (lane / 32) + e % 4 of the tile, column 32 (kNB wave + j) + lane % 32. Every
// wave of the column tile calls it (K-part waves have ended); sh.rs holds the tile's row scales.
// EQ: row quads of the MFMA output that can hold rows < M (the split-K traffic skips the others).
template <int MB, bool FUSED, int EQ = 4>
__device__ void tile_finish(const GemmArgs& a, const AppendArgs& ap, const BatchArgs& batch, const KvArgs& kv,
                            GemmShared& sh, float16_t (&C)[MB][nb_of(MB)], int tile, int z, int tn, int wave,
                            int lane) {
  constexpr int kNB = nb_of(MB), kGWaves = waves_of(MB), kBM = 32 * MB;
  const int kg = lane >> 5;
  const int m0 = (tile / a.tiles_n) * kBM;
  auto row_of = [&](int mb, int e) { return m0 + 32 * mb + 8 * (e >> 2) + 4 * kg + (e & 3); };
  const int colw = tn * kTileN + 32 * kNB * wave + (lane & 31);  // + 32 j

  // ---- split-K: the last of the tile's slices sums them in slice order -------------------------
  if (a.splits > 1) {
    float* part = a.ws_partials + size_t(tile) * a.splits * kBM * kTileN;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 4 * EQ; ++e) {
          const int r = row_of(mb, e) - m0;
          if (m0 + r < a.m)
            __hip_atomic_store(part + (size_t(z) * kBM + r) * kTileN + 32 * (kNB * wave + j) + (lane & 31), C[mb][j][e],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    // Hand-off without release/acquire fences: the partials are agent-scope atomic stores, which
    // gfx950 issues write-through past the XCD's L2 (sc1), s_waitcnt(0) waits until every one has
    // completed, the barrier orders all threads' completed stores before thread 0's arrival count,
    // and the last arrival reads the partials with agent-coherent (sc1) loads, which miss the
    // non-coherent L2. Agent-scope fences would add an L2 write-back (buffer_wbl2 sc1) and
    // invalidate (buffer_inv sc1) per workgroup: measured, they nearly doubled the small-M GEMM
    // (in-projection batch 8: 0.022 -> 0.041 ms; o-projection 0.017 -> 0.029 ms).
    __builtin_amdgcn_s_waitcnt(0);  // the write-through stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
      const int old = __hip_atomic_fetch_add(a.counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.last = old == a.splits - 1;
      if (sh.last) __hip_atomic_store(a.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!sh.last) return;
    // the slices in slice order, this workgroup's own included (its stores have completed), read
    // with agent-coherent (sc1) buffer loads; kZB slices' loads are issued together (a batch past
    // the last slice re-reads the last one and discards it)
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        part, short(0), int(size_t(a.splits) * kBM * kTileN * sizeof(float)), 0x00020000);
    constexpr int kSc1 = 16;  // cache policy bit sc1
    constexpr int kZB = MB == 1 ? 16 / EQ : 2;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) C[mb][j][e] = 0.0f;
    for (int zb = 0; zb < a.splits; zb += kZB) {
      float V[kZB][MB][kNB][4 * EQ];
#pragma unroll
      for (int q = 0; q < kZB; ++q) {
        const int zz = zb + q < a.splits ? zb + q : a.splits - 1;
        const int zoff = zz * kBM * kTileN * int(sizeof(float));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < kNB; ++j)
#pragma unroll
            for (int e = 0; e < 4 * EQ; ++e) {
              const int r = row_of(mb, e) - m0;
              const int off = (r * kTileN + 32 * (kNB * wave + j) + (lane & 31)) * int(sizeof(float));
              V[q][mb][j][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, off, zoff, kSc1));
            }
      }
#pragma unroll
      for (int q = 0; q < kZB; ++q) {
        const bool use = zb + q < a.splits;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int j = 0; j < kNB; ++j)
#pragma unroll
            for (int e = 0; e < 4 * EQ; ++e) C[mb][j][e] = use ? C[mb][j][e] + V[q][mb][j][e] : C[mb][j][e];
      }
    }
  }

  // ---- epilogues --------------------------------------------------------------------------------
  if (a.splits == 1) __syncthreads();  // sh.rs (the split-K path has passed barriers already)
  if constexpr (FUSED) {
    const int head = tn;  // proj column blocks: q heads, gate heads, k heads, v heads
    const int nq = ap.nq, nkv = ap.nkv;
    const bool is_gate = head >= nq && head < 2 * nq;
    float rs[MB][4][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) rs[mb][i][r] = sh.rs[row_of(mb, 4 * i + r) - m0];
    if (is_gate) {
      uint16_t* out = static_cast<uint16_t*>(a.out);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int row = row_of(mb, e);
            if (row < a.m) out[size_t(row) * a.ldo + colw + 32 * j] = bf16_bits(C[mb][j][e] * rs[mb][e >> 2][e & 3]);
          }
      return;
    }
    // q / k / v head: the bf16 tile (exactly what proj would hold) into LDS, then the append rows
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sh.tile[row_of(mb, e) - m0][32 * (kNB * wave + j) + (lane & 31)] = bf16_bits(C[mb][j][e] * rs[mb][e >> 2][e & 3]);
    __syncthreads();
    const int rtype = head < nq ? head : (head < 2 * nq + nkv ? nq + (head - 2 * nq) : nq + nkv + (head - 2 * nq - nkv));
    for (int r = wave; r < kBM && m0 + r < a.m; r += kGWaves) {
      RowLoads L;
      L.m = m0 + r;
      L.r = rtype;
      L.pos = batch.tok_pos[L.m];
      L.raw = *reinterpret_cast<const uint2*>(&sh.tile[r][4 * lane]);
      row_meta(ap, batch, kv, lane, L);
      append_row(ap, kv, sh.stage[wave], lane, L);
    }
    return;
  } else {
    if (a.kind == Q38A_EPI_RESIDUAL) {
      // residual += C; xbf = bf16(residual); sums of squares per 128 columns (reference
      // qgemm.cu:356-380; the sum's order differs: per column pair of waves)
      float ss[MB][4][4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) ss[mb][i][r] = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int row = row_of(mb, e), col = colw + 32 * j;
            if (row < a.m) {
              float* res = a.residual + size_t(row) * a.n + col;
              const float x = *res + C[mb][j][e];
              *res = x;
              a.xbf[size_t(row) * a.n + col] = bf16_bits(x);
              ss[mb][e >> 2][e & 3] += x * x;
            }
          }
      // 32 kNB columns of this wave per row: reduce over the 32 lanes of each half, then the waves
      // of each 128-column block in wave order
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = ss[mb][i][r];
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            ss[mb][i][r] = v;
          }
      for (int mb = 0; mb < MB; ++mb) {
        __syncthreads();
        if ((lane & 31) == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) sh.resid_ss[wave][8 * i + 4 * kg + r] = ss[mb][i][r];
        }
        __syncthreads();
        // 128-column block b: waves b wpb .. b wpb + wpb - 1
        constexpr int wpb = 4 / kNB;
        if (threadIdx.x < 2 * 32) {
          const int bw = threadIdx.x >> 5, r = threadIdx.x & 31;
          const int row = m0 + 32 * mb + r;
          float v = 0.0f;
#pragma unroll
          for (int w = 0; w < wpb; ++w) v += sh.resid_ss[wpb * bw + w][r];
          if (row < a.m) a.partials_out[size_t(row) * a.norm_blocks + (tn * kTileN) / 128 + bw] = v;
        }
      }
      return;
    }
    float rs[MB][4][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) rs[mb][i][r] = sh.rs[row_of(mb, 4 * i + r) - m0];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = row_of(mb, e), col = colw + 32 * j;
          if (row >= a.m || col >= a.n_store) continue;
          const float y = C[mb][j][e] * rs[mb][e >> 2][e & 3];
          if (a.kind == Q38A_EPI_STORE_F32) static_cast<float*>(a.out)[size_t(row) * a.ldo + col] = y;
          else static_cast<uint16_t*>(a.out)[size_t(row) * a.ldo + col] = bf16_bits(y);
        }
  }
}

// Group compute shared by both kernels: T = A . (128 + u) over the group's four 16-k steps of one
// column block, with A's steps in registers.
template <int BITS, int MB>
__device__ inline void group_products(float16_t (&T)[MB], const u32x4 (&Ab)[MB][4], const BWords& bw,
                                      uint32_t magic) {
  auto t_step = [&](auto step) {
    constexpr int s = decltype(step)::value;
    const bf16x8_t bo = b_operand<BITS, s>(bw, magic);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      T[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, Ab[mb][s]), bo,
                                                      s == 0 ? float16_t{} : T[mb], 0, 0, 0);
  };
  t_step(std::integral_constant<int, 0>{});
  t_step(std::integral_constant<int, 1>{});
  t_step(std::integral_constant<int, 2>{});
  t_step(std::integral_constant<int, 3>{});
}

// ---- larger M: 64 x 256 tiles, four waves of 64 x 64 ------------------------------------------
// A and B stream from global memory, two groups in flight per wave; S_g (the rows' sums over a
// group) from one more MFMA per step against a ones operand.
template <int BITS, bool FUSED>
__global__ void __launch_bounds__(threads_of(2)) __attribute__((amdgpu_waves_per_eu(2)))
qgemm_kernel(GemmArgs a, AppendArgs ap, BatchArgs batch, KvArgs kv, MergeIn) {
  constexpr int MB = 2, kNB = nb_of(MB), kBM = 32 * MB;
  __shared__ GemmShared sh;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, kg = lane >> 5;
  const int z = blockIdx.x % a.splits, tile = blockIdx.x / a.splits;
  const int tn = tile % a.tiles_n, m0 = (tile / a.tiles_n) * kBM;
  const int G = a.k / 64;
  const int g0 = int((long long)z * G / a.splits), g1 = int((long long)(z + 1) * G / a.splits);
  const int nb0 = tn * (kTileN / 32) + wave * kNB;  // this wave's first 32-column block

  // A rows of this lane through a buffer resource over the tile's valid rows: rows past M fall
  // outside its range and load as zero without a memory request
  const int valid_rows = a.m - m0 < kBM ? a.m - m0 : kBM;
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(const_cast<uint16_t*>(a.a) + size_t(m0) * a.k), short(0), valid_rows * a.k * int(sizeof(uint16_t)),
      0x00020000);
  const BPlanes bp = make_bplanes<BITS>(a);
  int aoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) aoff[mb] = ((32 * mb + (lane & 31)) * a.k + 8 * kg) * int(sizeof(uint16_t));
  float16_t C[MB][kNB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < kNB; ++j) C[mb][j] = float16_t{};
  const float c0 = 128.0f + float(1 << (BITS - 1));
  const uint32_t magic = 0x43004300u;  // bf16 128 in both halves
  bf16x8_t ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = __bf16(1.0f);

  // two register buffers rotate over the groups; the rotation loop is unrolled, so every buffer
  // index is a constant
  constexpr int kDepth = 2;
  u32x4 A[kDepth][MB][4];
  BWords B[kDepth][kNB];
  auto load_group = [&](u32x4 (&Ab)[MB][4], BWords (&Bb)[kNB], int g) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        Ab[mb][s] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff[mb], (64 * g + 16 * s) * 2, 0));
#pragma unroll
    for (int j = 0; j < kNB; ++j) load_bwords<BITS>(Bb[j], bp, nb0 + j, g, G, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch where it is issued
  };
  // compute_group adds a group's products only when `take` (a padded step of the rotation re-reads
  // the slice's last group and discards it), so the rotation loop has no exits mid-way.
  auto compute_group = [&](const u32x4 (&Ab)[MB][4], const BWords (&Bb)[kNB], bool take) {
    float16_t S[MB];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        S[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, Ab[mb][s]), ones,
                                                        s == 0 ? float16_t{} : S[mb], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      float16_t T[MB];
      group_products<BITS, MB>(T, Ab, Bb[j], magic);
      // a discarded group adds scale 0 times finite sums (non-finite sums already reached C from the
      // group's own step)
      const float sc = take ? bf16_value(uint16_t(Bb[j].scale)) : 0.0f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          C[mb][j][e] = __builtin_fmaf(sc, __builtin_fmaf(-c0, S[mb][e], T[mb][e]), C[mb][j][e]);
    }
  };
  // Loads are unconditional (past the slice end they re-read its last group, which is cached): a
  // load under a branch makes the wait-count bookkeeping assume the worst at the join and wait for
  // the prefetched groups too. (Every slice holds a group: the host plans splits <= k / 64.)
  const int glast = g1 - 1;
  auto gc = [&](int g) { return g < glast ? g : glast; };
  // the tile's row scales (the epilogue reads them after a barrier): before any weight load is in
  // flight, as a branch over outstanding loads would make the loop's waits conservative
  if (threadIdx.x < kBM) sh.rs[threadIdx.x] = row_scale(a, m0 + threadIdx.x);
#pragma unroll
  for (int d = 0; d + 1 < kDepth; ++d) load_group(A[d], B[d], gc(g0 + d));
  for (int g = g0; g < g1; g += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      load_group(A[(d + kDepth - 1) % kDepth], B[(d + kDepth - 1) % kDepth], gc(g + d + kDepth - 1));
      compute_group(A[d], B[d], g + d < g1);
    }
  }
  tile_finish<MB, FUSED>(a, ap, batch, kv, sh, C, tile, z, tn, wave, lane);
}

// ---- large M: 256 x 256 tiles, weights dequantised once per workgroup --------------------------
// Eight waves (4 x 2) of 64 rows x 128 columns. Per 64-k group the workgroup stages its A rows and
// dequantises its 256 columns once into LDS, the weights as bf16(code x scale) (the reference's own
// weight rounding, qgemm.cu), laid out as the MFMA B operand (block, step, lane, 8 k); every wave
// reads its operands with conflict-free 16-byte reads and the MFMA accumulates across groups
// directly: no per-group epilogue, no row-sum MFMA. Each thread loads and dequantises its share of
// the next group while the waves run the current one; one barrier per group. The tile count fills
// the CUs, so no split-K.
constexpr int kBigRows = 256;
constexpr int kBigWaves = 8;
constexpr int kBigThreads = 64 * kBigWaves;

struct alignas(16) BigShared {
  uint16_t b[2][8][4][64][8];  // two groups of the tile's weights: [block][step][lane][k]
  // two groups of the tile's A rows, copied by the DMA path of buffer loads (no registers): row r's
  // 16-byte chunk c (k 8 c .. 8 c + 7) sits in slot c ^ (r % 8), so the MFMA reads of one chunk
  // over 8 consecutive rows hit 8 different bank groups
  u32x4 a[2][kBigRows][8];
  float rs[kBigRows];  // row scales of the folded RMSNorm
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Two dequantised codes -> packed bf16(code x scale) (RNE): x0, x1 are fp32 128 + u (u the stored
// code), sneg = -(128 + 2^(b-1)) * scale, exact in fp32, so fma gives (u - 2^(b-1)) * scale
// exactly before the one rounding to bf16.
__device__ inline uint32_t scaled_pair(float x0, float x1, float sc, float sneg) {
  const float2_t f{__builtin_fmaf(x0, sc, sneg), __builtin_fmaf(x1, sc, sneg)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// Codes 2P and 2P + 1 of step S of a lane word (k 16 S + 8 kg + 2P + e) as fp32 128 + u.
template <int BITS, int S, int P>
__device__ inline void pair_codes(const BWords& b, float& y0, float& y1) {
  constexpr int q = 4 * S + P;
  uint32_t x0 = ((b.lo[S] << (16 - 4 * P)) & 0x000F0000u) | 0x43000000u;  // nibble at bit 4P
  uint32_t x1 = ((b.lo[S] >> (4 * P)) & 0x000F0000u) | 0x43000000u;       // nibble at bit 16 + 4P
  if constexpr (BITS == 5) {
    x0 |= shr<q - 20>(b.hi.x) & 0x00100000u;
    x1 |= shr<q - 4>(b.hi.x) & 0x00100000u;
  }
  if constexpr (BITS == 6) {
    constexpr int r = 2 * (q & 7);
    const uint32_t h = q < 8 ? b.hi.x : b.hi.y;
    x0 |= shr<r - 20>(h) & 0x00300000u;
    x1 |= shr<r - 4>(h) & 0x00300000u;
  }
  y0 = __builtin_bit_cast(float, x0);
  y1 = __builtin_bit_cast(float, x1);
}

// The 8 codes of step S (k 16 S + 8 kg + i, i < 8) as fp32 128 + u.
template <int BITS, int S>
__device__ inline void step_codes(const BWords& b, float (&x)[8]) {
  pair_codes<BITS, S, 0>(b, x[0], x[1]);
  pair_codes<BITS, S, 1>(b, x[2], x[3]);
  pair_codes<BITS, S, 2>(b, x[4], x[5]);
  pair_codes<BITS, S, 3>(b, x[6], x[7]);
}

// load_bwords for a lane-dependent block: the block's part of every offset is per lane (a vector
// offset), the group's part wave-uniform (scalar), so the buffer resource stays uniform.
template <int BITS>
__device__ inline void load_bwords_lane(BWords& b, const BPlanes& p, int nb, int g, int G, int l) {
  constexpr int hb = BITS == 4 ? 0 : BITS == 5 ? 4 : 8;
  const int unit0 = nb * G;  // this lane's block at group 0
  b.lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(p.lo, (unit0 * 64 + l) * 16, g * 1024, 0));
  if constexpr (BITS == 5)
    b.hi = u32x2{__builtin_amdgcn_raw_buffer_load_b32(p.hi, (unit0 * 64 + l) * hb, g * 64 * hb, 0), 0u};
  else if constexpr (BITS == 6)
    b.hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(p.hi, (unit0 * 64 + l) * hb, g * 64 * hb, 0));
  else b.hi = u32x2{0u, 0u};
  b.scale = __builtin_amdgcn_raw_buffer_load_b16(p.sc, (unit0 * 32 + (l & 31)) * 2, g * 64, 0);
}

// Step S of dequant_to_lds (the group's k 16 S .. 16 S + 15 of this lane word).
template <int BITS, int S>
__device__ inline void dequant_step_to_lds(BigShared& sh, int buf, const BWords& b, int blk, int l) {
  const float sc = bf16_value(uint16_t(b.scale));
  const float sneg = -(128.0f + float(1 << (BITS - 1))) * sc;
  float x[8];
  step_codes<BITS, S>(b, x);
  const u32x4 w{scaled_pair(x[0], x[1], sc, sneg), scaled_pair(x[2], x[3], sc, sneg),
                scaled_pair(x[4], x[5], sc, sneg), scaled_pair(x[6], x[7], sc, sneg)};
  *reinterpret_cast<u32x4*>(&sh.b[buf][blk][S][l][0]) = w;
}

template <int BITS>
__device__ inline void dequant_to_lds(BigShared& sh, int buf, const BWords& b, int blk, int l) {
  const float sc = bf16_value(uint16_t(b.scale));
  const float sneg = -(128.0f + float(1 << (BITS - 1))) * sc;
  auto step = [&](auto st) {
    constexpr int S = decltype(st)::value;
    float x[8];
    step_codes<BITS, S>(b, x);
    const u32x4 w{scaled_pair(x[0], x[1], sc, sneg), scaled_pair(x[2], x[3], sc, sneg),
                  scaled_pair(x[4], x[5], sc, sneg), scaled_pair(x[6], x[7], sc, sneg)};
    *reinterpret_cast<u32x4*>(&sh.b[buf][blk][S][l][0]) = w;
  };
  step(std::integral_constant<int, 0>{});
  step(std::integral_constant<int, 1>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 3>{});
}

template <int BITS>
__global__ void __launch_bounds__(kBigThreads) __attribute__((amdgpu_waves_per_eu(2)))
qgemm_big_kernel(GemmArgs a) {
  __shared__ BigShared sh;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, kg = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  // (readfirstlane: wave-uniform values the buffer resources are built from stay in scalar registers)
  const int tn = __builtin_amdgcn_readfirstlane(blockIdx.x % a.tiles_n);
  const int m0 = __builtin_amdgcn_readfirstlane((blockIdx.x / a.tiles_n) * kBigRows);
  const int G = a.k / 64;
  const BPlanes bp = make_bplanes<BITS>(a);

  // the staging thread's half column of weights: block dblk of the tile, lane word dl
  const int dcol = threadIdx.x & 255, dblk = dcol >> 5, dl = (dcol & 31) + 32 * (threadIdx.x >> 8);
  const int dnb = tn * 8 + dblk;
  // and its four 16-byte chunks of A (rows past M load as zero through the buffer's range)
  const int valid_rows = __builtin_amdgcn_readfirstlane(a.m - m0 < kBigRows ? a.m - m0 : kBigRows);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(const_cast<uint16_t*>(a.a) + size_t(m0) * a.k), short(0), valid_rows * a.k * int(sizeof(uint16_t)),
      0x00020000);
  // A rows of group g into buffer buf by the DMA path: wave w copies rows 32 w .. 32 w + 31 in four
  // 1 KB instructions (8 rows each; lane l: row 8 i + l / 8, slot l % 8, i.e. chunk (l % 8) ^ (row % 8))
  auto dma_a = [&](int g, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 32 * wave + 8 * i + (lane >> 3), c = (lane & 7) ^ (r & 7);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ars, (__attribute__((address_space(3))) void*)&sh.a[buf][32 * wave + 8 * i][0], 16, (r * a.k + 8 * c) * 2,
          128 * g, 0, 0);
    }
  };

  float16_t C[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) C[mb][j] = float16_t{};

  if (threadIdx.x < kBigRows) sh.rs[threadIdx.x] = row_scale(a, m0 + threadIdx.x);
  const int glast = G - 1;
  auto gcl = [&](int g) { return g < glast ? g : glast; };
  // the weights two groups ahead in registers: bq[g & 1] holds group g until its dequantisation
  BWords bq[2];
  dma_a(0, 0);
  load_bwords_lane<BITS>(bq[0], bp, dnb, 0, G, dl);
  load_bwords_lane<BITS>(bq[1], bp, dnb, gcl(1), G, dl);
  dequant_to_lds<BITS>(sh, 0, bq[0], dblk, dl);
  __builtin_amdgcn_s_waitcnt(0);  // the DMA copies of group 0 have landed
  __syncthreads();
  // one group: cur = g & 1 (a compile-time constant, so the register ring is indexed statically)
  auto group = [&](int g, auto curc) {
    constexpr int cur = decltype(curc)::value;
    // the next group's A rows into the other buffer (read during the previous group, before its
    // barrier), then group g + 2's weights into the registers group g held
    dma_a(gcl(g + 1), cur ^ 1);
    load_bwords_lane<BITS>(bq[cur], bp, dnb, gcl(g + 2), G, dl);
    const BWords& bnext = bq[cur ^ 1];
    auto step = [&](auto st) {
      constexpr int s = decltype(st)::value;
      bf16x8_t ao[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int r = 64 * wm + 32 * mb + (lane & 31);
        ao[mb] = __builtin_bit_cast(bf16x8_t, sh.a[cur][r][(2 * s + kg) ^ (r & 7)]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8_t bo = *reinterpret_cast<const bf16x8_t*>(&sh.b[cur][4 * wn + j][s][lane][0]);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) C[mb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao[mb], bo, C[mb][j], 0, 0, 0);
      }
      // group g + 1's step s dequantised into the other buffer while these MFMAs run (past the last
      // group: a copy nobody reads)
      dequant_step_to_lds<BITS, s>(sh, cur ^ 1, bnext, dblk, dl);
    };
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    // the DMA copies of group g + 1 have landed (the weight loads issued after them may still be
    // in flight: vmcnt counts in order, three loads per lane word, two for 4-bit weights)
    __builtin_amdgcn_s_waitcnt(BITS == 4 ? 0x0F72 : 0x0F73);
    __syncthreads();
  };
  for (int g = 0; g < G; g += 2) {
    group(g, std::integral_constant<int, 0>{});
    if (g + 1 < G) group(g + 1, std::integral_constant<int, 1>{});
  }

  // ---- epilogue: C element e of (mb, j): row 64 wm + 32 mb + 8 (e / 4) + 4 kg + e % 4, column
  // 256 tn + 128 wn + 32 j + lane % 32
  auto row_of = [&](int mb, int e) { return m0 + 64 * wm + 32 * mb + 8 * (e >> 2) + 4 * kg + (e & 3); };
  const int col0 = tn * kTileN + 128 * wn + (lane & 31);
  if (a.kind == Q38A_EPI_RESIDUAL) {
    // residual += C; xbf = bf16(residual); the wave's 128 columns are one norm block: sums of
    // squares over its 4 column blocks, then over the 32 lanes of each half
    float ss[2][16];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        ss[mb][e] = 0.f;
        const int row = row_of(mb, e);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (row < a.m) {
            const int col = col0 + 32 * j;
            float* res = a.residual + size_t(row) * a.n + col;
            const float x = *res + C[mb][j][e];
            *res = x;
            a.xbf[size_t(row) * a.n + col] = bf16_bits(x);
            ss[mb][e] = __builtin_fmaf(x, x, ss[mb][e]);
          }
        }
      }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float v = ss[mb][e];
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        const int row = row_of(mb, e);
        if ((lane & 31) == 0 && row < a.m) a.partials_out[size_t(row) * a.norm_blocks + (col0 - (lane & 31)) / 128] = v;
      }
    return;
  }
  __syncthreads();  // sh.rs
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = row_of(mb, e);
      if (row >= a.m) continue;
      const float rs = sh.rs[row - m0];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = col0 + 32 * j;
        if (col >= a.n_store) continue;
        const float y = C[mb][j][e] * rs;
        if (a.kind == Q38A_EPI_STORE_F32) static_cast<float*>(a.out)[size_t(row) * a.ldo + col] = y;
        else static_cast<uint16_t*>(a.out)[size_t(row) * a.ldo + col] = bf16_bits(y);
      }
    }
}

// ---- small M (<= 32 rows): 32 x 256 tiles, sixteen waves ---------------------------------------
// A decode step's rows are few, so the launch is a stream of weights: per CU as many weight bytes
// in flight as registers allow. The workgroup's A slice (its rows x the slice's k) and the rows'
// group sums S_g are staged in LDS once; waves keep only weight words in their register pipeline
// (kGemvDepth groups deep). Two sets of eight waves (K parts) each cover half the slice's groups
// for all 256 columns and add their sums through LDS. EV: row quads of the MFMA output that can hold
// rows < M (1 for M <= 8: the epilogue arithmetic of the other 12 elements is skipped).
constexpr int kGemvDepth = 6;
constexpr int kSliceG = 20;                 // most 64-k groups in a workgroup's slice (LDS budget)
constexpr int kSliceStride = 64 * kSliceG + 8;  // bf16 per staged A row (+16 B against bank conflicts)

constexpr int kMaxNormBlocks = 64;  // folded-norm partials per row (hidden <= 8192)
constexpr int kStageChunks = (32 * 8 * kSliceG + 1023) / 1024;      // A chunks per thread
constexpr int kStagePartials = (32 * kMaxNormBlocks + 1023) / 1024;  // partials per thread

struct alignas(16) GemvShared {
  uint16_t a[32][kSliceStride];  // the tile's A rows over the slice (rows >= M: stale)
  float s[kSliceG][32];          // S_g per row
  float p[32 * kMaxNormBlocks];  // the rows' folded-norm partials
};

// MERGE: the staged A is the gated merge of decode split partials (MergeIn) instead of a.a.
template <int BITS, int EV, bool FUSED, bool MERGE>
__global__ void __launch_bounds__(threads_of(1)) __attribute__((amdgpu_waves_per_eu(4)))
qgemv_kernel(GemmArgs a, AppendArgs ap, BatchArgs batch, KvArgs kv, MergeIn mi) {
  constexpr int kKP = kparts_of(1);
  __shared__ GemmShared sh;
  __shared__ GemvShared sv;
  const int hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, wave = hw % waves_of(1), kp = hw / waves_of(1);
  const int kg = lane >> 5;
  const int z = blockIdx.x % a.splits, tile = blockIdx.x / a.splits;
  const int tn = tile % a.tiles_n, m0 = (tile / a.tiles_n) * 32;
  const int G = a.k / 64;
  const int gs0 = int((long long)z * G / a.splits), gs1 = int((long long)(z + 1) * G / a.splits);
  const int gm = gs0 + (gs1 - gs0) / kKP;  // K part 0: [gs0, gm), part 1: [gm, gs1)
  const int g0 = kp == 0 ? gs0 : gm, g1 = kp == 0 ? gm : gs1;
  const int nb = tn * (kTileN / 32) + wave;  // this wave's 32-column block
  const int valid_rows = a.m - m0 < 32 ? a.m - m0 : 32;
  const BPlanes bp = make_bplanes<BITS>(a);

  // B pipeline first, then the staging loads, so one round trip covers them all; loads past the
  // part's end re-read its last group (unconditional loads keep the loop's waits exact)
  BWords B[kGemvDepth];
  const int glast = g1 - 1;
  auto gc = [&](int g) { return g < glast ? g : glast; };
#pragma unroll
  for (int d = 0; d + 1 < kGemvDepth; ++d) {
    load_bwords<BITS>(B[d], bp, nb, gc(g0 + d), G, lane);
    __builtin_amdgcn_sched_barrier(0);  // issue order per group, as in the loop (exact waits there)
  }
  // stage the A rows < M over the slice (16-byte chunks; LDS rows >= M keep whatever they hold: an
  // MFMA output row depends on its A row only, and rows >= M are never stored) and the partials
  // of the folded norm
  {
    const int cpr = 8 * (gs1 - gs0);  // chunks per row
    const int chunks = MERGE ? 0 : valid_rows * cpr;
    u32x4 v[kStageChunks];
#pragma unroll
    for (int i = 0; i < kStageChunks; ++i) {
      const int c = int(threadIdx.x) + i * threads_of(1), r = c / cpr, kc = c % cpr;
      if (c < chunks) v[i] = *reinterpret_cast<const u32x4*>(a.a + size_t(m0 + r) * a.k + 64 * gs0 + 8 * kc);
    }
    if constexpr (MERGE) {
      // four dims of one (row, q head) per step; a row that is not a decode row (n != 1) is zero
      const DecodePlan pl = wave_decode_plan(batch, mi.nkv, mi.max_splits, mi.target_items);
      const int qpr = 16 * (gs1 - gs0);  // quads per row
      for (int c = threadIdx.x; c < valid_rows * qpr; c += threads_of(1)) {
        const int r = c / qpr, kq = c % qpr, k = 64 * gs0 + 4 * kq;
        const int h = k / kHeadDim, d = k % kHeadDim, row = m0 + r;
        const int b = batch.tok_seq[row];
        const int L = decode_len(batch, b);
        uint16_t y[4] = {0, 0, 0, 0};
        if (L > 0)
          merge_quad(mi.scratch + (size_t(b) * mi.nq + h) * mi.max_splits * (kHeadDim + 2),
                     ceil_div_i(ceil_div_i(L, kPageTokens), pl.cp), kHeadDim + 2, d,
                     mi.gate + size_t(row) * mi.ld_gate + h * kHeadDim + d, y);
        *reinterpret_cast<uint2*>(&sv.a[r][4 * kq]) =
            uint2{uint32_t(y[0]) | (uint32_t(y[1]) << 16), uint32_t(y[2]) | (uint32_t(y[3]) << 16)};
      }
    }
    float pv[kStagePartials];
    const int np = valid_rows * a.norm_blocks;
#pragma unroll
    for (int i = 0; i < kStagePartials; ++i) {
      const int c = int(threadIdx.x) + i * threads_of(1);
      if (a.partials_in && c < np) pv[i] = a.partials_in[size_t(m0) * a.norm_blocks + c];
    }
#pragma unroll
    for (int i = 0; i < kStageChunks; ++i) {
      const int c = int(threadIdx.x) + i * threads_of(1), r = c / cpr, kc = c % cpr;
      if (c < chunks) *reinterpret_cast<u32x4*>(&sv.a[r][8 * kc]) = v[i];
    }
#pragma unroll
    for (int i = 0; i < kStagePartials; ++i) {
      const int c = int(threadIdx.x) + i * threads_of(1);
      if (a.partials_in && c < np) sv.p[c] = pv[i];
    }
    __syncthreads();
    // row scales (in block order, as row_scale) and group sums S_g (rows >= M: unused)
    if (threadIdx.x < 32) {
      float rs = 1.0f;
      if (a.partials_in && int(threadIdx.x) < valid_rows) {
        float acc = 0.0f;
        for (int b = 0; b < a.norm_blocks; ++b) acc += sv.p[threadIdx.x * a.norm_blocks + b];
        rs = 1.0f / __builtin_sqrtf(acc * a.inv_hidden + a.eps);
      }
      sh.rs[threadIdx.x] = rs;
    }
    const int ng = gs1 - gs0;
    for (int t = threadIdx.x; t < 32 * ng; t += threads_of(1)) {
      const int gl = t >> 5, r = t & 31;
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(&sv.a[r][64 * gl + 8 * c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc += __builtin_bit_cast(float, w[i] << 16);
          acc += __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
        }
      }
      sv.s[gl][r] = acc;
    }
    __syncthreads();
  }

  float16_t C[1][1];
  C[0][0] = float16_t{};
  const float c0 = 128.0f + float(1 << (BITS - 1));
  const uint32_t magic = 0x43004300u;
  const int arow = lane & 31;
  for (int g = g0; g < g1; g += kGemvDepth) {
#pragma unroll
    for (int d = 0; d < kGemvDepth; ++d) {
      load_bwords<BITS>(B[(d + kGemvDepth - 1) % kGemvDepth], bp, nb, gc(g + d + kGemvDepth - 1), G, lane);
      __builtin_amdgcn_sched_barrier(0);
      const int gl = gc(g + d) - gs0;
      u32x4 Ab[1][4];
#pragma unroll
      for (int s = 0; s < 4; ++s) Ab[0][s] = *reinterpret_cast<const u32x4*>(&sv.a[arow][64 * gl + 16 * s + 8 * kg]);
      float16_t T[1];
      group_products<BITS, 1>(T, Ab, B[d], magic);
      const float sc = g + d < g1 ? bf16_value(uint16_t(B[d].scale)) : 0.0f;
#pragma unroll
      for (int i = 0; i < EV; ++i) {
        const float4 sq = *reinterpret_cast<const float4*>(&sv.s[gl][8 * i + 4 * kg]);
        const float sr[4] = {sq.x, sq.y, sq.z, sq.w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          C[0][0][4 * i + r] = __builtin_fmaf(sc, __builtin_fmaf(-c0, sr[r], T[0][4 * i + r]), C[0][0][4 * i + r]);
      }
    }
  }

  // part 1 hands its sums to part 0 and ends (barriers count only the waves still running)
  if (kp == 1) {
#pragma unroll
    for (int e = 0; e < 4 * EV; ++e) sh.kpart[wave][e][lane] = C[0][0][e];
  }
  __syncthreads();
  if (kp == 1) return;
#pragma unroll
  for (int e = 0; e < 4 * EV; ++e) C[0][0][e] += sh.kpart[wave][e][lane];
  __syncthreads();  // the union's other uses may overwrite kpart from here on
  tile_finish<1, FUSED, EV>(a, ap, batch, kv, sh, C, tile, z, tn, wave, lane);
}

// ---- decode-size M (<= 8 rows) on a wide column grid: 64-column tiles over the whole K --------------
// One 8-wave workgroup per 64-column tile (the in-projection: 224 tiles for 256 CUs). The tile's K
// groups are cut into fixed chunks (two or three groups, both 32-column blocks); the waves take
// chunks from a counter in LDS as they finish, so a wave that the memory system serves late takes
// fewer (with a fixed share of K per wave, the workgroup waited ~4 us for its slowest wave after the
// mean wave was done). Each chunk's sums go to its own LDS slot and the slots are added in chunk
// order: the result does not depend on which wave took which chunk. A wave keeps its next group in
// flight across chunk boundaries (it claims the next chunk when it issues that chunk's first
// loads). A group's A rows come in one 16-byte load per lane (8 rows x 64 k, rows >= M load as
// zero) and pass through the wave's LDS buffer into the MFMA operand layout (loaded straight into
// that layout, 48 of a load's 64 lanes held rows >= 8, four loads per group). Weights are loaded
// non-temporal (read once). Only the 4 MFMA output elements per lane that can hold rows < 8 take
// the per-group epilogue arithmetic. StoreBF16 / StoreF32 only (the residual epilogue's 128-column
// sums of squares would span two tiles).
//
// Measured on the in-projection at M = 8 (HIP events, weights rotating through 8 copies): 17.1 us
// with a fixed share of K per wave and A loaded into the operand layout; 16.1 with the chunk
// claims; 15.0 with the compact A loads and non-temporal weights; 14.7 with 8 waves instead of 16.
// More groups in flight per wave (3 or 4), or 4 waves with 4 in flight, were slower (16-19 us), as
// was staging all of A in LDS once per workgroup (17.4 us).
constexpr int kWideWaves = 8;
constexpr int kWideRows = 8;
constexpr int kWideSlotFloats = 40 * 2 * 4 * 64;  // the chunks' sums in LDS (80 KB)
constexpr int kWideMaxSplits = 8;

// Chunks of a workgroup's Gs groups for tiles of nb 32-column blocks: at most as many as fill the
// LDS slots (40 of two blocks, 20 of four), at least one group each.
__host__ __device__ constexpr int wide_chunks(int nb, int gs) {
  return gs < kWideSlotFloats / (nb * 256) ? gs : kWideSlotFloats / (nb * 256);
}

struct alignas(16) WideShared {
  u32x4 a[kWideWaves][2][8][8];  // per wave and buffer: the group's A rows, [k chunk][row]
  float c[kWideSlotFloats];      // per chunk: [block][element (rows 4 kg + e)][lane]
  float rs[kWideRows];
  float ss[kWideWaves][2];       // residual epilogue: per wave, its two rows' sums of squares
  int next;                      // the next unclaimed chunk
  int last;                      // split-K: this workgroup arrived last
};

// NB: 32-column blocks per tile (2: StoreBF16 / StoreF32; 4: the residual epilogue, whose tile is
// one 128-column block of the sums of squares). gridDim.y: K splits; with more than one, every
// split writes its tile sums (write-through, as in the split-K kernel) and the last to arrive adds
// them in split order and runs the epilogue.
template <int BITS, int NB, bool RES>
__global__ void __launch_bounds__(64 * kWideWaves) qgemv_wide_kernel(GemmArgs a) {
  static_assert(!RES || NB == 4, "the residual epilogue needs 128-column tiles");
  constexpr int kOut = NB * 4 * 64 / (64 * kWideWaves);  // output values per thread
  __shared__ WideShared sh;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, kg = lane >> 5;
  const int tn = blockIdx.x, ks = blockIdx.y, KS = gridDim.y;
  const int G = a.k / 64;
  const int gb = ks * G / KS, Gs = (ks + 1) * G / KS - gb;
  const int NC = wide_chunks(NB, Gs);
  const int nb0 = tn * NB;
  // the counter's first value before any wave claims, and the row scales before any weight load (a
  // branch over outstanding loads would make the waits conservative)
  if (threadIdx.x == 0) sh.next = kWideWaves;
  __syncthreads();
  if (!RES && threadIdx.x < kWideRows) sh.rs[threadIdx.x] = row_scale(a, threadIdx.x);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(const_cast<uint16_t*>(a.a)), short(0), a.m * a.k * int(sizeof(uint16_t)), 0x00020000);
  const BPlanes bp = make_bplanes<BITS>(a);
  // compact A loads: lane = 8 chunk + row (every lane useful; rows >= M load as zero)
  const int aoff = ((lane & 7) * a.k + 8 * (lane >> 3)) * int(sizeof(uint16_t));
  const float c0 = 128.0f + float(1 << (BITS - 1));
  const uint32_t magic = 0x43004300u;
  bf16x8_t ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = __bf16(1.0f);
  float C[NB][4];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) C[j][e] = 0.0f;
  auto chunk_begin = [&](int c) { return gb + c * Gs / NC; };
  // load cursor (wave-uniform): chunk lc (>= NC once the chunks are gone), group lg of it
  int lc = wave, lg = chunk_begin(wave), lend = chunk_begin(wave + 1);
  // two register buffers rotate over the groups
  constexpr int kDepth = 2;
  u32x4 A[kDepth];
  BWords B[kDepth][NB];
  int rc[kDepth], rg[kDepth];  // chunk and group in each buffer (wave-uniform)
  auto load_next = [&](int d) {
    if (lc < NC && lg == lend) {
      int c = 0;
      if (lane == 0) c = atomicAdd(&sh.next, 1);
      lc = __builtin_amdgcn_readfirstlane(c);
      if (lc < NC) { lg = chunk_begin(lc); lend = chunk_begin(lc + 1); }
    }
    const int g = lc < NC ? lg : gb;  // past the last chunk: a valid address, never used
    rc[d] = lc;
    rg[d] = lg;
    A[d] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff, 128 * g, 0));
#pragma unroll
    for (int j = 0; j < NB; ++j) load_bwords<BITS, kNonTemporal>(B[d][j], bp, nb0 + j, g, G, lane);
    __builtin_amdgcn_sched_barrier(0);
    ++lg;
  };
  auto compute = [&](int d) {
    // through the wave's LDS buffer into the operand layout: row lane % 32 (rows >= 8 repeat rows
    // 0-7; their output rows are never read), k chunk 2 s + lane / 32
    sh.a[wave][d][lane >> 3][lane & 7] = A[d];
    u32x4 Ab[1][4];
#pragma unroll
    for (int s = 0; s < 4; ++s) Ab[0][s] = sh.a[wave][d][2 * s + kg][lane & 7];
    // S (the rows' sums over the group) from two 16 x 16 x 32 MFMAs against ones: MFMA row r is
    // A row 4 (r / 8) + r % 4, so that output element e of lane l is row 4 (l / 32) + e, the row of
    // C element e (rows >= 8 of the 32 x 32 output are never read)
    float4_t S = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h)
      S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8_t, sh.a[wave][d][4 * h + (lane >> 4)][4 * ((lane >> 3) & 1) + (lane & 3)]), ones, S,
          0, 0, 0);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      float16_t T[1];
      group_products<BITS, 1>(T, Ab, B[d][j], magic);
      const float sc = bf16_value(uint16_t(B[d][j].scale));
#pragma unroll
      for (int e = 0; e < 4; ++e) C[j][e] = __builtin_fmaf(sc, __builtin_fmaf(-c0, S[e], T[0][e]), C[j][e]);
    }
    if (rg[d] + 1 == chunk_begin(rc[d] + 1)) {  // the chunk's last group: its sums to its slot
      float* slot = sh.c + rc[d] * (NB * 256);
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          slot[(4 * j + e) * 64 + lane] = C[j][e];
          C[j][e] = 0.0f;
        }
    }
  };
  load_next(0);
  for (;;) {
    load_next(1);
    if (rc[0] >= NC) break;
    compute(0);
    load_next(0);
    if (rc[1] >= NC) break;
    compute(1);
  }
  __syncthreads();
  // output value i of this thread: index x = t + 512 i = (block j, element e, lane l); the chunks'
  // sums in chunk order
  const int t = threadIdx.x;
  float v[kOut];
#pragma unroll
  for (int i = 0; i < kOut; ++i) {
    float x = 0.0f;
    for (int c = 0; c < NC; ++c) x += sh.c[c * (NB * 256) + t + 64 * kWideWaves * i];
    v[i] = x;
  }
  if (KS > 1) {
    // the tile's K splits: write-through partials, an arrival count, the last arrival sums them in
    // split order with agent-coherent loads (the hand-off of the split-K kernel, tile_finish)
    float* part = a.ws_partials + size_t(tn) * KS * (NB * 256);
#pragma unroll
    for (int i = 0; i < kOut; ++i)
      __hip_atomic_store(part + ks * (NB * 256) + t + 64 * kWideWaves * i, v[i], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the write-through stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
      const int old = __hip_atomic_fetch_add(a.counters + tn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.last = old == KS - 1;
      if (sh.last) __hip_atomic_store(a.counters + tn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!sh.last) return;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(part, short(0), KS * (NB * 256) * int(sizeof(float)), 0x00020000);
    constexpr int kSc1 = 16;  // cache policy bit sc1
    float V[kWideMaxSplits][kOut];
#pragma unroll
    for (int z = 0; z < kWideMaxSplits; ++z)
#pragma unroll
      for (int i = 0; i < kOut; ++i) {
        const int zz = z < KS ? z : KS - 1;  // past the last split: re-read it, not added
        V[z][i] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(prs, (t + 64 * kWideWaves * i) * 4, zz * NB * 1024, kSc1));
      }
#pragma unroll
    for (int i = 0; i < kOut; ++i) {
      float x = 0.0f;
#pragma unroll
      for (int z = 0; z < kWideMaxSplits; ++z) x = z < KS ? x + V[z][i] : x;
      v[i] = x;
    }
  }
  if constexpr (RES) {
    // residual += C; xbf = bf16(residual); the tile's 128 columns' sums of squares per row: this
    // thread's values (blocks j and j + 2 of row 4 (l / 32) + e), then the 32 lanes of each half
    // wave, then the two waves of each row in wave order
    const int e = (t >> 6) & 3, l = t & 63, row = 4 * (l >> 5) + e;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kOut; ++i) {
      const int j = (t + 64 * kWideWaves * i) >> 8;
      const int col = tn * (32 * NB) + 32 * j + (l & 31);
      if (row < a.m) {
        float* res = a.residual + size_t(row) * a.n + col;
        const float x = *res + v[i];
        *res = x;
        a.xbf[size_t(row) * a.n + col] = bf16_bits(x);
        ss += x * x;
      }
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((lane & 31) == 0) sh.ss[wave][lane >> 5] = ss;
    __syncthreads();
    if (threadIdx.x < kWideRows) {
      // row r = 4 h + e: waves e and e + 4 (blocks 0-1 and 2-3 of element e), half h
      const int r = threadIdx.x, ee = r & 3, h = r >> 2;
      if (r < a.m) a.partials_out[size_t(r) * a.norm_blocks + tn] = sh.ss[ee][h] + sh.ss[ee + 4][h];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kOut; ++i) {
      const int x = t + 64 * kWideWaves * i, j = x >> 8, e = (x >> 6) & 3, l = x & 63;
      const int row = 4 * (l >> 5) + e, col = tn * (32 * NB) + 32 * j + (l & 31);
      if (row >= a.m || col >= a.n_store) continue;
      const float y = v[i] * sh.rs[row];
      if (a.kind == Q38A_EPI_STORE_F32) static_cast<float*>(a.out)[size_t(row) * a.ldo + col] = y;
      else static_cast<uint16_t*>(a.out)[size_t(row) * a.ldo + col] = bf16_bits(y);
    }
  }
}

// The wide-tile plan of a GEMM, or tiles = 0 when the shape does not take it: decode-size M, a
// store epilogue on a weight wide enough to fill the CUs with 64-column tiles (no split-K), or the
// residual epilogue on 128-column tiles with K split to fill the CUs.
struct WidePlan {
  int nb, tiles, splits;
};

WidePlan plan_wide(int m, int n, int k, int kind, int cus) {
  WidePlan p{0, 0, 1};
  const int G = k / 64;
  if (m > kWideRows) return p;
  if (kind != Q38A_EPI_RESIDUAL) {
    if (n / 64 >= (3 * cus) / 4 && wide_chunks(2, G) >= kWideWaves) p = WidePlan{2, n / 64, 1};
  } else if (n % 128 == 0) {
    const int tiles = n / 128;
#ifdef WKS
    int s = WKS;
#else
    int s = cus / tiles;
#endif
    if (s > kWideMaxSplits) s = kWideMaxSplits;
    while (s > 1 && wide_chunks(4, G / s) < kWideWaves) --s;
    if (s >= 1 && tiles * s >= cus / 2 && wide_chunks(4, G / s) >= kWideWaves) p = WidePlan{4, tiles, s};
  }
  return p;
}

// Split-K plan. Small M (qgemv_kernel, one 1024-thread workgroup per CU): slices of at most
// kSliceG groups (the staged A), and at most as many as fill the CUs once without a second round;
// each of the two K parts keeps a group. Larger M (qgemm_kernel): enough workgroups to stream the weights at
// HBM speed (about two per CU), at least four groups per slice.
struct GemmPlan {
  int mb, tiles_m, tiles_n, splits;
};

GemmPlan plan_gemm(int m, int n, int k, int cus) {
  GemmPlan p;
  const int G = k / 64;
  p.mb = m <= 32 && G >= 2 ? 1 : 2;
  p.tiles_m = (m + 32 * p.mb - 1) / (32 * p.mb);
  p.tiles_n = n / kTileN;
  const int tiles = p.tiles_m * p.tiles_n;
  int s = 1;
  if (p.mb == 1) {
    // fill the CUs, but keep about 12 groups per slice at least: a slice's fixed costs (staging,
    // the split-K tail) cost more than idle CUs below that (measured on the o-projection: 8 slices
    // of 12 groups 17.6 us, 12 slices of 8 groups 19.0 us)
    const int s_min = (G + kSliceG - 1) / kSliceG, s_fill = cus / tiles, s_work = G / 12;
    s = s_fill < s_work ? s_fill : s_work;
    if (s < s_min) s = s_min;
    if (s > G / kparts_of(1)) s = G / kparts_of(1);
    if (s < s_min) s = s_min;  // (G / 2 >= ceil(G / 20) for every G >= 2)
  } else {
    while (tiles * s < 2 * cus && G / (2 * s) >= 4 && s < 16) s *= 2;
  }
  p.splits = s;
  return p;
}

}  // namespace

int gemm_workspace_size(int m, int n, int k, int cus, size_t out[2]) {
  const GemmPlan p = plan_gemm(m, n, k, cus);
  const size_t tiles = size_t(p.tiles_m) * p.tiles_n;
  out[0] = p.splits > 1 ? tiles * p.splits * size_t(32 * p.mb) * kTileN : 0;
  out[1] = p.splits > 1 ? tiles : 0;
  // the wide-tile kernel's split partials (residual epilogue), whichever epilogue the caller uses
  const WidePlan wp = plan_wide(m, n, k, Q38A_EPI_RESIDUAL, cus);
  if (wp.tiles > 0 && wp.splits > 1) {
    out[0] = std::max(out[0], size_t(wp.tiles) * wp.splits * wp.nb * 256);
    out[1] = std::max(out[1], size_t(wp.tiles));
  }
  return Q38A_OK;
}

template <int BITS>
void launch_bits(const GemmPlan& pl, bool ev1, int mode, dim3 grid, dim3 block, hipStream_t stream, const GemmArgs& g,
                 const AppendArgs& aa, const BatchArgs& ba, const KvArgs& ka, const MergeIn& mi) {
  if (pl.mb == 1) {
    if (mode == 1) {
      if (ev1) hipLaunchKernelGGL((qgemv_kernel<BITS, 1, true, false>), grid, block, 0, stream, g, aa, ba, ka, mi);
      else hipLaunchKernelGGL((qgemv_kernel<BITS, 4, true, false>), grid, block, 0, stream, g, aa, ba, ka, mi);
    } else if (mode == 2) {
      if (ev1) hipLaunchKernelGGL((qgemv_kernel<BITS, 1, false, true>), grid, block, 0, stream, g, aa, ba, ka, mi);
      else hipLaunchKernelGGL((qgemv_kernel<BITS, 4, false, true>), grid, block, 0, stream, g, aa, ba, ka, mi);
    } else {
      if (ev1) hipLaunchKernelGGL((qgemv_kernel<BITS, 1, false, false>), grid, block, 0, stream, g, aa, ba, ka, mi);
      else hipLaunchKernelGGL((qgemv_kernel<BITS, 4, false, false>), grid, block, 0, stream, g, aa, ba, ka, mi);
    }
  } else {
    if (mode == 1) hipLaunchKernelGGL((qgemm_kernel<BITS, true>), grid, block, 0, stream, g, aa, ba, ka, mi);
    else hipLaunchKernelGGL((qgemm_kernel<BITS, false>), grid, block, 0, stream, g, aa, ba, ka, mi);
  }
}

// ap: the fused in-projection append; mi: the o-projection's A merged from decode partials (only
// plans on the small-M kernel: the caller checks gemm_merge_fits). b: the batch of either.
int launch_qgemm(const uint16_t* A, int m, const q38a_bq_weight& w, const q38a_gemm_epilogue& ep,
                 const q38a_gemm_workspace& ws, const q38a_qk_norm_rope_params* ap, const q38a_batch_desc* b,
                 const q38a_kv_cache_desc* kv, const MergeIn* mi, hipStream_t stream) {
  if (m <= 0) return Q38A_OK;
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  const GemmPlan pl = plan_gemm(m, w.n, w.k, cus);
  if (pl.splits > 1) {
    const size_t tiles = size_t(pl.tiles_m) * pl.tiles_n;
    if (!ws.partials || !ws.counters || ws.partial_floats < tiles * pl.splits * size_t(32 * pl.mb) * kTileN ||
        size_t(ws.num_counters) < tiles)
      return set_error(Q38A_ERR_INVALID, "qgemm: workspace too small (q38a_qgemm_workspace_size)");
  }
  if (pl.mb == 1 && ep.partials_in && ep.kind != Q38A_EPI_RESIDUAL && ep.hidden / 128 > kMaxNormBlocks)
    return set_error(Q38A_ERR_INVALID, "qgemm: hidden %d above %d for the folded norm", ep.hidden,
                     128 * kMaxNormBlocks);
  GemmArgs g{};
  g.a = A;
  g.m = m;
  g.n = w.n;
  g.k = w.k;
  g.lo = w.lo;
  g.hi = w.hi;
  g.scales = w.scales;
  g.kind = ap ? kEpiFused : ep.kind;
  g.out = ep.out;
  g.ldo = ep.ldo;
  g.n_store = ep.n_store > 0 ? ep.n_store : w.rows;
  g.residual = ep.residual;
  g.xbf = ep.xbf;
  g.partials_out = ep.partials_out;
  g.partials_in = ep.kind == Q38A_EPI_RESIDUAL ? nullptr : ep.partials_in;  // (the residual epilogue has no row scale)
  g.norm_blocks = ep.kind == Q38A_EPI_RESIDUAL ? w.n / 128 : ep.hidden / 128;
  g.inv_hidden = ep.hidden > 0 ? 1.0f / float(ep.hidden) : 0.0f;
  g.eps = ep.eps;
  g.tiles_n = pl.tiles_n;
  g.splits = pl.splits;
  g.ws_partials = ws.partials;
  g.counters = ws.counters;
  AppendArgs aa{};
  BatchArgs ba{};
  KvArgs ka{};
  MergeIn mg{};
  if (ap) {
    aa = AppendArgs{ap->proj, ap->ld_proj, ap->q_norm, ap->k_norm, ap->eps, ap->num_q_heads, ap->num_kv_heads,
                    ap->q_out, ap->attn_layer, ap->rope_cos_sin, ap->rope_rows};
    ka = to_args(*kv);
  }
  if (b) ba = to_args(*b);
  if (mi) {
    if (pl.mb != 1) return set_error(Q38A_ERR_INVALID, "qgemm: the merged A needs the small-M kernel");
    mg = *mi;
  }
  const int mode = ap ? 1 : mi ? 2 : 0;
  // large M: 256 x 256 tiles with the weights dequantised once per workgroup, when those tiles fill
  // the CUs. With the append requested, that GEMM and then the append launch: at these sizes the
  // append in the per-group-epilogue kernel's column tiles costs more than the proj round trip
  // (2,048 rows of the in-projection: 0.686 ms fused against 0.455 ms), and the result is then the
  // same bits as the two calls made separately.
  const int big_tiles = ((m + kBigRows - 1) / kBigRows) * (w.n / kTileN);
  if (pl.mb == 2 && mode != 2 && big_tiles >= cus) {
    if (mode == 1) g.kind = ep.kind;
    g.tiles_n = w.n / kTileN;
    g.splits = 1;
    const dim3 bgrid{unsigned(big_tiles)}, bblock{unsigned(kBigThreads)};
    switch (w.bits) {
      case 4: hipLaunchKernelGGL((qgemm_big_kernel<4>), bgrid, bblock, 0, stream, g); break;
      case 5: hipLaunchKernelGGL((qgemm_big_kernel<5>), bgrid, bblock, 0, stream, g); break;
      case 6: hipLaunchKernelGGL((qgemm_big_kernel<6>), bgrid, bblock, 0, stream, g); break;
      default: return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: %d-bit weights are not supported", w.bits);
    }
    if (int rc = check_hip(hipGetLastError(), "qgemm launch")) return rc;
    return mode == 1 ? launch_qk_norm_rope_append(*ap, *b, *kv, stream) : Q38A_OK;
  }
  // decode-size M on a wide weight: the wide-tile kernel (store epilogues: 64-column tiles, no
  // split-K; residual: 128-column tiles, K split). With the append requested, that GEMM and then the
  // append launch (the same bits as the two calls).
  const WidePlan wp = mode == 2 ? WidePlan{0, 0, 1} : plan_wide(m, w.n, w.k, ep.kind, cus);
  if (wp.tiles > 0 && (wp.splits == 1 || (ws.partials && ws.counters &&
                                          ws.partial_floats >= size_t(wp.tiles) * wp.splits * wp.nb * 256 &&
                                          ws.num_counters >= wp.tiles))) {
    if (mode == 1) g.kind = ep.kind;
    const dim3 wgrid(unsigned(wp.tiles), unsigned(wp.splits)), wblock(64 * kWideWaves);
#define Q38A_WIDE(B)                                                                            \
  case B:                                                                                       \
    if (wp.nb == 4) hipLaunchKernelGGL((qgemv_wide_kernel<B, 4, true>), wgrid, wblock, 0, stream, g); \
    else hipLaunchKernelGGL((qgemv_wide_kernel<B, 2, false>), wgrid, wblock, 0, stream, g);       \
    break;
    switch (w.bits) {
      Q38A_WIDE(4)
      Q38A_WIDE(5)
      Q38A_WIDE(6)
      default: return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: %d-bit weights are not supported", w.bits);
    }
#undef Q38A_WIDE
    if (int rc = check_hip(hipGetLastError(), "qgemm launch")) return rc;
    return mode == 1 ? launch_qk_norm_rope_append(*ap, *b, *kv, stream) : Q38A_OK;
  }
  const dim3 grid(unsigned(pl.tiles_m * pl.tiles_n * pl.splits)), block(unsigned(threads_of(pl.mb)));
  const bool ev1 = m <= 8;
  switch (w.bits) {
    case 4: launch_bits<4>(pl, ev1, mode, grid, block, stream, g, aa, ba, ka, mg); break;
    case 5: launch_bits<5>(pl, ev1, mode, grid, block, stream, g, aa, ba, ka, mg); break;
    case 6: launch_bits<6>(pl, ev1, mode, grid, block, stream, g, aa, ba, ka, mg); break;
    default: return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: %d-bit weights are not supported", w.bits);
  }
  return check_hip(hipGetLastError(), "qgemm launch");
}

// Whether q38a_qgemm_merge_oproj runs the merge inside the GEMM for m rows (the small-M kernel).
bool gemm_merge_fits(int m, int n, int k, int cus) { return plan_gemm(m, n, k, cus).mb == 1; }

}  // namespace q38a

using namespace q38a;

namespace {

int validate_gemm(const uint16_t* a, int m, const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
                  const q38a_gemm_workspace* ws) {
  if (!a || !w || !ep || !ws) return set_error(Q38A_ERR_INVALID, "qgemm: null argument");
  if (m < 0) return set_error(Q38A_ERR_INVALID, "qgemm: negative m");
  if (w->bits != 4 && w->bits != 5 && w->bits != 6)
    return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: %d-bit weights are not supported", w->bits);
  if (w->n <= 0 || w->k <= 0 || w->n % 256 || w->k % 64 || w->rows <= 0 || w->rows > w->n)
    return set_error(Q38A_ERR_INVALID, "qgemm: weight %d x %d (rows %d): n % 256 and k % 64 must be 0", w->n, w->k,
                     w->rows);
  if (!w->lo || !w->scales || (w->bits > 4 && !w->hi)) return set_error(Q38A_ERR_INVALID, "qgemm: null weight plane");
  if (ep->kind == Q38A_EPI_RESIDUAL) {
    if (!ep->residual || !ep->xbf || !ep->partials_out)
      return set_error(Q38A_ERR_INVALID, "qgemm: the residual epilogue needs residual, xbf and partials_out");
  } else if (ep->kind == Q38A_EPI_STORE_BF16 || ep->kind == Q38A_EPI_STORE_F32) {
    if (!ep->out || ep->ldo < (ep->n_store > 0 ? ep->n_store : w->rows))
      return set_error(Q38A_ERR_INVALID, "qgemm: out must be set and ldo must cover the stored columns");
  } else {
    return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: epilogue kind %d is not supported", ep->kind);
  }
  if (ep->partials_in && (ep->hidden <= 0 || ep->hidden % 128))
    return set_error(Q38A_ERR_INVALID, "qgemm: folded-norm hidden size must be a positive multiple of 128");
  return Q38A_OK;
}

}  // namespace

extern "C" {

int q38a_qgemm_workspace_size(int m, int n, int k, size_t out[2]) {
  clear_error();
  if (!out || m < 0 || n <= 0 || k <= 0 || n % 256 || k % 64)
    return set_error(Q38A_ERR_INVALID, "qgemm_workspace_size: bad shape");
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  return gemm_workspace_size(m, n, k, cus, out);
}

int q38a_qgemm(const uint16_t* a, int m, const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
               const q38a_gemm_workspace* ws, void* stream) {
  clear_error();
  if (int rc = validate_gemm(a, m, w, ep, ws)) return rc;
  return launch_qgemm(a, m, *w, *ep, *ws, nullptr, nullptr, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

int q38a_qgemm_qkv_append(const uint16_t* a, int m, const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
                          const q38a_gemm_workspace* ws, const q38a_qk_norm_rope_params* p,
                          const q38a_batch_desc* batch, const q38a_kv_cache_desc* kv, void* stream) {
  clear_error();
  if (int rc = validate_gemm(a, m, w, ep, ws)) return rc;
  if (!p || !batch || !kv) return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: null argument");
  if (ep->kind != Q38A_EPI_STORE_BF16)
    return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: the in-projection epilogue is STORE_BF16 into proj");
  if (int rc = validate_batch(batch, true)) return rc;
  if (int rc = validate_kv(kv)) return rc;
  if (batch->num_tokens != m) return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: m %d != batch tokens %d", m, batch->num_tokens);
  const int nq = p->num_q_heads, nkv = p->num_kv_heads;
  if (nq <= 0 || nkv <= 0 || nkv != kv->kv_heads || w->n != 2 * (nq + nkv) * kHeadDim || w->rows != w->n)
    return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: weight rows must be [q | gate | k | v] heads of 256");
  if (!p->q_out || !p->q_norm || !p->k_norm || !p->rope_cos_sin || p->rope_rows <= 0)
    return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: q_out, norms and the RoPE table must be set");
  if (ep->out != p->proj || ep->ldo != p->ld_proj)
    return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: the epilogue's out/ldo must be the append's proj/ld_proj");
  if (ep->n_store != 0 && ep->n_store != w->n)
    return set_error(Q38A_ERR_INVALID, "qgemm_qkv_append: n_store must cover the whole projection");
  return launch_qgemm(a, m, *w, *ep, *ws, p, batch, kv, nullptr, static_cast<hipStream_t>(stream));
}

namespace {

// in_loader: the merge in the small-M GEMM's A staging where the plan takes that kernel
int merge_oproj(const q38a_attention_params* attn, const q38a_batch_desc* batch, const q38a_bq_weight* w,
                const q38a_gemm_epilogue* ep, const q38a_gemm_workspace* ws, void* stream, bool in_loader) {
  clear_error();
  if (!attn || !batch) return set_error(Q38A_ERR_INVALID, "qgemm_merge_oproj: null argument");
  if (int rc = validate_gemm(attn->out, batch->num_tokens, w, ep, ws)) return rc;
  if (int rc = validate_batch(batch, true)) return rc;
  const int nq = attn->num_q_heads, nkv = attn->num_kv_heads;
  if (nq <= 0 || nkv <= 0 || nq % nkv || !attn->gate || !attn->split_scratch || attn->max_splits <= 0 ||
      attn->max_splits > kMaxMergeSplits || attn->ld_gate < nq * kHeadDim)
    return set_error(Q38A_ERR_INVALID, "qgemm_merge_oproj: attention heads, gate, split scratch or max_splits invalid");
  if (batch->num_tokens != batch->num_seqs)
    return set_error(Q38A_ERR_INVALID, "qgemm_merge_oproj: one token per sequence required (M %d, B %d)",
                     batch->num_tokens, batch->num_seqs);
  if (w->k != nq * kHeadDim)
    return set_error(Q38A_ERR_INVALID, "qgemm_merge_oproj: weight k %d != %d q heads x 256", w->k, nq);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int m = batch->num_tokens;
  int cus = 0, grid = 0, target = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  if (int rc = decode_grid(&grid, &target)) return rc;
  if (!in_loader || !gemm_merge_fits(m, w->n, w->k, cus)) {
    // the merge kernel writes attn->out, which the GEMM reads
    if (int rc = launch_attention_merge(*attn, *batch, st)) return rc;
    return launch_qgemm(attn->out, m, *w, *ep, *ws, nullptr, batch, nullptr, nullptr, st);
  }
  const MergeIn mi{attn->split_scratch, attn->gate, attn->ld_gate, nq, nkv, attn->max_splits, target};
  return launch_qgemm(attn->out, m, *w, *ep, *ws, nullptr, batch, nullptr, &mi, st);
}

}  // namespace

int q38a_qgemm_merge_oproj(const q38a_attention_params* attn, const q38a_batch_desc* batch, const q38a_bq_weight* w,
                           const q38a_gemm_epilogue* ep, const q38a_gemm_workspace* ws, void* stream) {
  return merge_oproj(attn, batch, w, ep, ws, stream, false);
}

int q38a_qgemm_merge_oproj_in_loader(const q38a_attention_params* attn, const q38a_batch_desc* batch,
                                     const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
                                     const q38a_gemm_workspace* ws, void* stream) {
  return merge_oproj(attn, batch, w, ep, ws, stream, true);
}

}  // extern "C"
