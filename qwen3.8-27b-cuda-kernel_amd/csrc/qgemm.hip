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
#include "append.hpp"
#include "q38a_gemm.h"

namespace q38a {
namespace {

constexpr int kGWaves = 4;
constexpr int kGThreads = 64 * kGWaves;
constexpr int kNB = 2;                          // 32-column MFMA blocks per wave
constexpr int kTileN = 32 * kNB * kGWaves;      // 256 columns per workgroup
constexpr int kEpiFused = 100;                  // epilogue kind of the fused in-projection

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

// One lane's share of one (32-column block, group) of weights: 32 low nibbles, their high bits, and
// the column's scale.
struct BWords {
  u32x4 lo;
  u32x2 hi;
  float scale;
};

template <int BITS>
__device__ inline void load_bwords(BWords& b, const GemmArgs& a, int nb, int g, int G, int lane) {
  const size_t unit = size_t(nb) * G + g;
  b.lo = *reinterpret_cast<const u32x4*>(a.lo + (unit * 64 + lane) * 16);
  if constexpr (BITS == 5) b.hi = u32x2{*reinterpret_cast<const uint32_t*>(a.hi + (unit * 64 + lane) * 4), 0u};
  else if constexpr (BITS == 6) b.hi = *reinterpret_cast<const u32x2*>(a.hi + (unit * 64 + lane) * 8);
  else b.hi = u32x2{0u, 0u};
  b.scale = bf16_value(a.scales[unit * 32 + (lane & 31)]);
}

// B operand of step s: eight bf16 values 128 + u (pairs p = 0..3 of word s), exact.
template <int BITS>
__device__ inline bf16x8_t b_operand(const BWords& b, int s) {
  u32x4 v;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t w = ((b.lo[s] >> (4 * p)) & 0x000F000Fu) | 0x43004300u;
    const int q = 4 * s + p;
    if constexpr (BITS == 5) w |= ((b.hi.x >> q) << 4) & 0x00100010u;
    if constexpr (BITS == 6) w |= (((q < 8 ? b.hi.x : b.hi.y) >> (2 * (q & 7))) << 4) & 0x00300030u;
    v[p] = w;
  }
  return __builtin_bit_cast(bf16x8_t, v);
}

// Row scale of the folded RMSNorm (reference qgemm.cu:288-297).
__device__ inline float row_scale(const GemmArgs& a, int row) {
  if (!a.partials_in || row >= a.m) return 1.0f;
  const float* pr = a.partials_in + size_t(row) * a.norm_blocks;
  float s = 0.0f;
  for (int b = 0; b < a.norm_blocks; ++b) s += pr[b];
  return 1.0f / __builtin_sqrtf(s * a.inv_hidden + a.eps);
}

struct alignas(16) GemmShared {
  union {
    uint16_t tile[64][kTileN + 8];  // fused epilogue: the bf16 head tile (rows x 256)
    float resid_ss[kGWaves][64][2];  // residual epilogue: per-wave sums of squares of 64 columns
  };
  double stage[kGWaves][kHeadDim];  // the append's sequential-sum fallback
  int last;
};

// C element e of (row block mb, column block j) in this lane: row 32 mb + 8 (e / 4) + 4 (lane / 32) +
// e % 4 of the tile, column 64 wave + 32 j + lane % 32.
template <int BITS, int MB, bool FUSED>
__global__ void __launch_bounds__(kGThreads) qgemm_kernel(GemmArgs a, AppendArgs ap, BatchArgs batch, KvArgs kv) {
  __shared__ GemmShared sh;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = lane >> 5;
  constexpr int kBM = 32 * MB;
  const int bid = blockIdx.x;
  const int z = bid % a.splits, tile = bid / a.splits;
  const int tn = tile % a.tiles_n, tm = tile / a.tiles_n;
  const int m0 = tm * kBM;
  const int G = a.k / 64;
  const int g0 = int((long long)z * G / a.splits), g1 = int((long long)(z + 1) * G / a.splits);
  const int nb0 = tn * (kTileN / 32) + wave * kNB;  // this wave's first 32-column block

  // A rows of this lane (rows past M read as zero)
  const uint16_t* arow[MB];
  bool aok[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = m0 + 32 * mb + (lane & 31);
    aok[mb] = row < a.m;
    arow[mb] = a.a + size_t(aok[mb] ? row : 0) * a.k + 8 * kg;
  }
  float16_t C[MB][kNB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < kNB; ++j) C[mb][j] = float16_t{};
  const float c0 = 128.0f + float(1 << (BITS - 1));
  bf16x8_t ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = __bf16(1.0f);

  u32x4 A[2][MB][4];
  BWords B[2][kNB];
  auto load_group = [&](int buf, int g) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(arow[mb] + 64 * g + 16 * s);
        A[buf][mb][s] = aok[mb] ? v : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
    for (int j = 0; j < kNB; ++j) load_bwords<BITS>(B[buf][j], a, nb0 + j, g, G, lane);
  };
  if (g0 < g1) load_group(0, g0);
  for (int g = g0; g < g1; ++g) {
    const int cur = (g - g0) & 1;
    if (g + 1 < g1) load_group(cur ^ 1, g + 1);
    float16_t T[MB][kNB], S[MB];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bf16x8_t x = __builtin_bit_cast(bf16x8_t, A[cur][mb][s]);
#pragma unroll
        for (int j = 0; j < kNB; ++j)
          T[mb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, b_operand<BITS>(B[cur][j], s),
                                                              s == 0 ? float16_t{} : T[mb][j], 0, 0, 0);
        S[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, ones, s == 0 ? float16_t{} : S[mb], 0, 0, 0);
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        const float sc = B[cur][j].scale;
#pragma unroll
        for (int e = 0; e < 16; ++e) C[mb][j][e] = __builtin_fmaf(sc, __builtin_fmaf(-c0, S[mb][e], T[mb][j][e]), C[mb][j][e]);
      }
  }

  auto row_of = [&](int mb, int e) { return m0 + 32 * mb + 8 * (e >> 2) + 4 * kg + (e & 3); };
  const int colw = tn * kTileN + 64 * wave + (lane & 31);  // + 32 j

  // ---- split-K: the last of the tile's slices sums them in slice order -------------------------
  if (a.splits > 1) {
    float* part = a.ws_partials + size_t(tile) * a.splits * kBM * kTileN;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = row_of(mb, e) - m0;
          if (m0 + r < a.m)
            __hip_atomic_store(part + (size_t(z) * kBM + r) * kTileN + 64 * wave + 32 * j + (lane & 31), C[mb][j][e],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    __builtin_amdgcn_s_waitcnt(0);  // the write-through stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
      const int old = __hip_atomic_fetch_add(a.counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.last = old == a.splits - 1;
      if (sh.last) __hip_atomic_store(a.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!sh.last) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = row_of(mb, e) - m0;
          float sum = 0.0f;
          if (m0 + r < a.m) {
            for (int zz = 0; zz < a.splits; ++zz)
              sum += zz == z ? C[mb][j][e]
                             : __hip_atomic_load(part + (size_t(zz) * kBM + r) * kTileN + 64 * wave + 32 * j + (lane & 31),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          C[mb][j][e] = sum;
        }
  }

  // ---- epilogues --------------------------------------------------------------------------------
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
        for (int r = 0; r < 4; ++r) rs[mb][i][r] = row_scale(a, row_of(mb, 4 * i + r));
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
          sh.tile[row_of(mb, e) - m0][64 * wave + 32 * j + (lane & 31)] = bf16_bits(C[mb][j][e] * rs[mb][e >> 2][e & 3]);
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
      // 64 columns of this wave per row: reduce over the 32 lanes of each half, then pair waves
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
            for (int r = 0; r < 4; ++r) sh.resid_ss[wave][8 * i + 4 * kg + r][0] = ss[mb][i][r];
        }
        __syncthreads();
        // 128-column block b = (64 wave) / 128: waves 2b and 2b + 1
        if (threadIdx.x < 2 * 32) {
          const int bw = threadIdx.x >> 5, r = threadIdx.x & 31;
          const int row = m0 + 32 * mb + r;
          if (row < a.m)
            a.partials_out[size_t(row) * a.norm_blocks + (tn * kTileN) / 128 + bw] =
                sh.resid_ss[2 * bw][r][0] + sh.resid_ss[2 * bw + 1][r][0];
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
        for (int r = 0; r < 4; ++r) rs[mb][i][r] = row_scale(a, row_of(mb, 4 * i + r));
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

// Split-K plan: enough workgroups to stream the weights at HBM speed (about two per CU), at least
// four groups per slice.
struct GemmPlan {
  int mb, tiles_m, tiles_n, splits;
};

GemmPlan plan_gemm(int m, int n, int k, int cus) {
  GemmPlan p;
  p.mb = m <= 32 ? 1 : 2;
  p.tiles_m = (m + 32 * p.mb - 1) / (32 * p.mb);
  p.tiles_n = n / kTileN;
  const int tiles = p.tiles_m * p.tiles_n;
  const int G = k / 64;
  int s = 1;
  while (tiles * s < 2 * cus && G / (2 * s) >= 4 && s < 16) s *= 2;
  p.splits = s;
  return p;
}

}  // namespace

int gemm_workspace_size(int m, int n, int k, int cus, size_t out[2]) {
  const GemmPlan p = plan_gemm(m, n, k, cus);
  const size_t tiles = size_t(p.tiles_m) * p.tiles_n;
  out[0] = p.splits > 1 ? tiles * p.splits * size_t(32 * p.mb) * kTileN : 0;
  out[1] = p.splits > 1 ? tiles : 0;
  return Q38A_OK;
}

int launch_qgemm(const uint16_t* A, int m, const q38a_bq_weight& w, const q38a_gemm_epilogue& ep,
                 const q38a_gemm_workspace& ws, const q38a_qk_norm_rope_params* ap, const q38a_batch_desc* b,
                 const q38a_kv_cache_desc* kv, hipStream_t stream) {
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
  g.partials_in = ep.partials_in;
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
  if (ap) {
    aa = AppendArgs{ap->proj, ap->ld_proj, ap->q_norm, ap->k_norm, ap->eps, ap->num_q_heads, ap->num_kv_heads,
                    ap->q_out, ap->attn_layer, ap->rope_cos_sin, ap->rope_rows};
    ba = to_args(*b);
    ka = to_args(*kv);
  }
  const dim3 grid(unsigned(pl.tiles_m * pl.tiles_n * pl.splits)), block(kGThreads);
#define Q38A_QGEMM_LAUNCH(BITS)                                                                            \
  do {                                                                                                     \
    if (ap) {                                                                                              \
      if (pl.mb == 1) hipLaunchKernelGGL((qgemm_kernel<BITS, 1, true>), grid, block, 0, stream, g, aa, ba, ka); \
      else hipLaunchKernelGGL((qgemm_kernel<BITS, 2, true>), grid, block, 0, stream, g, aa, ba, ka);        \
    } else {                                                                                               \
      if (pl.mb == 1) hipLaunchKernelGGL((qgemm_kernel<BITS, 1, false>), grid, block, 0, stream, g, aa, ba, ka); \
      else hipLaunchKernelGGL((qgemm_kernel<BITS, 2, false>), grid, block, 0, stream, g, aa, ba, ka);       \
    }                                                                                                      \
  } while (0)
  switch (w.bits) {
    case 4: Q38A_QGEMM_LAUNCH(4); break;
    case 5: Q38A_QGEMM_LAUNCH(5); break;
    case 6: Q38A_QGEMM_LAUNCH(6); break;
    default: return set_error(Q38A_ERR_UNSUPPORTED, "qgemm: %d-bit weights are not supported", w.bits);
  }
#undef Q38A_QGEMM_LAUNCH
  return check_hip(hipGetLastError(), "qgemm launch");
}

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
  return launch_qgemm(a, m, *w, *ep, *ws, nullptr, nullptr, nullptr, static_cast<hipStream_t>(stream));
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
  return launch_qgemm(a, m, *w, *ep, *ws, p, batch, kv, static_cast<hipStream_t>(stream));
}

}  // extern "C"
