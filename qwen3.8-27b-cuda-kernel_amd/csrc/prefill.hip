// Causal chunked prefill attention over the paged KV cache on gfx950 fp16 MFMA.
//
// Semantics follow reference src/kernels/attention_prefill.cu:154-313 (exact form
// src/ref/ops.cpp:144-171 applied per token): token i of sequence b (absolute position
// seq_pos0[b] + i) attends to keys [0, seq_pos0[b] + i] of its own cache (the chunk's K/V are
// already appended), softmax(q.k / 16), weighted V, times sigmoid(gate), stored as bf16.
//
// MI355X design (one kv head per workgroup, all of its GQA q heads together):
//   * the q rows of a kv head are the (token, head) pairs of the chunk in token-major order; a
//     workgroup takes 128 consecutive rows (4 waves x 32 rows), so every K/V tile it stages is
//     shared by all 6 q heads, and tiles that straddle tokens need no special casing (the causal
//     limit is per row);
//   * K/V tiles of 32 keys are read as int8 codes + fp16 scales with coalesced 16-byte loads one
//     tile ahead, dequantised (code * scale, rounded once to fp16, exactly like the reference's
//     fp16 staging) into double-buffered LDS: K as [key][dim], V transposed as [dim][key];
//   * S^T[32 keys][32 rows] = K . Q^T on v_mfma_f32_32x32x16_f16 with Q held in registers: the
//     accumulator layout gives each lane one query row and 16 of the tile's keys, so the online
//     softmax needs a single cross-lane step per tile;
//   * O^T[256 dims][32 rows] += V^T . P^T on the same MFMA: the probabilities never leave their
//     lanes (the key order inside the MFMA is permuted to match), O^T stays in 128 registers per
//     lane, and the epilogue divides by l, applies sigmoid(gate) and stores bf16;
//   * workgroups are launched last-tile-first so the longest (latest) rows start first.
#include "plan.hpp"

namespace q38a {
namespace {

constexpr int kPWaves = 4;
constexpr int kPThreads = kPWaves * 64;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerTile = kPWaves * kRowsPerWave;  // 128 (token, head) rows per workgroup
constexpr int kKeyTile = 32;
constexpr int kKStride = kHeadDim + 8;    // halves per K row in LDS (16 B pad: conflict-free reads)
constexpr int kVStride = kKeyTile + 4;    // halves per V^T row in LDS (8 B pad)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kScoreScale = kLog2e / 16.0f;
constexpr float kRescaleSlack = 8.0f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* gate;
  int ld_gate;
  uint16_t* out;
  int nq, nkv, group;
  int attn_layer;
  int tiles_x;  // grid.x (tile index is reversed so the longest rows start first)
};

struct KvTile {
  uint16_t k[kKeyTile][kKStride];  // dequantised K, [key][dim]
  uint16_t vt[kHeadDim][kVStride]; // dequantised V, transposed [dim][key]
};

// One thread's share of a raw int8 tile in registers: K codes of key t/8, dims 32 (t % 8) + [0, 32);
// V codes of keys 8 (t / 64) + [0, 8), dims 4 (t % 64) + [0, 4); and the scales it needs.
struct RawTile {
  u32x4 k[2];
  uint32_t v[8];
  uint16_t ks;      // K scale of (key t/8, group (t % 8) / 2)
  uint16_t vs[8];   // V scales of the 8 keys, group (t % 64) / 16
};

__device__ inline uint16_t half_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// Per-lane byte offsets of a thread's share of a tile, relative to the tile's first key row (K
// and V rows) or first scale entry; V rows and V scales of the 8 keys follow at +256 / +8 per key.
struct TileOffsets {
  int k, ks, v, vs;
};

__device__ inline TileOffsets tile_offsets(const PageLayout& L, int kvh, int tid) {
  TileOffsets o;
  o.k = int(L.k_row(kvh, tid >> 3)) + 32 * (tid & 7);
  o.ks = int(L.k_scales(kvh, tid >> 3)) + 2 * ((tid & 7) >> 1);
  o.v = int(L.v_row(kvh, 8 * (tid >> 6))) + 4 * (tid & 63);
  o.vs = int(L.v_scales(kvh, 8 * (tid >> 6))) + 2 * ((tid & 63) >> 4);
  return o;
}

// rows: page + 256 * (first key of the tile within the page); sc: page + 8 * (same key)
__device__ inline void load_raw(RawTile& R, const uint8_t* rows, const uint8_t* sc, const TileOffsets& o) {
  R.k[0] = *reinterpret_cast<const u32x4*>(rows + o.k);
  R.k[1] = *reinterpret_cast<const u32x4*>(rows + o.k + 16);
  R.ks = *reinterpret_cast<const uint16_t*>(sc + o.ks);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    R.v[e] = *reinterpret_cast<const uint32_t*>(rows + o.v + kHeadDim * e);
    R.vs[e] = *reinterpret_cast<const uint16_t*>(sc + o.vs + 8 * e);
  }
}

// code * scale rounded once to fp16, for a pair: the biased fp16 (1024 + c + 128) minus 1152 is the
// code exactly, and one packed multiply rounds the product.
__device__ inline half2_t dequant_pair(uint32_t biased_pair, half2_t s) {
  const half2_t bias = {_Float16(1152.0f), _Float16(1152.0f)};
  return (__builtin_bit_cast(half2_t, biased_pair) - bias) * s;
}

// Dequantises the raw tile into LDS; keys at or past `limit` (beyond the sequence) become zero.
__device__ inline void store_tile(KvTile& T, const RawTile& R, int key0, int limit, int tid) {
  {
    const int kl = tid >> 3, d0 = 32 * (tid & 7);
    const _Float16 s = key0 + kl < limit ? __builtin_bit_cast(_Float16, R.ks) : _Float16(0.0f);
    const half2_t sv = {s, s};
    uint32_t out[16];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t u = R.k[w >> 2][w & 3] ^ 0x80808080u;
      out[2 * w] = __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), sv));
      out[2 * w + 1] =
          __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), sv));
    }
    u32x4* dst = reinterpret_cast<u32x4*>(&T.k[kl][d0]);
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c] = u32x4{out[4 * c], out[4 * c + 1], out[4 * c + 2], out[4 * c + 3]};
  }
  {
    const int kb = 8 * (tid >> 6), d0 = 4 * (tid & 63);
    half2_t sv[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const _Float16 s0 = key0 + kb + 2 * p < limit ? __builtin_bit_cast(_Float16, R.vs[2 * p]) : _Float16(0.0f);
      const _Float16 s1 = key0 + kb + 2 * p + 1 < limit ? __builtin_bit_cast(_Float16, R.vs[2 * p + 1]) : _Float16(0.0f);
      sv[p] = half2_t{s0, s1};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // dim d0 + i: the 8 keys' byte i
      uint32_t o[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t sel = 0x0C000C00u | (uint32_t(4 + i) << 16) | uint32_t(i);
        const uint32_t x = __builtin_amdgcn_perm(R.v[2 * p + 1], R.v[2 * p], sel) ^ 0x64806480u;
        o[p] = __builtin_bit_cast(uint32_t, dequant_pair(x, sv[p]));
      }
      *reinterpret_cast<u32x2*>(&T.vt[d0 + i][kb]) = u32x2{o[0], o[1]};
      *reinterpret_cast<u32x2*>(&T.vt[d0 + i][kb + 4]) = u32x2{o[2], o[3]};
    }
  }
}

__global__ void __launch_bounds__(kPThreads, 2) attn_prefill_kernel(PrefillArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ KvTile tiles[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = a.tiles_x - 1 - int(blockIdx.x), kvh = blockIdx.y, b = blockIdx.z;
  const int G = a.group;
  const int s0 = batch.seq_start[b];
  const int n = batch.seq_start[b + 1] - s0;
  const int rows = n * G;
  const int r0 = tile * kRowsPerTile;
  if (r0 >= rows) return;
  const int pos0 = batch.seq_pos0[b];
  const int* bt = kv.block_table + size_t(batch.seq_slot[b]) * kv.max_pages_per_seq;
  const uint8_t* layer = kv.pool + size_t(a.attn_layer) * kv.layer_stride;
  const int last_row = min(rows, r0 + kRowsPerTile) - 1;
  const int kend = pos0 + last_row / G + 1;  // keys [0, kend) are needed by this workgroup
  const int ntiles = (kend + kKeyTile - 1) / kKeyTile;

  // this lane's query row (MFMA column): r = r0 + 32 wave + (lane & 31)
  const int col = lane & 31, kg = lane >> 5;
  const int my_row = r0 + kRowsPerWave * wave + col;
  const bool row_ok = my_row < rows;
  const int tok = row_ok ? my_row / G : 0, head = row_ok ? my_row % G : 0;
  const int qpos = pos0 + tok;
  const int wave_qpos_min = pos0 + min(r0 + kRowsPerWave * wave, rows - 1) / G;

  // Q^T operand: step s (dims 16 s + [0, 16)) lane holds dims 16 s + 8 kg + [0, 8) of its row
  half8_t qf[16];
  {
    const uint16_t* qr = a.q + (size_t(s0 + tok) * a.nq + kvh * G + head) * kHeadDim + 8 * kg;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      u32x4 w = *reinterpret_cast<const u32x4*>(qr + 16 * s);
      if (!row_ok) w = u32x4{0u, 0u, 0u, 0u};
      qf[s] = __builtin_bit_cast(half8_t, w);
    }
  }

  float16_t O[8];  // O^T tile dt: dims 32 dt + 8 blk + 4 kg + r (element 4 blk + r), column = row
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) O[dt] = float16_t{};
  float m_run = -INFINITY, l_run = 0.f;

  // The next tile's raw bytes are loaded into registers while the current tile is computed from
  // LDS, then dequantised into the other LDS buffer.
  RawTile R;
  auto page_ptr = [&](int key0) { return layer + size_t(bt[key0 / kPageTokens]) * kv.page_bytes; };
  const TileOffsets toff = tile_offsets(kv.layout, kvh, tid);
  auto fetch = [&](RawTile& RT, int j) {
    if (j < ntiles) {  // uniform
      const uint8_t* pg = page_ptr(j * kKeyTile);
      const int in_page = (j * kKeyTile) % kPageTokens;
      load_raw(RT, pg + in_page * kHeadDim, pg + in_page * 8, toff);
    }
  };
  auto compute = [&](const KvTile& T, int key0) {

    // S^T = K . Q^T: element 4 blk + r is key key0 + 8 blk + 4 kg + r of this lane's row
    float16_t S = {};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const half8_t kf = *reinterpret_cast<const half8_t*>(&T.k[col][16 * s + 8 * kg]);
      S = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], S, 0, 0, 0);
      // bound how far the scheduler hoists operand reads (keeps the live register set small)
      if ((s & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    const bool need_mask = key0 + kKeyTile - 1 > wave_qpos_min;  // wave-uniform
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float x = S[e] * kScoreScale;
      if (need_mask) {
        const int key = key0 + 8 * (e >> 2) + 4 * kg + (e & 3);
        if (key > qpos) x = -INFINITY;
      }
      S[e] = x;
      tmax = fmaxf(tmax, x);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    // Lazy rescaling: the running reference max only moves when a tile's max exceeds it by more
    // than kRescaleSlack (log2 units), so probabilities stay below 2^kRescaleSlack (exact enough in
    // fp16 and fp32) and the O rescale is almost never needed after the first tiles.
    const bool bump = tmax > m_run + kRescaleSlack;
    float corr = 1.0f;
    if (__any(bump)) {
      const float mnew = bump ? tmax : m_run;
      corr = bump ? __builtin_amdgcn_exp2f(m_run - mnew) : 1.0f;
      m_run = mnew;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) O[dt] *= corr;
    }
    // a row that has seen no key yet keeps m = -inf; 0 is then a safe exponent base
    const float base = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    half4_t P[4];  // P^T of this lane: keys 8 blk + 4 kg + r -> P[blk][r]
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = __builtin_amdgcn_exp2f(S[e] - base);
      psum += pe;
      P[e >> 2][e & 3] = _Float16(pe);
    }
    l_run = l_run * corr + psum;
    // O^T += V^T . P^T: MFMA step t covers keys 16 t + {0..3, 8..11} (k-group 0) and
    // 16 t + {4..7, 12..15} (k-group 1), matching where P^T already sits
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const half8_t pb = {P[2 * t][0], P[2 * t][1], P[2 * t][2], P[2 * t][3],
                          P[2 * t + 1][0], P[2 * t + 1][1], P[2 * t + 1][2], P[2 * t + 1][3]};
      const int kk = 16 * t + 4 * kg;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* vr = &T.vt[32 * dt + col][0];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vr + kk);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + kk + 8);
        const half8_t va = __builtin_bit_cast(half8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
        O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, O[dt], 0, 0, 0);
        if ((dt & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  fetch(R, 0);
  store_tile(tiles[0], R, 0, kend, tid);
  __syncthreads();
  for (int j = 0; j < ntiles; ++j) {
    fetch(R, j + 1);
    compute(tiles[j & 1], j * kKeyTile);
    // unconditional (past the last tile it only fills the idle buffer) so that the dequantisation
    // can be scheduled between the MFMAs of this tile
    store_tile(tiles[(j + 1) & 1], R, (j + 1) * kKeyTile, kend, tid);
    __syncthreads();
  }

  // epilogue: O / l * sigmoid(gate) -> bf16
  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  if (!row_ok) return;
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  const size_t m = size_t(s0 + tok);
  const int hq = kvh * G + head;
  const uint16_t* grow = a.gate + m * a.ld_gate + hq * kHeadDim;
  uint16_t* orow = a.out + (m * a.nq + hq) * kHeadDim;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int d = 32 * dt + 8 * blk + 4 * kg;
      const u32x2 gw = *reinterpret_cast<const u32x2*>(grow + d);
      uint32_t o[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float g0 = bf16_value(uint16_t(gw[h])), g1 = bf16_value(uint16_t(gw[h] >> 16));
        const float y0 = O[dt][4 * blk + 2 * h] * inv * (1.0f / (1.0f + expf(-g0)));
        const float y1 = O[dt][4 * blk + 2 * h + 1] * inv * (1.0f / (1.0f + expf(-g1)));
        o[h] = uint32_t(bf16_bits(y0)) | (uint32_t(bf16_bits(y1)) << 16);
      }
      *reinterpret_cast<u32x2*>(orow + d) = u32x2{o[0], o[1]};
    }
  }
}

}  // namespace

int launch_attention_prefill(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                             hipStream_t stream) {
  if (b.num_seqs == 0 || b.num_tokens == 0) return Q38A_OK;
  if (kv.dtype != Q38A_KV_INT8) return set_error(Q38A_ERR_UNSUPPORTED, "attention_prefill: bf16 pages not built yet");
  const int G = p.num_q_heads / p.num_kv_heads;
  const int tiles_x = int((size_t(b.max_tokens_per_seq) * G + kRowsPerTile - 1) / kRowsPerTile);
  PrefillArgs a{p.q, p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, G, p.attn_layer, tiles_x};
  hipLaunchKernelGGL(attn_prefill_kernel, dim3(tiles_x, p.num_kv_heads, b.num_seqs), dim3(kPThreads), 0, stream, a,
                     to_args(b), to_args(kv));
  return check_hip(hipGetLastError(), "attention_prefill launch");
}

int launch_attention_ragged(const q38a_attention_params&, const q38a_batch_desc&, const q38a_kv_cache_desc&,
                            hipStream_t) {
  return set_error(Q38A_ERR_UNSUPPORTED, "attention_ragged: not built yet");
}

}  // namespace q38a
