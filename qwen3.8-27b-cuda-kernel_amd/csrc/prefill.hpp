// Causal chunked prefill attention over the paged KV cache on gfx950 fp16 MFMA.
//
// Semantics follow reference src/kernels/attention_prefill.cu:154-313 (exact form
// src/ref/ops.cpp:144-171 applied per token): token i of sequence b (absolute position
// seq_pos0[b] + i) attends to keys [0, seq_pos0[b] + i] of its own cache (the chunk's K/V are
// already appended), softmax(q.k / 16), weighted V, times sigmoid(gate), stored as bf16.
//
// MI355X design (one kv head per workgroup, all of its GQA q heads together):
//   * the q rows of a kv head are the (token, head) pairs of the chunk in token-major order; a
//     workgroup of eight waves takes 256 consecutive rows (32 per wave), so every K/V tile it
//     stages is shared by all of its rows, and tiles that straddle tokens need no special casing
//     (the causal limit is per row);
//   * K/V tiles of 32 keys are read as int8 codes + fp16 scales with coalesced 16-byte loads one
//     tile ahead and staged into double-buffered LDS, K and V both as [key][dim]: K as its exact
//     codes (int8 -> fp16 by a byte permute and one packed add) with the tile's K scales beside
//     them, V dequantised (code * scale rounded once to fp16, like the reference's fp16 staging);
//     bf16 pages are converted to fp16 instead (exact for |x| in fp16's normal range);
//   * S^T[32 keys][32 rows] = K . Q^T on v_mfma_f32_32x32x16_f16: for int8 pages each 64-dim
//     group's partial (exact codes times q, summed in fp32) is multiplied by its per-(key, group) K
//     scale in fp32 and added up, so scores carry no K rounding (the reference's fp16 K staging
//     rounds each value to 2^-11); the accumulator layout gives each lane one query row and 16 of
//     the tile's keys, so the online softmax needs a single cross-lane step per tile;
//   * O^T[256 dims][32 rows] += V^T . P^T on the same MFMA: the V^T operand (4 consecutive keys
//     of one dim per lane) comes straight from the [key][dim] tile through gfx950's transposing
//     LDS read (ds_read_b64_tr_b16), the probabilities never leave their lanes (the key order
//     inside the MFMA is permuted to match), O^T stays in 128 registers per lane, and the epilogue
//     divides by l, applies sigmoid(gate) and stores bf16;
//   * workgroups are launched last-tile-first so the longest (latest) rows start first.
#pragma once

#include <type_traits>

#include "plan.hpp"

namespace q38a {
namespace {

// p[i] through the constant address space (read-only launch metadata): a scalar load
__device__ inline int const_load(const int* p, int i) {
  return reinterpret_cast<const __attribute__((address_space(4))) int*>(reinterpret_cast<uintptr_t>(p))[i];
}

constexpr int kPWaves = 8;
constexpr int kPThreads = kPWaves * 64;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerTile = kPWaves * kRowsPerWave;  // 256 (token, head) rows per workgroup
static_assert(kRowsPerTile == kPrefillRows, "ragged prefill units are prefill workgroup tiles");
// LDS row strides (halves). K rows are read 16 B per lane by 32 different keys (528 B apart: 16
// consecutive keys cover all banks once). V rows are read by ds_read_b64_tr_b16: 32 lanes read 64
// contiguous bytes of each of four consecutive key rows.
//   * int8 pages: a tile is written 16 lanes per key row (one contiguous 256-byte run of the row
//     per store instruction, whatever the stride), so the V stride serves the reads: 576 B (144
//     dwords = 16 mod 64 banks) puts the four rows' 64-byte runs on disjoint banks. Against 16 keys
//     per store instruction and 624 B rows: LDS bank-conflict cycles 9% -> 5% of CU cycles, config
//     3 0.420 -> 0.416 ms. The same staging for bf16 and int8 VT pages was slower (0.415 -> 0.477
//     and 0.467 -> 0.489 ms: the bf16 loop then spilled).
//   * the other tiles write 16 B per lane for 16 consecutive keys per store instruction; their V
//     stride was chosen by measurement: 624 B (and 576, 608, 672) ran the kernel ~15% faster than
//     560, 592, 640 or 656 B.
constexpr int kKStride = kHeadDim + 8;
constexpr int kVStride = kHeadDim + 56;
constexpr int kVStrideRuns = kHeadDim + 32;
// int8 VT pages stage V^T: [dim][key] rows of 32 keys (64 B) padded to 80 B; inside each 16-key
// half the keys are stored in the order 0-3, 8-11, 4-7, 12-15, so the eight keys a lane feeds to
// one PV MFMA (16 t + 4 kg + [0, 4) and + 8) are one 16-byte read.
constexpr int kVtStride = kKeyTile + 8;
constexpr float kRescaleSlack = 8.0f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short short4_lds __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* gate;
  int ld_gate;
  uint16_t* out;
  int nq, nkv, group;
  int attn_layer;
};

template <int VS>
struct alignas(16) KvTileS {
  uint16_t k[kKeyTile][kKStride];  // K, [key][dim]: int8 pages the exact codes, bf16 pages the values
  union {
    uint16_t v[kKeyTile][VS];          // dequantised V, [key][dim]
    uint16_t vt[kHeadDim][kVtStride];  // int8 VT pages: dequantised V^T, [dim][key] (keys permuted)
  };
  // int8 pages: fp16 K scale of (key, 64-dim group g) at ks[g][kg][e] for key 8 (e / 4) + 4 kg + e % 4,
  // the order in which a lane of k-group kg holds its 16 keys of S^T (zero for keys past the sequence)
  uint16_t ks[kHeadDim / 64][2][16];
};
using KvTile = KvTileS<kVStride>;
using KvTileRuns = KvTileS<kVStrideRuns>;  // int8 pages
template <int DT>
using KvTileFor = std::conditional_t<DT == Q38A_KV_INT8, KvTileRuns, KvTile>;

__device__ inline uint16_t half_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// Per-lane byte offsets of a thread's share of a tile, relative to the tile's first key row (K
// and V rows) or first scale entry.
// Per-lane byte offsets of a thread's share of a tile, relative to the tile's first key row (K
// and V rows) or first scale entry.
struct TileOffsets {
  int k, ks, v, vs;
};

// A page as a buffer resource: its loads take a scalar base, this lane's 32-bit offset and a scalar
// offset (the tile's first key), so no 64-bit per-lane addresses are kept in registers.
__device__ inline __amdgpu_buffer_rsrc_t page_rsrc(const uint8_t* page, size_t page_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(page), short(0), int(page_bytes), 0x00020000);
}

// code * scale rounded once to fp16, for a pair: the biased fp16 (1024 + c + 128) minus 1152 is the
// code exactly, and one packed multiply rounds the product.
__device__ inline half2_t dequant_pair(uint32_t biased_pair, half2_t s) {
  const half2_t bias = {_Float16(1152.0f), _Float16(1152.0f)};
  return (__builtin_bit_cast(half2_t, biased_pair) - bias) * s;
}

// 16 int8 codes (one 16-byte word) -> their exact fp16 values at dst (16-byte aligned).
__device__ inline void codes_store16(uint16_t* dst, const u32x4& w) {
  const half2_t bias = {_Float16(1152.0f), _Float16(1152.0f)};
  uint32_t out[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = w[i] ^ 0x80808080u;
    out[2 * i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    out[2 * i + 1] =
        __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
  }
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  d[0] = u32x4{out[0], out[1], out[2], out[3]};
  d[1] = u32x4{out[4], out[5], out[6], out[7]};
}

// Where key k's scales sit in KvTileS::ks (see there).
__device__ inline int ks_slot(int k) { return ((k >> 2) & 1) * 16 + ((k >> 3) << 2) + (k & 3); }

// The K scale of (key, group) into the tile's scale table; zero past the sequence, so those keys'
// scores are finite (they are masked to -inf after QK^T) whatever the page holds there.
template <int VS>
__device__ inline void store_kscale(KvTileS<VS>& T, int key, int group, uint16_t ks, bool live) {
  (&T.ks[group][0][0])[ks_slot(key)] = live ? ks : uint16_t(0);
}

// A thread's share of a raw int8 tile: the K and V codes of key t / 16, dims 16 (t % 16) + [0, 16),
// and the scales of their 64-dim group (16 lanes read a key's whole 256-byte row and write it to
// LDS as one contiguous run).
struct RawTile8 {
  u32x4 k, v;
  uint16_t ks, vs;
};

__device__ inline TileOffsets tile_offsets8(const PageLayout& L, int kvh, int tid) {
  TileOffsets o;
  const int key = tid >> 4, slice = tid & 15;
  o.k = int(L.k_row(kvh, key)) + 16 * slice;
  o.ks = int(L.k_scales(kvh, key)) + 2 * (slice >> 2);
  o.v = int(L.v_row(kvh, key)) + 16 * slice;
  o.vs = int(L.v_scales(kvh, key)) + 2 * (slice >> 2);
  return o;
}

__device__ inline void load_raw(RawTile8& R, __amdgpu_buffer_rsrc_t pg, int srow, int ssc, const TileOffsets& o) {
  R.k = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.k, srow, 0));
  R.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.v, srow, 0));
  R.ks = __builtin_amdgcn_raw_buffer_load_b16(pg, o.ks, ssc, 0);
  R.vs = __builtin_amdgcn_raw_buffer_load_b16(pg, o.vs, ssc, 0);
}

// 16 codes times one scale -> 16 fp16 at dst (16-byte aligned), as dequant_store32.
__device__ inline void dequant_store16(uint16_t* dst, const u32x4& w, _Float16 s) {
  const half2_t sv = {s, s};
  uint32_t out[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u = w[i] ^ 0x80808080u;
    out[2 * i] = __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), sv));
    out[2 * i + 1] =
        __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), sv));
  }
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  d[0] = u32x4{out[0], out[1], out[2], out[3]};
  d[1] = u32x4{out[4], out[5], out[6], out[7]};
}

__device__ inline void store_tile(KvTileRuns& T, const RawTile8& R, int key0, int limit, int tid) {
  const int key = tid >> 4, slice = tid & 15, d0 = 16 * slice;
  const bool live = key0 + key < limit;
  codes_store16(&T.k[key][d0], R.k);
  if ((slice & 3) == 0) store_kscale(T, key, slice >> 2, R.ks, live);
  dequant_store16(&T.v[key][d0], R.v, live ? __builtin_bit_cast(_Float16, R.vs) : _Float16(0.0f));
}

// bf16 pages: key t % 32, dims 16 (t / 32) + [0, 16) of K and V.
struct RawTileBf16x8 {
  u32x4 k[2], v[2];
};

__device__ inline TileOffsets tile_offsets_bf16x8(const PageLayout& L, int kvh, int tid) {
  TileOffsets o;
  const int key = tid & 31, slice = tid >> 5;
  o.k = int(L.k_row(kvh, key)) + 32 * slice;
  o.v = int(L.v_row(kvh, key)) + 32 * slice;
  o.ks = o.vs = 0;
  return o;
}

__device__ inline void load_raw(RawTileBf16x8& R, __amdgpu_buffer_rsrc_t pg, int srow, int, const TileOffsets& o) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    R.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.k, srow + 16 * i, 0));
    R.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.v, srow + 16 * i, 0));
  }
}

// 16 bf16 values -> fp16 at dst (exact for |x| in the fp16 normal range; zero when !live).
__device__ inline void bf16_store16(uint16_t* dst, const u32x4 (&w)[2], bool live) {
  u32x4* d = reinterpret_cast<u32x4*>(dst);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = w[c][i];
      const half2_t h = {_Float16(__uint_as_float(x << 16)), _Float16(__uint_as_float(x & 0xffff0000u))};
      o[i] = live ? __builtin_bit_cast(uint32_t, h) : 0u;
    }
    d[c] = o;
  }
}

__device__ inline void store_tile(KvTile& T, const RawTileBf16x8& R, int key0, int limit, int tid) {
  const int key = tid & 31, d0 = 16 * (tid >> 5);
  const bool live = key0 + key < limit;
  bf16_store16(&T.k[key][d0], R.k, live);
  bf16_store16(&T.v[key][d0], R.v, live);
}

// int8 VT pages: K codes of key t % 32, dims 16 (t / 32) + [0, 16) and
// their group's scale; V^T of dim t / 2, keys 16 (t % 2) + [0, 16) of the tile (one 16-token quarter:
// 16 contiguous bytes), and those keys' scales of the dim's group (group-major: 32 contiguous bytes).
struct RawTileVt8 {
  u32x4 k;
  uint16_t ks;
  u32x4 v;
  u32x4 vs[2];
};

struct TileOffsetsVt {
  int k, ks, v, vs;
};

__device__ inline TileOffsetsVt tile_offsets_vt8(const PageLayout& L, int kvh, int tid) {
  TileOffsetsVt o;
  const int key = tid & 31, slice = tid >> 5;
  o.k = int(L.k_row(kvh, key)) + 16 * slice;
  o.ks = int(L.k_scales(kvh, key)) + 2 * (slice >> 2);
  const int dim = tid >> 1, half = tid & 1;
  o.v = int(L.vt_code(kvh, dim, 16 * half));
  o.vs = int(L.vt_scale(kvh, dim >> 6, 16 * half));
  return o;
}

// in_page: the tile's first token within the page (K rows and V^T quarters advance 256 B per
// token, K scales 8 B, VT V scales 2 B)
__device__ inline void load_raw_vt(RawTileVt8& R, __amdgpu_buffer_rsrc_t pg, int in_page, const TileOffsetsVt& o) {
  R.k = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.k, in_page * kHeadDim, 0));
  R.ks = __builtin_amdgcn_raw_buffer_load_b16(pg, o.ks, in_page * 8, 0);
  R.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.v, in_page * kHeadDim, 0));
  R.vs[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.vs, 2 * in_page, 0));
  R.vs[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pg, o.vs, 2 * in_page + 16, 0));
}

__device__ inline void store_tile(KvTile& T, const RawTileVt8& R, int key0, int limit, int tid) {
  {
    const int key = tid & 31, slice = tid >> 5, d0 = 16 * slice;
    codes_store16(&T.k[key][d0], R.k);
    if ((slice & 3) == 0) store_kscale(T, key, slice >> 2, R.ks, key0 + key < limit);
  }
  // V^T: 16 codes of one dim, each times its own key's scale (zero past the sequence)
  const int dim = tid >> 1, kb = 16 * (tid & 1);
  uint32_t out[8];  // keys kb + 2 i, kb + 2 i + 1 as fp16 pairs
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t u = R.v[w] ^ 0x80808080u;
    const uint32_t sw0 = R.vs[w >> 1][2 * (w & 1)], sw1 = R.vs[w >> 1][2 * (w & 1) + 1];  // scales of keys 4w..4w+3
    half2_t s01 = __builtin_bit_cast(half2_t, sw0), s23 = __builtin_bit_cast(half2_t, sw1);
    const int k = key0 + kb + 4 * w;
    if (k >= limit) s01[0] = _Float16(0.0f);
    if (k + 1 >= limit) s01[1] = _Float16(0.0f);
    if (k + 2 >= limit) s23[0] = _Float16(0.0f);
    if (k + 3 >= limit) s23[1] = _Float16(0.0f);
    out[2 * w] = __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), s01));
    out[2 * w + 1] = __builtin_bit_cast(uint32_t, dequant_pair(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), s23));
  }
  // stored key order 0-3, 8-11, 4-7, 12-15 (8-byte chunks 0, 2, 1, 3)
  u32x4* d = reinterpret_cast<u32x4*>(&T.vt[dim][kb]);
  d[0] = u32x4{out[0], out[1], out[4], out[5]};
  d[1] = u32x4{out[2], out[3], out[6], out[7]};
}

// Four consecutive keys of one dim from V [key][dim] in LDS: the lanes of each 16-lane group pass
// the addresses of V[key0 + j / 4][dim0 + 4 (j % 4)] (j = lane % 16) and lane j receives
// V[key0 + 0..3][dim0 + j].
template <int VS>
__device__ inline half4_t v_keys4(const KvTileS<VS>& T, int key0, int dim0, int j) {
  typedef __attribute__((address_space(3))) short4_lds* lds_ptr;
  const uint16_t* src = &T.v[key0 + (j >> 2)][dim0 + 4 * (j & 3)];
  const short4_lds r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(src));
  return __builtin_bit_cast(half4_t, r);
}

// int8 units keep the Q operand of dims 128..255 in LDS instead of registers: the exact-code QK^T
// needs a second 16-register accumulator and the group scales, which do not fit in a wave's 256
// registers beside O^T (128) and all of Q (64). Each lane reads back only what it wrote (its own row
// and k-group), so the table needs no barrier: [wave][step - 8][lane], 16 B each.
struct alignas(16) QHalfLds {
  u32x4 q[kPWaves][8][64];
};
template <int DT>
constexpr bool kQHalfInLds = DT != Q38A_KV_BF16;

// A split tile's partial row: the normalised output O / l as fp16 (a convex combination of V rows,
// so within V's range; relative error 2^-11, a twentieth of the output tolerance), then the row's
// running max m and sum l in fp32, padded to 528 bytes. Half the bytes of an fp32 accumulator row.
constexpr int kPartialRowFloats = kHeadDim / 2 + 4;

// Row tile `tile` (256 rows) of sequence b and kv head kvh, key blocks [part * kt / parts,
// (part + 1) * kt / parts) of the tile's kt = ceil(kend / 32) blocks. With parts == 1 the result is
// final (normalised, gated, bf16 into a.out); otherwise the tile's partial goes to `partial`:
// [rows][kPartialRowFloats] (O / l in fp16, then m, l per row in the exp2 domain; m = -inf and l = 0
// for a row without keys). qlds: the Q table (int8 pages; unused for bf16 pages).
template <int DT>
__device__ __attribute__((always_inline)) inline void prefill_unit(const PrefillArgs& a, const BatchArgs& batch,
                                                                   const KvArgs& kv, KvTileFor<DT> (&tiles)[2], int b,
                                                                   int kvh, int tile, int part, int parts,
                                                                   float* partial, QHalfLds* qlds) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.group;
  // launch metadata through the constant address space: scalar loads, wave-uniform values (a vector
  // load after a store in the same launch would make every bound derived from it divergent)
  const int s0 = const_load(batch.seq_start, b);
  const int n = const_load(batch.seq_start, b + 1) - s0;
  const int rows = n * G;
  const int r0 = tile * kRowsPerTile;
  if (r0 >= rows) return;
  const int pos0 = const_load(batch.seq_pos0, b);
  const int* bt = kv.block_table + size_t(const_load(batch.seq_slot, b)) * kv.max_pages_per_seq;
  const uint8_t* layer = kv.pool + size_t(a.attn_layer) * kv.layer_stride;
  const int last_row = min(rows, r0 + kRowsPerTile) - 1;
  const int kend = pos0 + last_row / G + 1;  // keys [0, kend) are needed by this workgroup
  const int kt = (kend + kKeyTile - 1) / kKeyTile;
  const int jb = part * kt / parts, je = (part + 1) * kt / parts;  // this unit's key blocks

  // this lane's query row (MFMA column): r = r0 + 32 wave + (lane & 31)
  const int col = lane & 31, kg = lane >> 5;
  const int my_row = r0 + kRowsPerWave * wave + col;
  const bool row_ok = my_row < rows;
  const int tok = row_ok ? my_row / G : 0, head = row_ok ? my_row % G : 0;
  const int qpos = pos0 + tok;
  const int wave_qpos_min = pos0 + min(r0 + kRowsPerWave * wave, rows - 1) / G;

  // Q^T operand: step s (dims 16 s + [0, 16)) lane holds dims 16 s + 8 kg + [0, 8) of its row; int8
  // pages keep steps 8..15 in the LDS table
  constexpr bool kQLds = kQHalfInLds<DT>;
  half8_t qf[16];
  {
    const uint16_t* qr = a.q + (size_t(s0 + tok) * a.nq + kvh * G + head) * kHeadDim + 8 * kg;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      u32x4 w = *reinterpret_cast<const u32x4*>(qr + 16 * s);
      if (!row_ok) w = u32x4{0u, 0u, 0u, 0u};
      if (kQLds && s >= 8) qlds->q[wave][s - 8][lane] = w;
      else qf[s] = __builtin_bit_cast(half8_t, w);
    }
  }

  float16_t O[8];  // O^T tile dt: dims 32 dt + 8 blk + 4 kg + r (element 4 blk + r), column = row
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) O[dt] = float16_t{};
  float m_run = -INFINITY, l_run = 0.f;

  // The next tile's raw bytes are loaded into registers while the current tile is computed from
  // LDS, then staged into the other LDS buffer.
  constexpr bool kVt = DT == Q38A_KV_INT8_VT;
  using Raw = std::conditional_t<kVt, RawTileVt8, std::conditional_t<DT == Q38A_KV_INT8, RawTile8, RawTileBf16x8>>;
  constexpr int kRowBytes = DT != Q38A_KV_BF16 ? kHeadDim : 2 * kHeadDim;
  Raw R;
  // page ids through the constant address space: scalar loads, so a tile's page is a scalar base
  const __attribute__((address_space(4))) int* btc = (const __attribute__((address_space(4))) int*)(bt);
  auto page_ptr = [&](int key0) { return layer + size_t(btc[key0 / kPageTokens]) * kv.page_bytes; };
  using Offsets = std::conditional_t<kVt, TileOffsetsVt, TileOffsets>;
  Offsets toff;
  if constexpr (kVt) toff = tile_offsets_vt8(kv.layout, kvh, tid);
  else if constexpr (DT == Q38A_KV_INT8) toff = tile_offsets8(kv.layout, kvh, tid);
  else toff = tile_offsets_bf16x8(kv.layout, kvh, tid);
  auto fetch = [&](Raw& RT, int j) {
    if (j < je) {  // uniform
      const int in_page = (j * kKeyTile) % kPageTokens;
      if constexpr (kVt) load_raw_vt(RT, page_rsrc(page_ptr(j * kKeyTile), kv.page_bytes), in_page, toff);
      else load_raw(RT, page_rsrc(page_ptr(j * kKeyTile), kv.page_bytes), in_page * kRowBytes, in_page * 8, toff);
    }
  };
  auto compute = [&](const KvTileFor<DT>& T, int key0) {
    // S^T = K . Q^T: element 4 blk + r is key key0 + 8 blk + 4 kg + r of this lane's row
    float16_t S = {};
    // K operand reads run two steps ahead of their MFMA, so an MFMA does not wait for the full LDS
    // latency of its own operand
    constexpr int kKDepth = 2;
    half8_t kb[kKDepth];
    auto kread = [&](int s) { return *reinterpret_cast<const half8_t*>(&T.k[col][16 * s + 8 * kg]); };
#pragma unroll
    for (int s = 0; s < kKDepth; ++s) kb[s] = kread(s);
    if constexpr (DT != Q38A_KV_BF16) {
      // int8 pages: the K operand is the exact codes, so each 64-dim group's partial Sg = codes_g .
      // q_g is a sum of exact products in fp32; the group's K scales (fp16, one per key) multiply it
      // in fp32 as soon as its four MFMAs are done: S = sum_g scale_g * Sg. The Q operand of steps
      // 8..15 comes from the LDS table, read as far ahead as K's. (A second partial buffer, so that
      // a group's fold overlaps the next group's MFMAs, spills and ran config 3 at 0.72 vs 0.53 ms;
      // so did pinning the order with scheduling groups, 0.85 ms.)
      half8_t qb[kKDepth];
      auto qread = [&](int s) { return __builtin_bit_cast(half8_t, qlds->q[wave][s - 8][lane]); };
      half8_t sc[2];  // the scales of this lane's 16 keys in the current group
      auto read_scales = [&](int g) {
        sc[0] = *reinterpret_cast<const half8_t*>(&T.ks[g][kg][0]);
        sc[1] = *reinterpret_cast<const half8_t*>(&T.ks[g][kg][8]);
      };
      read_scales(0);
      float16_t Sg;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const int g = s >> 2;
        const half8_t kf = kb[s % kKDepth];
        const half8_t qv = s < 8 ? qf[s] : qb[s % kKDepth];
        const int nx = s + kKDepth;  // the step whose operands are read now
        if (nx < 16) {
          kb[s % kKDepth] = kread(nx);
          if (nx >= 8) qb[s % kKDepth] = qread(nx);
        }
        Sg = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qv, (s & 3) == 0 ? float16_t{} : Sg, 0, 0, 0);
        if ((s & 3) == 3) {  // group g is complete: fold it, then read the next group's scales
#pragma unroll
          for (int e = 0; e < 16; ++e) S[e] = __builtin_fmaf(Sg[e], float(sc[e >> 3][e & 7]), g == 0 ? 0.0f : S[e]);
          if (g < 3) read_scales(g + 1);
        }
      }
    } else {
      // bf16 pages: K values staged as fp16. The scheduling groups pin the lookahead order (they
      // match by instruction type only: the prologue's reads, then MFMA s and the read for
      // s + kKDepth); left to itself the compiler reads every operand into one register quad right
      // before use.
      __builtin_amdgcn_sched_group_barrier(0x100, kKDepth, 0);  // the prologue's reads first
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const half8_t kf = kb[s % kKDepth];
        if (s + kKDepth < 16) kb[s % kKDepth] = kread(s + kKDepth);
        S = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], S, 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // then MFMA s, read s + depth, ...
        if (s + kKDepth < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    const bool need_mask = key0 + kKeyTile - 1 > wave_qpos_min;  // wave-uniform
    if (need_mask) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = key0 + 8 * (e >> 2) + 4 * kg + (e & 3);
        if (key > qpos) S[e] = -INFINITY;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, S[e]);
    // scores enter the exp2 domain as S * kScoreScale (> 0, so the max commutes with it)
    tmax = xor32_max(tmax) * kScoreScale;
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
      const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(S[e], kScoreScale, -base));
      psum += pe;
      P[e >> 2][e & 3] = _Float16(pe);
    }
    l_run = l_run * corr + psum;
    // O^T += V^T . P^T: MFMA step t covers keys 16 t + {0..3, 8..11} (k-group 0) and
    // 16 t + {4..7, 12..15} (k-group 1), matching where P^T already sits
    // as for K, two transposing reads per operand, three operands ahead (config 3 0.476 -> 0.465 ms;
    // four: no better)
    constexpr int kVDepth = 3;
    auto vread = [&](int i) {  // operand i = 8 t + dt
      const int t = i >> 3, dt = i & 7;
      if constexpr (kVt) {  // V^T rows: the lane's eight keys are adjacent (see kVtStride)
        return *reinterpret_cast<const half8_t*>(&T.vt[32 * dt + (lane & 31)][16 * t + 8 * kg]);
      } else {
        const int kk = 16 * t + 4 * kg;
        const int dim0 = 32 * dt + 16 * ((lane >> 4) & 1);
        const half4_t lo = v_keys4(T, kk, dim0, lane & 15);
        const half4_t hi = v_keys4(T, kk + 8, dim0, lane & 15);
        return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    };
    // A wave issuing its PV MFMAs runs at raised priority, so the other wave of its SIMD (in its
    // softmax or staging) does not delay the MFMA chain (config 3 0.466 -> 0.450-0.459 ms, 4096
    // tokens 0.255 -> 0.242 ms; around QK^T too: no better)
    __builtin_amdgcn_s_setprio(1);
    half8_t vb[kVDepth];
#pragma unroll
    for (int i = 0; i < kVDepth; ++i) vb[i] = vread(i);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kVDepth, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = i >> 3, dt = i & 7;
      const half8_t pb = {P[2 * t][0], P[2 * t][1], P[2 * t][2], P[2 * t][3],
                          P[2 * t + 1][0], P[2 * t + 1][1], P[2 * t + 1][2], P[2 * t + 1][3]};
      const half8_t va = vb[i % kVDepth];
      if (i + kVDepth < 16) vb[i % kVDepth] = vread(i + kVDepth);
      O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, O[dt], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kVDepth < 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  fetch(R, jb);
  store_tile(tiles[jb & 1], R, jb * kKeyTile, kend, tid);
  __syncthreads();
  for (int j = jb; j < je; ++j) {
    fetch(R, j + 1);
    compute(tiles[j & 1], j * kKeyTile);
    // unconditional (past the last tile it only fills the idle buffer) so that the staging can be
    // scheduled between the MFMAs of this tile
    store_tile(tiles[(j + 1) & 1], R, (j + 1) * kKeyTile, kend, tid);
    __syncthreads();
  }

  const float lt = xor32_sum(l_run);
  if (!row_ok) return;
  if (parts > 1) {  // partial row (kPartialRowFloats): O / l as fp16 [256], then m, l (fp32)
    float* row = partial + size_t(my_row - r0) * kPartialRowFloats;
    uint16_t* dst = reinterpret_cast<uint16_t*>(row);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int d = 32 * dt + 8 * blk + 4 * kg;
        const half2_t a = {_Float16(O[dt][4 * blk] * inv), _Float16(O[dt][4 * blk + 1] * inv)};
        const half2_t c = {_Float16(O[dt][4 * blk + 2] * inv), _Float16(O[dt][4 * blk + 3] * inv)};
        *reinterpret_cast<u32x2*>(dst + d) = u32x2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, c)};
      }
    if (kg == 0) *reinterpret_cast<float2*>(row + kHeadDim / 2) = float2{m_run, lt};
    return;
  }
  // final: O / l * sigmoid(gate) -> bf16
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
        const float y0 = O[dt][4 * blk + 2 * h] * inv * fast_sigmoid(g0);
        const float y1 = O[dt][4 * blk + 2 * h + 1] * inv * fast_sigmoid(g1);
        o[h] = uint32_t(bf16_bits(y0)) | (uint32_t(bf16_bits(y1)) << 16);
      }
      *reinterpret_cast<u32x2*>(orow + d) = u32x2{o[0], o[1]};
    }
  }
}

}  // namespace
}  // namespace q38a
