// Device-side split-KV work plan shared by the decode, ragged and merge kernels.
//
// The reference splits every sequence into the same number of equal token ranges
// (src/kernels/attention_decode.cu:272-277, :107-109), which leaves CUs idle when contexts are
// ragged. Here the unit of work is an "item" = (sequence, kv head, run of chunk_pages pages), with
// chunk_pages chosen once per launch so that
//   - every sequence needs at most max_splits items per kv head (bounds the partial scratch), and
//   - the whole batch yields about `target_items` items (a few per resident workgroup),
// so a persistent grid can stride over items of (nearly) equal size. The plan depends only on
// device-resident metadata (seq_start, seq_pos0), so launches stay graph-capturable, and every
// kernel recomputes it identically.
#pragma once

#include "common.hpp"

namespace q38a {

constexpr int kPlanThreads = 512;  // the ragged launch's workgroup (eight waves)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kScoreScale = kLog2e / 16.0f;  // 1/sqrt(256) folded into the exp2 domain
constexpr int kMaxSeqs = 1024;  // sequences per step accepted by the attention launchers

struct PlanShared {
  int prefix[kMaxSeqs + 1];  // prefill units before sequence b
  int wave_tot[kPlanThreads / 64];
  long long red_sum[kPlanThreads / 64];
  int red_max[kPlanThreads / 64];
  int chunk_pages;  // prefill plan: key blocks per part
};

// Keys of decode row b (a sequence with exactly one token in the step): [0, seq_pos0[b] + 1).
// p[i] for a wave-uniform i as a scalar load (through the constant address space: only for data no
// kernel of the launch writes)
__device__ inline int scalar_load(const int* p, int i) {
  return reinterpret_cast<const __attribute__((address_space(4))) int*>(reinterpret_cast<uintptr_t>(p))[i];
}

// Four such loads issued together (the compiler otherwise sinks a load to its first use, behind
// the others' round trip).
__device__ inline void scalar_load4(const int* p0, int i0, const int* p1, int i1, const int* p2, int i2, const int* p3,
                                    int i3, int& v0, int& v1, int& v2, int& v3) {
  typedef const volatile __attribute__((address_space(4))) int* cp;
  v0 = reinterpret_cast<cp>(reinterpret_cast<uintptr_t>(p0))[i0];
  v1 = reinterpret_cast<cp>(reinterpret_cast<uintptr_t>(p1))[i1];
  v2 = reinterpret_cast<cp>(reinterpret_cast<uintptr_t>(p2))[i2];
  v3 = reinterpret_cast<cp>(reinterpret_cast<uintptr_t>(p3))[i3];
}

__device__ inline int decode_len(const BatchArgs& b, int s) {
  // the three loads are independent (seq_pos0 is read whatever the row's length), so they are one
  // round trip to memory rather than two
  const int s0 = b.seq_start[s], s1 = b.seq_start[s + 1], p = b.seq_pos0[s];
  return s1 - s0 == 1 ? p + 1 : 0;
}

__device__ inline int ceil_div_i(int a, int b) { return (a + b - 1) / b; }

constexpr int kPlanPer = (kMaxSeqs + kPlanThreads - 1) / kPlanThreads;  // sequences per thread

// Block-wide sum and max of per-thread values (all kPlanThreads threads call it).
__device__ inline void block_sum_max(long long v_sum, int v_max, PlanShared& sh, long long& sum, int& mx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v_sum += __shfl_xor(v_sum, off, 64);
    v_max = max(v_max, __shfl_xor(v_max, off, 64));
  }
  if (lane == 0) {
    sh.red_sum[wave] = v_sum;
    sh.red_max[wave] = v_max;
  }
  __syncthreads();
  sum = 0;
  mx = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    sum += sh.red_sum[w];
    mx = max(mx, sh.red_max[w]);
  }
  __syncthreads();
}

// Exclusive prefix sum over sequences: thread t owns sequences t * kPlanPer + i with counts v[i];
// writes dst[s] for s in [0, B] (dst[B] = total). dst may be LDS or global memory.
__device__ inline void block_scan_store(const int (&v)[kPlanPer], int B, int* dst, PlanShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int local[kPlanPer];
  int run = 0;
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) {
    local[i] = run;
    run += v[i];
  }
  int incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int x = __shfl_up(incl, off, 64);
    if (lane >= off) incl += x;
  }
  if (lane == 63) sh.wave_tot[wave] = incl;
  __syncthreads();
  int wave_base = 0;
  for (int w = 0; w < wave; ++w) wave_base += sh.wave_tot[w];
  const int excl = wave_base + incl - run;
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) {
    const int s = tid * kPlanPer + i;
    if (s <= B) dst[s] = excl + local[i];
  }
  __syncthreads();
}

// Decode plan, computed by every wave on its own (no LDS, no barrier), so a workgroup's first loads
// wait only for the sequence metadata. Sequences are scanned 64 at a time, one per lane.
__device__ inline int wave_sum_i(int x) {
  return int(wave_allreduce(uint32_t(x), [](uint32_t a, uint32_t b) { return a + b; }));
}
__device__ inline int wave_max_i(int x) { return wave_max_i32(x); }

struct DecodePlan {
  int cp;      // pages per item (wave-uniform)
  int pages0;  // pages of decode row `lane` (rows 0..63), kept so locating items rereads nothing
  int items;   // decode items of the launch (wave-uniform)
};

__device__ inline int decode_pages(const BatchArgs& batch, int s) {
  return s < batch.num_seqs ? ceil_div_i(decode_len(batch, s), kPageTokens) : 0;
}

// Pages per item of a decode launch: every row needs at most max_splits items per kv head, and the
// batch yields about target_items items.
__device__ inline DecodePlan wave_decode_plan(const BatchArgs& batch, int nkv, int max_splits, int target_items) {
  const int lane = threadIdx.x & 63;
  DecodePlan pl;
  pl.pages0 = decode_pages(batch, lane);
  int psum = pl.pages0, pmax = pl.pages0;  // pages: < 2^31 for any pool a 32-bit block table addresses
  for (int s0 = 64; s0 < batch.num_seqs; s0 += 64) {
    const int p = decode_pages(batch, s0 + lane);
    psum += p;
    pmax = max(pmax, p);
  }
  psum = wave_sum_i(psum);
  pmax = wave_max_i(pmax);
  const int by_splits = ceil_div_i(pmax, max_splits);
  const int by_target = int((static_cast<long long>(psum) * nkv + target_items - 1) / target_items);
  pl.cp = __builtin_amdgcn_readfirstlane(max(1, max(by_splits, by_target)));
  int items = ceil_div_i(pl.pages0, pl.cp);
  for (int s0 = 64; s0 < batch.num_seqs; s0 += 64) items += ceil_div_i(decode_pages(batch, s0 + lane), pl.cp);
  pl.items = __builtin_amdgcn_readfirstlane(wave_sum_i(items) * nkv);
  return pl;
}

struct ItemSpot {
  int seq;    // decode row of the item, or -1 past the last item
  int local;  // item index within the row's items
};

// Locates decode item `item`: the items of row b are ceil(pages_b / cp) * nkv, in row order
// (wave-uniform result).
__device__ inline ItemSpot wave_locate(const BatchArgs& batch, int nkv, const DecodePlan& pl, int item) {
  const int lane = threadIdx.x & 63;
  ItemSpot r{-1, 0};
  int base = 0;
  for (int s0 = 0; s0 < batch.num_seqs && base <= item; s0 += 64) {
    const int p = s0 == 0 ? pl.pages0 : decode_pages(batch, s0 + lane);
    const int n = ceil_div_i(p, pl.cp) * nkv;
    const int incl = wave_incl_scan(n);
    const int excl = base + incl - n;
    const unsigned long long hit = __ballot(n > 0 && excl <= item && item < excl + n);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      r.seq = s0 + l;
      r.local = item - __builtin_amdgcn_readlane(excl, l);
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  r.seq = __builtin_amdgcn_readfirstlane(r.seq);
  r.local = __builtin_amdgcn_readfirstlane(r.local);
  return r;
}

// ---- prefill units ------------------------------------------------------------------------------
// A prefill chunk of n > 1 tokens is cut, per kv head, into row tiles of kPrefillRows consecutive
// (token, q head) rows (token-major). A tile's keys [0, kend) are processed in kKeyTile blocks; the
// ragged launch further cuts every tile of sequence b into parts_b key ranges of at least `chunk` key
// blocks: parts_b = max(1, floor(kt_b / chunk)), kt_b = key blocks of the sequence's last tile,
// chunk = max(min_chunk, ceil(sum_b nkv tiles_b kt_b / target)). Rounding down keeps the split units
// within `target` (one wave of resident workgroups) instead of spilling a short second wave.
// Unit order: sequences in batch order; inside a sequence (tile from last to first, kv head, part),
// so the longest rows start first.
constexpr int kPrefillRows = 256;  // rows of a ragged-launch prefill unit (eight waves of 32)
constexpr int kKeyTile = 32;

__device__ inline int prefill_len(const BatchArgs& b, int s) {
  const int n = b.seq_start[s + 1] - b.seq_start[s];
  return n > 1 ? n : 0;
}
__device__ inline int prefill_tiles(int n, int group) { return ceil_div_i(n * group, kPrefillRows); }
__device__ inline int prefill_key_blocks(const BatchArgs& b, int s, int n) {
  return ceil_div_i(b.seq_pos0[s] + n, kKeyTile);
}
__device__ inline int prefill_parts(int kt, int chunk) { return max(1, kt / chunk); }

// Fills sh.prefix[0..B] (units before sequence b) and sh.chunk_pages (= the key-block chunk).
__device__ inline void build_prefill_plan(const BatchArgs& batch, int group, int nkv, int target, int min_chunk,
                                          PlanShared& sh) {
  const int B = batch.num_seqs;
  int tiles[kPlanPer], kt[kPlanPer];
  long long work = 0;
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) {
    const int s = threadIdx.x * kPlanPer + i;
    const int n = s < B ? prefill_len(batch, s) : 0;
    tiles[i] = n ? prefill_tiles(n, group) : 0;
    kt[i] = n ? prefill_key_blocks(batch, s, n) : 0;
    work += (long long)tiles[i] * kt[i] * nkv;
  }
  long long tot;
  int unused;
  block_sum_max(work, 0, sh, tot, unused);
  const int chunk = max(min_chunk, int((tot + target - 1) / target));
  if (threadIdx.x == 0) sh.chunk_pages = chunk;
  int units[kPlanPer];
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) units[i] = tiles[i] ? tiles[i] * nkv * prefill_parts(kt[i], chunk) : 0;
  block_scan_store(units, B, sh.prefix, sh);
}

// Largest b with prefix[b] <= item (prefix is non-decreasing; prefix[B] = total).
__device__ inline int find_seq(const PlanShared& sh, int B, int item) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (sh.prefix[mid] <= item) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

}  // namespace q38a
