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

constexpr int kPlanThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kScoreScale = kLog2e / 16.0f;  // 1/sqrt(256) folded into the exp2 domain
constexpr int kMaxSeqs = 1024;  // sequences per step accepted by the attention launchers

struct PlanShared {
  int prefix[kMaxSeqs + 1];  // items before sequence b (decode rows only)
  int wave_tot[kPlanThreads / 64];
  long long red_sum[kPlanThreads / 64];
  int red_max[kPlanThreads / 64];
  int chunk_pages;  // decode plan: pages per item; prefill plan: key blocks per part
};

// Keys of decode row b (a sequence with exactly one token in the step): [0, seq_pos0[b] + 1).
__device__ inline int decode_len(const BatchArgs& b, int s) {
  const int n = b.seq_start[s + 1] - b.seq_start[s];
  return n == 1 ? b.seq_pos0[s] + 1 : 0;
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

// Decode plan: fills sh.prefix[0..B] (items before decode row b) and sh.chunk_pages.
// Must be called by all kPlanThreads threads.
__device__ inline void build_plan(const BatchArgs& batch, int nkv, int max_splits, int target_items, PlanShared& sh) {
  const int B = batch.num_seqs;
  int pages[kPlanPer];
  long long psum = 0;
  int pmax = 0;
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) {
    const int s = threadIdx.x * kPlanPer + i;
    pages[i] = s < B ? ceil_div_i(decode_len(batch, s), kPageTokens) : 0;
    psum += pages[i];
    pmax = max(pmax, pages[i]);
  }
  long long tot;
  int mx;
  block_sum_max(psum, pmax, sh, tot, mx);
  const int by_splits = ceil_div_i(mx, max_splits);
  const int by_target = int((tot * nkv + target_items - 1) / target_items);
  const int cp = max(1, max(by_splits, by_target));
  if (threadIdx.x == 0) sh.chunk_pages = cp;
  int items[kPlanPer];
#pragma unroll
  for (int i = 0; i < kPlanPer; ++i) items[i] = ceil_div_i(pages[i], cp) * nkv;
  block_scan_store(items, B, sh.prefix, sh);
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
constexpr int kPrefillRows = 128;
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
