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
constexpr int kMaxSeqs = 1024;  // sequences per step accepted by the attention launchers

struct PlanShared {
  int prefix[kMaxSeqs + 1];  // items before sequence b (decode rows only)
  int wave_tot[kPlanThreads / 64];
  int red_sum[kPlanThreads / 64];
  int red_max[kPlanThreads / 64];
  int chunk_pages;
};

// Keys of decode row b (a sequence with exactly one token in the step): [0, seq_pos0[b] + 1).
__device__ inline int decode_len(const BatchArgs& b, int s) {
  const int n = b.seq_start[s + 1] - b.seq_start[s];
  return n == 1 ? b.seq_pos0[s] + 1 : 0;
}

__device__ inline int ceil_div_i(int a, int b) { return (a + b - 1) / b; }

// Fills sh.prefix[0..B] and sh.chunk_pages. Must be called by all kPlanThreads threads.
__device__ inline void build_plan(const BatchArgs& batch, int nkv, int max_splits, int target_items, PlanShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = batch.num_seqs;
  constexpr int kPer = (kMaxSeqs + kPlanThreads - 1) / kPlanThreads;
  int pages[kPer];
  int psum = 0, pmax = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int s = tid * kPer + i;
    pages[i] = s < B ? ceil_div_i(decode_len(batch, s), kPageTokens) : 0;
    psum += pages[i];
    pmax = max(pmax, pages[i]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    psum += __shfl_xor(psum, off, 64);
    pmax = max(pmax, __shfl_xor(pmax, off, 64));
  }
  if (lane == 0) {
    sh.red_sum[wave] = psum;
    sh.red_max[wave] = pmax;
  }
  __syncthreads();
  if (tid == 0) {
    long long tot = 0;
    int mx = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      tot += sh.red_sum[w];
      mx = max(mx, sh.red_max[w]);
    }
    const int by_splits = ceil_div_i(mx, max_splits);
    const int by_target = int((tot * nkv + target_items - 1) / target_items);
    sh.chunk_pages = max(1, max(by_splits, by_target));
  }
  __syncthreads();
  const int cp = sh.chunk_pages;
  // exclusive scan of items_b = ceil(pages_b / cp) * nkv
  int local[kPer];
  int run = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    local[i] = run;
    run += ceil_div_i(pages[i], cp) * nkv;
  }
  int incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) sh.wave_tot[wave] = incl;
  __syncthreads();
  int wave_base = 0;
  for (int w = 0; w < wave; ++w) wave_base += sh.wave_tot[w];
  const int excl = wave_base + incl - run;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int s = tid * kPer + i;
    if (s <= B) sh.prefix[s] = excl + local[i];
  }
  __syncthreads();
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
