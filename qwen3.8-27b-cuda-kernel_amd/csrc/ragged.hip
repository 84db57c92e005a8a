// Mixed continuous-batching attention (q38a_attention_ragged): decode rows (sequences with one new
// token) and prefill chunks (several new tokens) of one ragged batch in a single attention launch,
// followed by one merge launch.
//
// Semantics are those of attention_decode (reference src/kernels/attention_decode.cu:97-257) for the
// decode rows and attention_prefill (src/kernels/attention_prefill.cu:154-313) for the chunks; the
// reference runs them as separate launches (src/engine.cpp:133-182).
//
// Launch layout: grid = F decode workgroups, P prefill workgroups, then CUs - F more decode
// workgroups (F = CUs / 8 when the batch has a prefill chunk, else 0), all eight waves (512 threads)
// with the same register and LDS budget (one workgroup per CU), so both kinds share the CUs. Eight waves let a prefill unit stage each key tile once for 256 rows (half the staging
// per thread of four-wave units, the registers for the operand lookahead) and a decode item spread
// over eight waves. Workgroups are dispatched in index order: the first F decode workgroups stream
// decode pages from their CUs while the prefill units (aimed at the other CUs) keep the MFMA busy,
// and the later decode workgroups take the remaining decode items (a launch-wide item queue) as
// prefill units finish.
//   * prefill: every (row tile, kv head) of a chunk is cut into parts of about the same number of key
//     blocks (plan.hpp build_prefill_plan) so that a 512-token chunk still spreads over the whole
//     chip; a tile with one part stores its final output, otherwise each part stores an
//     unnormalised partial;
//   * decode: the persistent split-KV loop of attention_decode over the decode rows' items;
//   * merge: one workgroup per (decode row, q head) and one wave per row of each split prefill tile.
// The plan is recomputed on the device from seq_start / seq_pos0 (graph-capturable); the first
// workgroup of each kind records what the merge needs in the scratch header.
//
// Scratch (floats, q38a_ragged_scratch_floats): header (kHeaderInts ints) | claim counters
// (kClaimSlots lines of 128 bytes) | decode partials [B][nq][max_splits][258] | prefill partials
// [units][256 rows][kPartialRowFloats]. The header's queue counter and the claim counters must be
// zero before a scratch buffer's first launch (allocate it zeroed); every launch's merge kernel
// zeroes them again, so launches are independent of each other and of any other scratch buffer.
#include "decode.hpp"
#include "prefill.hpp"

namespace q38a {
namespace {

constexpr int kPrefillTarget = 256;  // prefill units aimed for per launch at most (one per CU on MI355X)
constexpr int kRaggedWaves = 8;
constexpr int kRaggedThreads = 64 * kRaggedWaves;
constexpr int kMinChunk = 16;        // key blocks per part at least (512 keys)
constexpr int kHeaderInts = 4096;
// header: [0] decode pages per item, [1] prefill key blocks per part, [2] decode items,
//         [kTaskPrefix + b] merge tasks (split tile, kv head) before sequence b,
//         [kUnitPrefix + b] prefill units before sequence b, [kParts + b] parts per tile,
//         [kQueue] the decode item queue (a 128-byte line of its own)
constexpr int kTaskPrefix = 4;
constexpr int kUnitPrefix = kTaskPrefix + kMaxSeqs + 1;
constexpr int kParts = kUnitPrefix + kMaxSeqs + 1;
constexpr int kQueue = kHeaderInts - kClaimStride;
static_assert(kParts + kMaxSeqs <= kQueue, "ragged scratch header");
constexpr size_t kClaimFloats = size_t(kClaimSlots) * kClaimStride;

struct RaggedArgs {
  int prefill_blocks;
  int decode_first;    // decode workgroups placed before the prefill units (0: after them)
  int prefill_target;  // prefill units aimed for
  int* header;
  float* prefill_partials;
};

__device__ inline int parts_of(const BatchArgs& batch, int s, int chunk) {
  const int n = prefill_len(batch, s);
  return n ? prefill_parts(prefill_key_blocks(batch, s, n), chunk) : 0;
}

template <int DT>
__global__ void __launch_bounds__(kRaggedThreads, 1)
    attn_ragged_kernel(RaggedArgs r, DecodeArgs d, PrefillArgs pa, BatchArgs batch, KvArgs kv) {
  static_assert(kRaggedThreads == kPThreads && kRaggedThreads == kPlanThreads, "one block shape for both kinds");
  __shared__ PlanShared plan;
  __shared__ union alignas(16) Work {
    struct {
      KvTileFor<DT> tiles[2];
      std::conditional_t<kQHalfInLds<DT>, QHalfLds, char> qh;
    } pre;
    DecodeShared<kRaggedWaves> dec;
  } sh;
  const int B = batch.num_seqs;
  const int bid = int(blockIdx.x);
  const bool is_prefill = bid >= r.decode_first && bid < r.decode_first + r.prefill_blocks;
  if (is_prefill) {
    {
      build_prefill_plan(batch, pa.group, pa.nkv, r.prefill_target, kMinChunk, plan);
      const int chunk = plan.chunk_pages;
      const int u = bid - r.decode_first;
      if (u == 0) {  // what the merge needs: parts, unit and merge-task offsets per sequence
        int tasks[kPlanPer];
#pragma unroll
        for (int i = 0; i < kPlanPer; ++i) {
          const int s = threadIdx.x * kPlanPer + i;
          const int parts = s < B ? parts_of(batch, s, chunk) : 0;
          tasks[i] = parts > 1 ? prefill_tiles(prefill_len(batch, s), pa.group) * pa.nkv : 0;
          if (s < B) r.header[kParts + s] = parts;
          if (s <= B) r.header[kUnitPrefix + s] = plan.prefix[s];
        }
        if (threadIdx.x == 0) r.header[1] = chunk;
        block_scan_store(tasks, B, r.header + kTaskPrefix, plan);
      }
      if (u >= plan.prefix[B]) return;
      const int b = __builtin_amdgcn_readfirstlane(find_seq(plan, B, u));
      const int local = u - plan.prefix[b];
      const int n = prefill_len(batch, b);
      const int parts = parts_of(batch, b, chunk);
      const int tile_r = local / (pa.nkv * parts), rem = local % (pa.nkv * parts);
      const int tile = prefill_tiles(n, pa.group) - 1 - tile_r;
      QHalfLds* qp = nullptr;
      if constexpr (kQHalfInLds<DT>) qp = &sh.pre.qh;
      prefill_unit<DT>(pa, batch, kv, sh.pre.tiles, b, rem / parts, tile, rem % parts,
                                                         parts,
                                                         r.prefill_partials + size_t(u) * kPrefillRows * kPartialRowFloats,
                                                         qp);
    }
  } else {
    const DecodePlan pl = wave_decode_plan(batch, d.nkv, d.max_splits, d.target_items);
    const int wg = bid < r.decode_first ? bid : bid - r.prefill_blocks;
    if (wg == 0 && threadIdx.x == 0) {
      r.header[0] = pl.cp;
      r.header[2] = pl.items;
    }
    decode_items<DT, kRaggedWaves>(d, batch, kv, pl, sh.dec, wg, int(gridDim.x) - r.prefill_blocks);
  }
}

struct RaggedMergeArgs {
  const uint16_t* gate;
  int ld_gate;
  uint16_t* out;
  int nq, nkv, group;
  const int* header;
  const float* decode_partials;
  const float* prefill_partials;
  int max_splits;
  int* queue;
  int* claims;
};

// grid: B * nq decode blocks (a workgroup per decode row and q head), then kPrefillRows / 4 blocks
// per possible merge task (a wave per row of the split tile).
__global__ void __launch_bounds__(kMergeThreads) attn_ragged_merge_kernel(RaggedMergeArgs a, BatchArgs batch) {
  __shared__ MergeShared sh;
  const int B = batch.num_seqs;
  const int blk = blockIdx.x;
  // The attention kernel has finished (same stream): zero the counters it used for the next launch.
  // Claim slots are indexed by a team's first item, so slots [0, items) cover every used one (the
  // attention kernel's first decode workgroup recorded the item count).
  {
    const int used = min(a.header[2], kClaimSlots);
    for (int i = blk * kMergeThreads + int(threadIdx.x); i < used; i += int(gridDim.x) * kMergeThreads)
      a.claims[size_t(i) * kClaimStride] = 0;
    if (blk == 0 && threadIdx.x == 0) *a.queue = 0;
  }
  if (blk < B * a.nq) {
    const int b = blk / a.nq, hq = blk % a.nq;
    // all four loads before the branch: one round trip before the partials
    const int L = decode_len(batch, b);
    const int row = batch.seq_start[b];
    const int cp = a.header[0];
    if (L == 0) return;
    const int splits = ceil_div_i(ceil_div_i(L, kPageTokens), cp);
    const float* src = a.decode_partials + (size_t(b) * a.nq + hq) * a.max_splits * (kHeadDim + 2);
    merge_row_wg(src, splits, kHeadDim + 2, a.gate + size_t(row) * a.ld_gate + hq * kHeadDim,
                 a.out + (size_t(row) * a.nq + hq) * kHeadDim, sh);
    return;
  }
  const int idx = blk - B * a.nq;
  constexpr int kBlocksPerTask = kPrefillRows / kMergeWaves;
  const int task = idx / kBlocksPerTask;
  const int rt = (idx % kBlocksPerTask) * kMergeWaves + int(threadIdx.x >> 6);  // row within the tile
  const int* tp = a.header + kTaskPrefix;
  const int G = a.group;
  int b, parts, local, n, unit0, start;
  if (B < 64) {
    // one round trip: lane s reads sequence s's task prefix (lane B: the task count), parts, unit
    // prefix and token range; the task's sequence is the largest s with prefix <= task (a binary
    // search over the prefix took four dependent loads: config 4's merge 17.1 -> 14.8 us)
    // (indices clamped so that every load is unconditional: one batch, one wait)
    const int s = threadIdx.x & 63;
    const bool in = s < B;
    const int sc = in ? s : B - 1;
    const int tps = tp[s <= B ? s : B];
    const int pts = a.header[kParts + sc], ups = a.header[kUnitPrefix + sc];
    const int s0 = batch.seq_start[sc], s1 = batch.seq_start[sc + 1];
    if (task >= __builtin_amdgcn_readlane(tps, B)) return;
    const unsigned long long le = __ballot(in && tps <= task);
    b = 63 - __builtin_clzll(le);
    parts = __builtin_amdgcn_readlane(pts, b);
    local = task - __builtin_amdgcn_readlane(tps, b);
    unit0 = __builtin_amdgcn_readlane(ups, b);
    start = __builtin_amdgcn_readlane(s0, b);
    const int len = __builtin_amdgcn_readlane(s1, b) - start;
    n = len > 1 ? len : 0;
  } else {
    if (task >= tp[B]) return;
    int lo = 0, hi = B - 1;  // sequence of the task: largest b with tp[b] <= task
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tp[mid] <= task) lo = mid;
      else hi = mid - 1;
    }
    b = lo;
    parts = a.header[kParts + b];
    local = task - tp[b];
    unit0 = a.header[kUnitPrefix + b];
    start = batch.seq_start[b];
    n = prefill_len(batch, b);
  }
  const int tile_r = local / a.nkv, kvh = local % a.nkv;
  const int row = kPrefillRows * (prefill_tiles(n, G) - 1 - tile_r) + rt;
  if (row >= n * G) return;
  const size_t unit = size_t(unit0) + size_t(tile_r * a.nkv + kvh) * parts;
  const size_t unit_floats = size_t(kPrefillRows) * kPartialRowFloats;
  const int tok = row / G, hq = kvh * G + row % G;
  const size_t m = size_t(start + tok);
  merge_row_h16(a.prefill_partials + unit * unit_floats + size_t(rt) * kPartialRowFloats, parts, unit_floats,
                a.gate + m * a.ld_gate + hq * kHeadDim, a.out + (m * a.nq + hq) * kHeadDim);
}

struct RaggedShape {
  size_t decode_floats, tasks_bound, units_bound;
};

RaggedShape ragged_shape(int num_seqs, int num_tokens, int max_tokens_per_seq, int nq, int nkv, int max_splits) {
  RaggedShape s{};
  s.decode_floats = size_t(num_seqs) * nq * max_splits * (kHeadDim + 2);
  if (max_tokens_per_seq > 1) {
    const size_t G = size_t(nq / nkv);
    // sum_b ceil(n_b G / 256) <= M G / 256 + B tiles per kv head; max(1, floor(kt / chunk)) parts per
    // tile add at most kPrefillTarget units
    s.tasks_bound = size_t(nkv) * ((size_t(num_tokens) * G) / kPrefillRows + size_t(num_seqs));
    s.units_bound = s.tasks_bound + kPrefillTarget;
  }
  return s;
}

}  // namespace

size_t ragged_scratch_floats(int num_seqs, int num_tokens, int max_tokens_per_seq, int nq, int nkv, int max_splits) {
  const RaggedShape s = ragged_shape(num_seqs, num_tokens, max_tokens_per_seq, nq, nkv, max_splits);
  return size_t(kHeaderInts) + kClaimFloats + s.decode_floats + s.units_bound * kPrefillRows * kPartialRowFloats;
}

namespace {
// Zeroes the counter region (header + claim lines) of a ragged scratch buffer: a plain fill kernel,
// so the call is also safe inside graph capture.
__global__ void __launch_bounds__(256) ragged_counters_zero_kernel(int* p, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) p[i] = 0;
}
}  // namespace

int ragged_scratch_init(float* scratch, hipStream_t stream) {
  const size_t n = size_t(kHeaderInts) + kClaimFloats;
  hipLaunchKernelGGL(ragged_counters_zero_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<int*>(scratch), n);
  return check_hip(hipGetLastError(), "ragged_scratch_init launch");
}

int launch_attention_ragged(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream) {
  if (b.num_seqs == 0 || b.num_tokens == 0) return Q38A_OK;
  if (b.num_seqs >= kMaxSeqs) return set_error(Q38A_ERR_INVALID, "attention_ragged: at most %d sequences", kMaxSeqs - 1);
  if (p.max_splits > kMaxMergeSplits)
    return set_error(Q38A_ERR_INVALID, "attention_ragged: max_splits %d exceeds %d", p.max_splits, kMaxMergeSplits);
  const int G = p.num_q_heads / p.num_kv_heads;
  const RaggedShape s = ragged_shape(b.num_seqs, b.num_tokens, b.max_tokens_per_seq, p.num_q_heads, p.num_kv_heads,
                                     p.max_splits);
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  // one eight-wave decode workgroup per CU, two items each (one item per workgroup: 54 vs 49 us for
  // config 4's decode rows alone; three: 55)
  // With prefill chunks in the batch, cus / 8 decode workgroups (4 per XCD) come first and stream
  // the decode rows' pages beside the MFMA-bound prefill units, which aim at the other CUs; the rest
  // follow the prefill units and join the item queue as CUs free up. Config 4: 187 -> 174 us (16,
  // 24, 40 and 48 first: 177, 176, 179, 178); a decode-heavy mix (a 128-token chunk + 15 rows of
  // 30-44K): 261 -> 250 us.
  const int dfirst = b.max_tokens_per_seq > 1 ? cus / 8 : 0;
  const int dgrid = cus, target = 2 * dgrid;
  int* header = reinterpret_cast<int*>(p.split_scratch);
  int* claims = header + kHeaderInts;
  float* dec = p.split_scratch + kHeaderInts + kClaimFloats;
  float* pre = dec + s.decode_floats;
  const int pblocks = int(s.units_bound);
  RaggedArgs r{pblocks, dfirst, min(kPrefillTarget, cus - dfirst), header, pre};
  DecodeArgs d{p.q, p.num_q_heads, p.num_kv_heads, G, p.attn_layer, dec, p.max_splits, target, p.gate, p.ld_gate,
               p.out, true, true, claims, header + kQueue};
  PrefillArgs pa{p.q, p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, G, p.attn_layer};
  const dim3 grid(unsigned(pblocks + dgrid));
  if (kv.dtype == Q38A_KV_INT8)
    hipLaunchKernelGGL(attn_ragged_kernel<Q38A_KV_INT8>, grid, dim3(kRaggedThreads), 0, stream, r, d, pa, to_args(b),
                       to_args(kv));
  else if (kv.dtype == Q38A_KV_INT8_VT)
    hipLaunchKernelGGL(attn_ragged_kernel<Q38A_KV_INT8_VT>, grid, dim3(kRaggedThreads), 0, stream, r, d, pa, to_args(b),
                       to_args(kv));
  else
    hipLaunchKernelGGL(attn_ragged_kernel<Q38A_KV_BF16>, grid, dim3(kRaggedThreads), 0, stream, r, d, pa, to_args(b),
                       to_args(kv));
  if (int rc = check_hip(hipGetLastError(), "attention_ragged launch")) return rc;
  RaggedMergeArgs m{p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, G, header, dec, pre, p.max_splits,
                    header + kQueue, claims};
  const size_t mblocks = size_t(b.num_seqs) * p.num_q_heads + s.tasks_bound * (kPrefillRows / kMergeWaves);
  hipLaunchKernelGGL(attn_ragged_merge_kernel, dim3(unsigned(mblocks)), dim3(kMergeThreads), 0, stream, m,
                     to_args(b));
  return check_hip(hipGetLastError(), "attention_ragged merge launch");
}

}  // namespace q38a
