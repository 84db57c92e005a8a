// Split-KV decode launch (q38a_attention_decode) and its gated split merge; the device code is in
// decode.hpp.
#include <mutex>
#include <vector>

#include "decode.hpp"

namespace q38a {

int max_group() { return kMaxGroup; }

namespace {

// The launch keeps no state between launches: the merge recomputes the decode plan (pages per item)
// from the same metadata, so concurrent launches on different streams with their own scratch are
// independent.
template <int DT>
__global__ void __launch_bounds__(kThreads, 2) attn_decode_kernel(DecodeArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ DecodeShared<> sh;
  const DecodePlan pl = wave_decode_plan(batch, a.nkv, a.max_splits, a.target_items);
  decode_items<DT>(a, batch, kv, pl, sh, blockIdx.x, gridDim.x);
}

struct MergeArgs {
  const uint16_t* gate;
  int ld_gate;
  uint16_t* out;
  int nq, nkv, group;
  const float* scratch;
  int max_splits;
  int target_items;  // the decode launch's plan target: the split count follows from it
};

// grid (nq, B): combine the item partials of (decode row b, q head); the split count follows from
// the decode plan, recomputed here from the launch's metadata exactly as the decode kernel made it.
__global__ void __launch_bounds__(kMergeThreads) attn_merge_kernel(MergeArgs a, BatchArgs batch) {
  __shared__ MergeShared sh;
  const int hq = blockIdx.x, b = blockIdx.y;
  const int L = decode_len(batch, b);
  const int row = batch.seq_start[b];
  const DecodePlan pl = wave_decode_plan(batch, a.nkv, a.max_splits, a.target_items);
  if (L == 0) return;
  const int splits = ceil_div_i(ceil_div_i(L, kPageTokens), pl.cp);
  const float* src = a.scratch + (size_t(b) * a.nq + hq) * a.max_splits * (kHeadDim + 2);
  merge_row_wg(src, splits, kHeadDim + 2, a.gate + size_t(row) * a.ld_gate + hq * kHeadDim,
               a.out + (size_t(row) * a.nq + hq) * kHeadDim, sh);
}

constexpr int kBlocksPerCu = 2;
constexpr int kItemsPerBlock = 1;

}  // namespace

// Decode grid: a persistent grid of kBlocksPerCu workgroups per CU; the plan targets one item each.
int decode_grid(int* grid, int* target_items) {
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  *grid = cus * kBlocksPerCu;
  *target_items = *grid * kItemsPerBlock;
  return Q38A_OK;
}

// The split kernel alone: partials into p.split_scratch (p.out untouched).
int launch_attention_decode_partials(const q38a_attention_params& p, const q38a_batch_desc& b,
                                     const q38a_kv_cache_desc& kv, hipStream_t stream) {
  if (b.num_seqs == 0) return Q38A_OK;
  if (b.num_seqs >= kMaxSeqs) return set_error(Q38A_ERR_INVALID, "attention_decode: at most %d sequences", kMaxSeqs - 1);
  if (p.max_splits > kMaxMergeSplits)
    return set_error(Q38A_ERR_INVALID, "attention_decode: max_splits %d exceeds %d", p.max_splits, kMaxMergeSplits);
  int grid = 0, target = 0;
  if (int rc = decode_grid(&grid, &target)) return rc;
  DecodeArgs a{p.q, p.num_q_heads, p.num_kv_heads, p.num_q_heads / p.num_kv_heads, p.attn_layer,
               p.split_scratch, p.max_splits, target, p.gate, p.ld_gate, p.out, false};
  if (kv.dtype == Q38A_KV_INT8)
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_INT8>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  else if (kv.dtype == Q38A_KV_INT8_VT)
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_INT8_VT>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  else
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_BF16>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  return check_hip(hipGetLastError(), "attention_decode launch");
}

// The gated split merge of a launch_attention_decode_partials into p.out.
int launch_attention_merge(const q38a_attention_params& p, const q38a_batch_desc& b, hipStream_t stream) {
  if (b.num_seqs == 0) return Q38A_OK;
  int grid = 0, target = 0;
  if (int rc = decode_grid(&grid, &target)) return rc;
  MergeArgs m{p.gate,          p.ld_gate,       p.out,       p.num_q_heads, p.num_kv_heads,
              p.num_q_heads / p.num_kv_heads, p.split_scratch, p.max_splits, target};
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.num_q_heads, b.num_seqs), dim3(kMergeThreads), 0, stream, m,
                     to_args(b));
  return check_hip(hipGetLastError(), "attention merge launch");
}

int launch_attention_decode(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream) {
  if (int rc = launch_attention_decode_partials(p, b, kv, stream)) return rc;
  return launch_attention_merge(p, b, stream);
}

// ---- decode without caller scratch --------------------------------------------------------------
// For callers that cannot allocate (code under graph capture, tight serving loops): the split
// partials go to a file-scope device array instead of p.split_scratch. Each GPU holds its own copy
// for the life of the process; every call on a GPU shares it, so calls that overlap in time on one
// GPU race (the decode partials need no clearing: the merge reads only splits the decode kernel of
// the same call wrote).
constexpr size_t kNoAllocScratchFloats = size_t(8) << 20;  // 32 MiB per GPU
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {

// Device address of `scratch` on the current device, looked up once per device (the array's name
// is a host-side stand-in: only this address may be passed to kernels).
int noalloc_scratch(float** out) {
  static std::mutex mu;
  static std::vector<float*> ptrs;
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "attention_decode_noalloc: hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lock(mu);
  if (int(ptrs.size()) <= dev) ptrs.resize(size_t(dev) + 1, nullptr);
  if (!ptrs[size_t(dev)]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "attention_decode_noalloc: hipGetSymbolAddress"))
      return rc;
    ptrs[size_t(dev)] = static_cast<float*>(p);
  }
  *out = ptrs[size_t(dev)];
  return Q38A_OK;
}

}  // namespace

size_t noalloc_scratch_floats() { return kNoAllocScratchFloats; }

int launch_attention_decode_noalloc(const q38a_attention_params& p, const q38a_batch_desc& b,
                                    const q38a_kv_cache_desc& kv, hipStream_t stream) {
  const size_t need = size_t(b.num_seqs) * size_t(p.num_q_heads) * size_t(p.max_splits) * (kHeadDim + 2);
  if (need > kNoAllocScratchFloats)
    return set_error(Q38A_ERR_INVALID,
                     "attention_decode_noalloc: %d rows x %d q heads x %d splits need %zu scratch floats; the "
                     "static scratch holds %zu",
                     b.num_seqs, p.num_q_heads, p.max_splits, need, kNoAllocScratchFloats);
  q38a_attention_params q = p;
  if (int rc = noalloc_scratch(&q.split_scratch)) return rc;
  return launch_attention_decode(q, b, kv, stream);
}

}  // namespace q38a
