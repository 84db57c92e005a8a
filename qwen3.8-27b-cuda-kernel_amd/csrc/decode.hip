// Split-KV decode launch (q38a_attention_decode) and its gated split merge; the device code is in
// decode.hpp.
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
  if (L == 0) return;
  const int row = batch.seq_start[b];
  const DecodePlan pl = wave_decode_plan(batch, a.nkv, a.max_splits, a.target_items);
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

int launch_attention_decode(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                            hipStream_t stream) {
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
  else
    hipLaunchKernelGGL(attn_decode_kernel<Q38A_KV_BF16>, dim3(grid), dim3(kThreads), 0, stream, a, to_args(b),
                       to_args(kv));
  if (int rc = check_hip(hipGetLastError(), "attention_decode launch")) return rc;
  MergeArgs m{p.gate,          p.ld_gate,       p.out,       p.num_q_heads, p.num_kv_heads,
              p.num_q_heads / p.num_kv_heads, p.split_scratch, p.max_splits, target};
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.num_q_heads, b.num_seqs), dim3(kMergeThreads), 0, stream, m,
                     to_args(b));
  return check_hip(hipGetLastError(), "attention merge launch");
}

}  // namespace q38a
