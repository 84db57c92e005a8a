// Prefill launch (q38a_attention_prefill): one eight-wave workgroup per (row tile of 256 rows,
// kv head, sequence), each tile over all of its keys; the device code is in prefill.hpp.
#include "prefill.hpp"

namespace q38a {
namespace {

// grid (tiles_x * nkv, B): block x = (tile from last to first, kv head), so the longest rows start
// first and the kv heads of one row tile are dispatched together. One workgroup per CU (LDS).
template <int DT>
__global__ void __launch_bounds__(kPThreads, 1) attn_prefill_kernel(PrefillArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ KvTileFor<DT> tiles[2];
  __shared__ std::conditional_t<kQHalfInLds<DT>, QHalfLds, char> qh;
  const int tiles_x = int(gridDim.x) / a.nkv;
  const int tile = tiles_x - 1 - int(blockIdx.x) / a.nkv, kvh = int(blockIdx.x) % a.nkv;
  QHalfLds* qp = nullptr;
  if constexpr (kQHalfInLds<DT>) qp = &qh;
  prefill_unit<DT>(a, batch, kv, tiles, blockIdx.y, kvh, tile, 0, 1, nullptr, qp);
}

}  // namespace

// Only eight-wave workgroups: the four-wave form (two per CU, or one per CU for launches with fewer
// 128-row tiles than CUs) was dropped with the exact-code K path, whose extra registers it has no
// room for at two per CU, and which at one per CU ran a 300-token chunk at 0.39 ms against 0.36 ms
// for the eight-wave form.
int launch_attention_prefill(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                             hipStream_t stream) {
  if (b.num_seqs == 0 || b.num_tokens == 0) return Q38A_OK;
  const int G = p.num_q_heads / p.num_kv_heads;
  const int tiles_x = int((size_t(b.max_tokens_per_seq) * G + kRowsPerTile - 1) / kRowsPerTile);
  PrefillArgs a{p.q, p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, G, p.attn_layer};
  const dim3 grid(tiles_x * p.num_kv_heads, b.num_seqs), block(kPThreads);
  switch (kv.dtype) {
    case Q38A_KV_INT8: hipLaunchKernelGGL(attn_prefill_kernel<Q38A_KV_INT8>, grid, block, 0, stream, a, to_args(b), to_args(kv)); break;
    case Q38A_KV_INT8_VT: hipLaunchKernelGGL(attn_prefill_kernel<Q38A_KV_INT8_VT>, grid, block, 0, stream, a, to_args(b), to_args(kv)); break;
    default: hipLaunchKernelGGL(attn_prefill_kernel<Q38A_KV_BF16>, grid, block, 0, stream, a, to_args(b), to_args(kv)); break;
  }
  return check_hip(hipGetLastError(), "attention_prefill launch");
}

}  // namespace q38a
