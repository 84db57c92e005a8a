// Prefill launch (q38a_attention_prefill): one workgroup per (row tile, kv head, sequence), each
// tile over all of its keys; the device code is in prefill.hpp.
#include "prefill.hpp"

namespace q38a {
namespace {

// grid (tiles_x * nkv, B): block x = (tile from last to first, kv head), so the longest rows start
// first and the kv heads of one row tile are dispatched together
template <int DT>
__global__ void __launch_bounds__(kPThreads, 2) attn_prefill_kernel(PrefillArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ KvTileFor<4, DT> tiles[2];
  const int tiles_x = int(gridDim.x) / a.nkv;
  const int tile = tiles_x - 1 - int(blockIdx.x) / a.nkv, kvh = int(blockIdx.x) % a.nkv;
  prefill_unit<DT, DT == Q38A_KV_INT8>(a, batch, kv, tiles, blockIdx.y, kvh, tile, 0, 1, nullptr);
}

// Eight-wave workgroups of 256 rows, one per CU (grid as above). Each dequantised key
// tile serves twice the rows, so a thread stages half the codes (and holds half the registers
// for them) of the four-wave kernel.
template <int DT>
__global__ void __launch_bounds__(2 * kPThreads, 1) attn_prefill8_kernel(PrefillArgs a, BatchArgs batch, KvArgs kv) {
  __shared__ KvTileFor<8, DT> tiles[2];
  const int tiles_x = int(gridDim.x) / a.nkv;
  const int tile = tiles_x - 1 - int(blockIdx.x) / a.nkv, kvh = int(blockIdx.x) % a.nkv;
  prefill_unit<DT, true, 8>(a, batch, kv, tiles, blockIdx.y, kvh, tile, 0, 1, nullptr);
}

}  // namespace

int launch_attention_prefill(const q38a_attention_params& p, const q38a_batch_desc& b, const q38a_kv_cache_desc& kv,
                             hipStream_t stream) {
  if (b.num_seqs == 0 || b.num_tokens == 0) return Q38A_OK;
  const int G = p.num_q_heads / p.num_kv_heads;
  const int tiles_x = int((size_t(b.max_tokens_per_seq) * G + kRowsPerTile - 1) / kRowsPerTile);
  PrefillArgs a{p.q, p.gate, p.ld_gate, p.out, p.num_q_heads, p.num_kv_heads, G, p.attn_layer};
  // 256-row workgroups (one per CU) once the 128-row ones would share CUs (two fit on one); with
  // fewer, the 128-row ones run one per CU and finish sooner
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  const long long units = (static_cast<long long>(b.num_tokens) * G + kRowsPerTile - 1) / kRowsPerTile * p.num_kv_heads;
  // bf16 and int8 VT pages always: the bf16 four-wave form spills (it measured 1.4-1.7x slower at
  // every size); the VT staging is written for 512 threads (two per dim)
  const bool wide = units > cus || kv.dtype != Q38A_KV_INT8;
  const int tiles8 = int((size_t(b.max_tokens_per_seq) * G + 2 * kRowsPerTile - 1) / (2 * kRowsPerTile));
  const dim3 grid8(tiles8 * p.num_kv_heads, b.num_seqs), grid4(tiles_x * p.num_kv_heads, b.num_seqs);
  if (kv.dtype == Q38A_KV_INT8 && wide)
    hipLaunchKernelGGL(attn_prefill8_kernel<Q38A_KV_INT8>, grid8, dim3(2 * kPThreads), 0, stream, a, to_args(b), to_args(kv));
  else if (kv.dtype == Q38A_KV_INT8)
    hipLaunchKernelGGL(attn_prefill_kernel<Q38A_KV_INT8>, grid4, dim3(kPThreads), 0, stream, a, to_args(b), to_args(kv));
  else if (kv.dtype == Q38A_KV_INT8_VT)
    hipLaunchKernelGGL(attn_prefill8_kernel<Q38A_KV_INT8_VT>, grid8, dim3(2 * kPThreads), 0, stream, a, to_args(b), to_args(kv));
  else
    hipLaunchKernelGGL(attn_prefill8_kernel<Q38A_KV_BF16>, grid8, dim3(2 * kPThreads), 0, stream, a, to_args(b), to_args(kv));
  return check_hip(hipGetLastError(), "attention_prefill launch");
}

}  // namespace q38a
