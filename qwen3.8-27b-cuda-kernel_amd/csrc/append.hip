// Fused q/k offset-RMSNorm + partial RoPE + KV append for gfx950.
//
// Behaviour follows the reference kernel src/kernels/qk_norm_rope.cu:12-90 and, to the last bit,
// its CPU twin src/ref/ops.cpp:79-142:
//   y = x * r * w with r = 1 / sqrt(float(sum_sq / 256) + eps), sum_sq accumulated in double;
//   RoPE on dims [0, 64): (y_i, y_{i+32}) <- (y_i c - y_{i+32} s, y_{i+32} c + y_i s);
//   q -> fp16 (RNE); k (normed + rotated) and v (as projected) -> page row: int8 with one fp16
//   scale = fp16(amax / 127) per 64-dim group and codes clamp(rint(y / scale), -127, 127), or bf16.
//
// Work mapping (MI355X-first): one wave64 per (token, head row); rows are the nq q heads, then the
// nkv k heads, then the nkv v heads of a token. Lane l owns dims [4l, 4l + 4), so a 64-dim
// quantisation group is exactly 16 lanes (one DPP row) and RoPE partners (i, i + 32) sit 8 lanes
// apart. Contraction is off for the whole file and division / square root are correctly rounded, so
// every operation rounds exactly as the reference's IEEE single-precision code does. cos/sin come
// from a host-built table (same libm calls as the CPU reference), read per position.
//
// Sum of squares: the reference sums x_i^2 in double, left to right. x is bf16, so every x_i^2 is
// exact in double; the sum is exact in any order whenever the total and the lowest set bit of the
// squares fit in 53 bits. The kernel checks that (a wave reduction) and then uses a tree reduction;
// otherwise one lane replays the left-to-right double sum from LDS.
#include "append.hpp"

// (append.hpp turns multiply-add contraction off for the whole file.)

namespace q38a {
namespace {

// kRows consecutive jobs (token-major rows) per wave: with one row per wave, a large launch is a
// sequence of rounds of resident waves, each waiting out its own dependent-load chain.
template <int kRows>
__global__ void __launch_bounds__(kWavesPerBlock * 64)
qk_norm_rope_append_kernel(AppendArgs p, BatchArgs batch, KvArgs kv, int jobs) {
  __shared__ double stage[kWavesPerBlock][kHeadDim];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int job0 = (blockIdx.x * kWavesPerBlock + wave) * kRows;
  if (job0 >= jobs) return;
  const int rows = p.nq + 2 * p.nkv;
  RowLoads L[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int job = min(job0 + j, jobs - 1);
    L[j].m = job / rows;
    L[j].r = job % rows;
    const bool is_q = L[j].r < p.nq;
    // q head r at column r*256; k head h at (2nq + h)*256; v head h at (2nq + nkv + h)*256
    const int col = (is_q ? L[j].r : p.nq + L[j].r) * kHeadDim;
    L[j].pos = batch.tok_pos[L[j].m];
    L[j].raw = *reinterpret_cast<const uint2*>(p.proj + size_t(L[j].m) * p.ld_proj + col + 4 * lane);
  }
#pragma unroll
  for (int j = 0; j < kRows; ++j) row_meta(p, batch, kv, lane, L[j]);
#pragma unroll
  for (int j = 0; j < kRows; ++j)
    if (job0 + j < jobs) append_row(p, kv, stage[wave], lane, L[j]);
}

}  // namespace

int launch_qk_norm_rope_append(const q38a_qk_norm_rope_params& p, const q38a_batch_desc& b,
                               const q38a_kv_cache_desc& kv, hipStream_t stream) {
  if (b.num_tokens == 0) return Q38A_OK;
  const int rows = p.num_q_heads + 2 * p.num_kv_heads;
  const long long jobs = (long long)b.num_tokens * rows;
  if (jobs > (1ll << 30)) return set_error(Q38A_ERR_INVALID, "qk_norm_rope_append: too many tokens (%d)", b.num_tokens);
  AppendArgs a{p.proj, p.ld_proj, p.q_norm, p.k_norm, p.eps, p.num_q_heads, p.num_kv_heads, p.q_out,
               p.attn_layer, p.rope_cos_sin, p.rope_rows};
  // four rows per wave for long chunks (2,048 tokens: 49.6 -> 45.2 us; at 519 tokens it was 7% slower)
  if (jobs > 32768) {
    const int blocks = int((jobs + 4 * kWavesPerBlock - 1) / (4 * kWavesPerBlock));
    hipLaunchKernelGGL(qk_norm_rope_append_kernel<4>, dim3(blocks), dim3(kWavesPerBlock * 64), 0, stream, a,
                       to_args(b), to_args(kv), int(jobs));
  } else {
    const int blocks = int((jobs + kWavesPerBlock - 1) / kWavesPerBlock);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel<1>, dim3(blocks), dim3(kWavesPerBlock * 64), 0, stream, a,
                       to_args(b), to_args(kv), int(jobs));
  }
  return check_hip(hipGetLastError(), "qk_norm_rope_append launch");
}

}  // namespace q38a
