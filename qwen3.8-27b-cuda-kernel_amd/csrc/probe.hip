// Measurement probes: the MFMA issue rate and the HBM read rate this GPU actually reaches, so that
// roofline fractions can be stated against measured ceilings as well as the published peaks.
//   * mfma probe: every wave runs a loop of independent v_mfma_f32_32x32x16_f16 chains on register
//     operands (no memory traffic), one workgroup of four waves per SIMD quad, several per CU;
//   * read probe: a grid-stride sum over a device buffer with 16-byte loads (one float written per
//     workgroup, so the reads cannot be dropped).
#include "common.hpp"

#include "q38a_probe.h"

namespace q38a {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kChains = 8;  // independent accumulators per wave: enough to cover the MFMA latency

__global__ void __launch_bounds__(kProbeThreads) mfma_probe_kernel(float* sink, int iters, float seed) {
  half8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = _Float16(seed * float(threadIdx.x + i));
    b[i] = _Float16(seed * float(i - int(threadIdx.x)));
  }
  float16_t acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = float16_t{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[c][e];
  if (s == 12345.678f) sink[blockIdx.x] = s;  // practically never: keeps the loop live
}

// Each workgroup reads whole 32 KiB chunks (eight 16-byte loads in flight per lane, streamed past
// the caches), chunks handed out grid-stride.
constexpr int kChunkLoads = 8;
constexpr size_t kChunk16 = size_t(kProbeThreads) * kChunkLoads;  // 16-byte words per chunk

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const u32x4_t* src, size_t n16, float* sink) {
  uint32_t x = 0;
  const size_t chunks = n16 / kChunk16;
  for (size_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const u32x4_t* p = src + c * kChunk16 + threadIdx.x;
    u32x4_t v[kChunkLoads];
#pragma unroll
    for (int u = 0; u < kChunkLoads; ++u) v[u] = __builtin_nontemporal_load(p + kProbeThreads * u);
#pragma unroll
    for (int u = 0; u < kChunkLoads; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (size_t i = chunks * kChunk16 + size_t(blockIdx.x) * kProbeThreads + threadIdx.x; i < n16;
       i += size_t(gridDim.x) * kProbeThreads)
    x ^= src[i].x;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x |= __shfl_xor(x, off, 64);
  if (threadIdx.x == 0) sink[blockIdx.x] = float(x & 1u);
}

}  // namespace
}  // namespace q38a

using namespace q38a;

extern "C" {

int q38a_probe_mfma(float* sink, int iters, void* stream, double* flops) {
  clear_error();
  if (!sink || iters <= 0 || !flops) return set_error(Q38A_ERR_INVALID, "probe_mfma: bad arguments");
  int cus = 0;
  if (int rc = device_cu_count(&cus)) return rc;
  const int blocks = cus * 2;  // two four-wave workgroups per CU: two waves per SIMD
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream), sink,
                     iters, 1e-3f);
  *flops = double(blocks) * (kProbeThreads / 64) * double(iters) * kChains * (32.0 * 32.0 * 16.0 * 2.0);
  return check_hip(hipGetLastError(), "probe_mfma launch");
}

int q38a_probe_read(const void* buf, size_t bytes, float* sink, int sink_len, void* stream) {
  clear_error();
  if (!buf || !sink || bytes % 16 || sink_len <= 0) return set_error(Q38A_ERR_INVALID, "probe_read: bad arguments");
  hipLaunchKernelGGL(read_probe_kernel, dim3(unsigned(sink_len)), dim3(kProbeThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4_t*>(buf), bytes / 16, sink);
  return check_hip(hipGetLastError(), "probe_read launch");
}

}  // extern "C"
