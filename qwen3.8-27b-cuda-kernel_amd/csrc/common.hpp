// Shared host/device definitions of the q38a library: error reporting, the paged KV byte layout,
// exact 16-bit float conversions and the MFMA operand vector types used by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "q38a.h"

namespace q38a {

constexpr int kPageTokens = Q38A_PAGE_TOKENS;
constexpr int kHeadDim = Q38A_HEAD_DIM;
constexpr int kRotaryDim = 64;  // partial RoPE over dims [0, 64): pairs (i, i + 32)

// ---- errors (host) ------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);  // records the message, returns `code`
void clear_error();
int check_hip(hipError_t e, const char* what);   // Q38A_OK or Q38A_ERR_HIP with the HIP message
int device_cu_count(int* out);                   // cached per device

// ---- paged KV layout (reference kernels.h:41-70, docs/FORMAT.md 3.1) --------------------------
// One (layer, page) block, int8:  K [kvh][64][256] i8 | V [kvh][64][256] i8 |
//                                 K scales [kvh][64][4] f16 | V scales [kvh][64][4] f16
//                         bf16:   K [kvh][64][256] bf16 | V [kvh][64][256] bf16
//                      int8 VT:   K [kvh][64][256] i8 | V^T [kvh][4][256][16] i8 (per 16-token quarter) |
//                                 K scales [kvh][64][4] f16 | V scales [kvh][4][64] f16
struct PageLayout {
  int kv_heads;
  int dtype;
  __host__ __device__ bool int8() const { return dtype != Q38A_KV_BF16; }  // int8 codes + fp16 scales
  __host__ __device__ size_t elem() const { return int8() ? 1 : 2; }
  __host__ __device__ size_t k_row(int h, int t) const {
    return (size_t(h) * kPageTokens + t) * kHeadDim * elem();
  }
  __host__ __device__ size_t v_row(int h, int t) const {
    return size_t(kv_heads) * kPageTokens * kHeadDim * elem() + k_row(h, t);
  }
  __host__ __device__ size_t k_scales(int h, int t) const {
    return 2 * size_t(kv_heads) * kPageTokens * kHeadDim + (size_t(h) * kPageTokens + t) * 8;
  }
  __host__ __device__ size_t v_scales(int h, int t) const {
    return k_scales(h, t) + size_t(kv_heads) * kPageTokens * 8;
  }
  __host__ __device__ size_t page_bytes() const {
    return int8() ? 2 * size_t(kv_heads) * kPageTokens * (kHeadDim + 8)
                  : 2 * size_t(kv_heads) * kPageTokens * kHeadDim * 2;
  }
  // int8 VT: V code of (head h, dim d, token t), and V scale of (head h, group g, token t). The
  // codes of a 16-token quarter are [dim][16 tokens], so token t + 16 is 4,096 bytes further, the
  // same stride as 16 K rows.
  __host__ __device__ size_t vt_code(int h, int d, int t) const {
    return size_t(kv_heads) * kPageTokens * kHeadDim + ((size_t(h) * 4 + t / 16) * kHeadDim + d) * 16 + t % 16;
  }
  __host__ __device__ size_t vt_scale(int h, int g, int t) const {
    return 2 * size_t(kv_heads) * kPageTokens * kHeadDim + size_t(kv_heads) * kPageTokens * 8 +
           ((size_t(h) * 4 + g) * kPageTokens + t) * 2;
  }
};

// ---- exact conversions --------------------------------------------------------------------------
__host__ __device__ inline uint32_t as_u32(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
__host__ __device__ inline float as_f32(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// IEEE binary16 from binary32, round to nearest even (subnormals kept, |f| >= 65520 -> inf): the
// hardware conversion (v_cvt_f16_f32 in the default round-to-nearest-even mode with fp16
// denormals enabled); NaN -> the canonical quiet NaN with f's sign.
__device__ inline uint16_t f16_bits(float f) {
  const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  return f != f ? uint16_t(((as_u32(f) >> 16) & 0x8000u) | 0x7e00u) : h;
}

// binary16 -> binary32, exact (v_cvt_f32_f16).
__device__ inline float f16_value(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// bfloat16 from binary32, round to nearest even; NaN -> quiet NaN.
__host__ __device__ inline uint16_t bf16_bits(float f) {
  const uint32_t u = as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__host__ __device__ inline float bf16_value(uint16_t b) { return as_f32(uint32_t(b) << 16); }

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal (each within ~1 ulp):
// the gated outputs are rounded to bf16 (8 significand bits), so the libm-accurate forms bought
// nothing and cost ~25 instructions per element in the epilogues. g -> -inf gives 0, +inf gives 1.
__device__ inline float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * g));
}

// ---- cross-lane steps on the VALU ----------------------------------------------------------------
// DPP moves and permlane swaps instead of LDS-routed shuffles (__shfl*: one ds_bpermute, an LDS
// round trip, per step of a dependent chain). Every lane of the wave must be active.
// dpp_move<C>(x): lane i receives x of the lane that DPP control C names (all lanes valid here).
template <int C>
__device__ inline uint32_t dpp_move(uint32_t x) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), C, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within each 8
constexpr int kDppMirror = 0x140;     // lane i <- 15 - i within each 16
constexpr int kDppRor8 = 0x128;       // lane i <- (i + 8) mod 16 within each 16 (= i ^ 8)
constexpr int kDppRor4 = 0x124;       // lane i <- (i + 4) mod 16 within each 16

// op over all 64 lanes, the result in every lane (op commutative and associative). After the
// quad steps a quad holds its total; the mirrors pair quad 0 with quad 1 and the two halves of a
// 16-lane row; the swaps pair rows 0-1 / 2-3, then the two halves of the wave.
template <class Op>
__device__ inline uint32_t wave_allreduce(uint32_t x, Op op) {
  x = op(x, dpp_move<kDppXor1>(x));
  x = op(x, dpp_move<kDppXor2>(x));
  x = op(x, dpp_move<kDppHalfMirror>(x));
  x = op(x, dpp_move<kDppMirror>(x));
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = op(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return op(b[0], b[1]);
}

__device__ inline int wave_min_i32(int x) {
  return int(wave_allreduce(uint32_t(x), [](uint32_t a, uint32_t b) { return uint32_t(min(int(a), int(b))); }));
}
__device__ inline int wave_max_i32(int x) {
  return int(wave_allreduce(uint32_t(x), [](uint32_t a, uint32_t b) { return uint32_t(max(int(a), int(b))); }));
}

// Inclusive prefix sum over the 64 lanes: Hillis-Steele within each 16-lane row (row_shr 1, 2, 4,
// 8, zeros shifted in), then row 0's total into row 1 and row 2's into row 3 (row_bcast15), then
// lane 31's running total into rows 2 and 3 (row_bcast31).
__device__ inline int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
  return x;
}

// x op (x of lane l ^ 32) in every lane l
__device__ inline float xor32_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ inline float xor32_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ inline float xor16_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// ---- MFMA operand types (gfx950) ----------------------------------------------------------------
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// Kernel-side copies of the C descriptors (passed by value as kernel arguments).
struct BatchArgs {
  int num_seqs, num_tokens, max_tokens_per_seq;
  const int32_t* seq_start;
  const int32_t* seq_slot;
  const int32_t* seq_pos0;
  const int32_t* tok_pos;
  const int32_t* tok_seq;
};
struct KvArgs {
  uint8_t* pool;
  PageLayout layout;
  int num_pages;
  size_t page_bytes;
  size_t layer_stride;
  const int32_t* block_table;
  int max_pages_per_seq;
};

inline BatchArgs to_args(const q38a_batch_desc& b) {
  return BatchArgs{b.num_seqs, b.num_tokens, b.max_tokens_per_seq, b.seq_start,
                   b.seq_slot, b.seq_pos0,   b.tok_pos,            b.tok_seq};
}

inline KvArgs to_args(const q38a_kv_cache_desc& k) {
  return KvArgs{k.pool, PageLayout{k.kv_heads, k.dtype}, k.num_pages, k.page_bytes, k.layer_stride,
                k.block_table, k.max_pages_per_seq};
}

// Host-side validation shared by the launchers.
int validate_batch(const q38a_batch_desc* b, bool need_tok);
int validate_kv(const q38a_kv_cache_desc* k);

}  // namespace q38a
