// Host-side repack of BQ weights from the reference's file layout into the q38a MFMA layout.
//
// The file layout (reference docs/FORMAT.md 2.2-2.5) is built around another GPU's 32-lane
// fragments: 16 (k) x 64 (n) slabs, lane 4g + t owning columns 8j + g and rows 2t, 2t + 1, 2t + 8,
// 2t + 9. On gfx950 the B operand of v_mfma_f32_32x32x16_bf16 wants, per lane, eight consecutive k
// of one column, so each weight is decoded once here (position by position, following the format
// spec) and stored as described in include/q38a_gemm.h: per 32-column block and 64-k group, one
// 16-byte word of low nibbles per lane (plus the high bits), so a wave loads a block's group as
// 1 KB of contiguous low-nibble data.
#include <cstring>
#include <vector>

#include "common.hpp"
#include "q38a_gemm.h"

namespace q38a {
namespace {

uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}

// Stored (unsigned) code of W[n][k] in the file layout (FORMAT.md 2.2-2.4).
unsigned file_code(int bits, int K, const uint8_t* lo, const uint8_t* hi, int n, int k) {
  const int nb = n / 64, kb = k / 16, nl = n % 64, kl = k % 16;
  const int j = nl / 8, gl = nl % 8, h = kl / 8, t = (kl % 8) / 2, e = kl % 2;
  const size_t slab = size_t(nb) * (K / 16) + kb;
  const int lane = 4 * gl + t, pair = 2 * j + h;
  const uint32_t w = rd32(lo + slab * 512 + lane * 16 + 4 * (pair >> 2));
  unsigned u = (w >> (e ? 16 + 4 * (pair & 3) : 4 * (pair & 3))) & 15u;
  if (bits == 5) {
    const uint32_t hw = rd32(hi + slab * 128 + lane * 4);
    u |= ((hw >> (e ? 16 + pair : pair)) & 1u) << 4;
  } else if (bits == 6) {
    const uint32_t hw = rd32(hi + slab * 256 + lane * 8 + 4 * (pair >> 3));
    const int r = pair & 7;
    u |= ((hw >> (e ? 16 + 2 * r : 2 * r)) & 3u) << 4;
  }
  return u;
}

// bf16 scale bits of (row n, group g) in the file layout (FORMAT.md 2.5).
uint16_t file_scale(int K, const uint16_t* scales, int n, int g) {
  const int nb = n / 64, nl = n % 64;
  return scales[(size_t(nb) * (K / 64) + g) * 64 + (nl % 8) * 8 + nl / 8];
}

size_t hi_lane_bytes(int bits) { return bits == 4 ? 0 : bits == 5 ? 4 : 8; }

}  // namespace
}  // namespace q38a

using namespace q38a;

extern "C" {

int q38a_bq_repacked_bytes(int bits, int n, int k, size_t out[3]) {
  clear_error();
  if (!out || (bits != 4 && bits != 5 && bits != 6) || n <= 0 || k <= 0 || n % 32 || k % 64)
    return set_error(Q38A_ERR_INVALID, "bq_repacked_bytes: bits 4/5/6, n % 32 == 0, k % 64 == 0");
  const size_t units = size_t(n / 32) * size_t(k / 64) * 64;  // (block, group, lane)
  out[0] = units * 16;
  out[1] = units * hi_lane_bytes(bits);
  out[2] = size_t(n / 32) * size_t(k / 64) * 32 * 2;
  return Q38A_OK;
}

int q38a_bq_repack(int bits, int n, int k, const uint8_t* ref_lo, const uint8_t* ref_hi, const uint16_t* ref_scales,
                   uint8_t* lo, uint8_t* hi, uint16_t* scales) {
  clear_error();
  if (bits == 8) return set_error(Q38A_ERR_UNSUPPORTED, "bq_repack: 8-bit weights are not supported");
  if ((bits != 4 && bits != 5 && bits != 6) || n <= 0 || k <= 0 || n % 64 || k % 64)
    return set_error(Q38A_ERR_INVALID, "bq_repack: bits 4/5/6, n % 64 == 0, k % 64 == 0");
  if (!ref_lo || !ref_scales || !lo || !scales || (bits > 4 && (!ref_hi || !hi)))
    return set_error(Q38A_ERR_INVALID, "bq_repack: null plane");
  const int G = k / 64;
  const size_t hb = hi_lane_bytes(bits);
  for (int nb = 0; nb < n / 32; ++nb)
    for (int g = 0; g < G; ++g) {
      const size_t unit = size_t(nb) * G + g;
      for (int l = 0; l < 64; ++l) {
        const int col = 32 * nb + (l & 31), kg = l >> 5;
        uint32_t wlo[4] = {0, 0, 0, 0}, whi[2] = {0, 0};
        for (int s = 0; s < 4; ++s)
          for (int i = 0; i < 8; ++i) {
            const unsigned u = file_code(bits, k, ref_lo, ref_hi, col, 64 * g + 16 * s + 8 * kg + i);
            const int p = i / 2, e = i % 2, q = 4 * s + p;
            wlo[s] |= uint32_t(u & 15u) << (e ? 16 + 4 * p : 4 * p);
            if (bits == 5) whi[0] |= uint32_t((u >> 4) & 1u) << (e ? 16 + q : q);
            if (bits == 6) whi[q >> 3] |= uint32_t((u >> 4) & 3u) << (e ? 16 + 2 * (q & 7) : 2 * (q & 7));
          }
        std::memcpy(lo + (unit * 64 + l) * 16, wlo, 16);
        if (hb) std::memcpy(hi + (unit * 64 + l) * hb, whi, hb);
      }
      for (int c = 0; c < 32; ++c) scales[unit * 32 + c] = file_scale(k, ref_scales, 32 * nb + c, g);
    }
  return Q38A_OK;
}

}  // extern "C"
