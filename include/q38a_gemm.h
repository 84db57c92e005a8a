/*
 * q38a GEMMs on either side of the attention path: the in-projection that produces `proj`, with
 * the q/k RMSNorm + RoPE + KV append optionally fused into its epilogue, and the o-projection
 * that consumes the attention output, with the decode split merge optionally fused into its A
 * loader. Weights are the reference's BQ format (docs/FORMAT.md section 2: b-bit codes in 64-wide
 * groups along K with one bf16 scale per (row, group)), repacked once at load time into this
 * library's MFMA layout (q38a_bq_repack). Same conventions as q38a.h: device pointers, asynchronous
 * on `stream`, no allocation, int status + q38a_last_error().
 */
#ifndef Q38A_GEMM_H
#define Q38A_GEMM_H

#include <stddef.h>
#include <stdint.h>

#include "q38a.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A BQ weight W[n][k] (n output features, k inputs) in the q38a MFMA layout. Mirrors reference
 * kernels.h:82-90 BQWeight (same fields; the planes are the repacked ones). bits: 4, 5 or 6;
 * n a multiple of 32, k a multiple of 64. Layout (32-column blocks nb, 64-k groups g, lanes l of a
 * wave: column 32 nb + l % 32, k 64 g + 16 s + 8 (l / 32) + i for steps s < 4 and i < 8):
 *   lo     [n/32][k/64][64 lanes][16 B]: word s, nibbles (i = 2p, 2p+1) at bits 4p and 16 + 4p;
 *   hi     [n/32][k/64][64 lanes][4 B] (bits 5: pair q = 4s + p, bit q and bit 16 + q) or
 *          [8 B] (bits 6: word q / 8, bits 2 (q % 8) and 16 + 2 (q % 8)); absent for bits 4;
 *   scales [n/32][k/64][32] bf16. Stored code u = c + 2^(bits-1). */
typedef struct q38a_bq_weight {
  const uint8_t* lo;
  const uint8_t* hi;
  const uint16_t* scales;
  int bits;
  int n;    /* rows (output features) */
  int k;    /* columns (inputs) */
  int rows; /* logical rows (<= n); columns of C beyond it are not stored */
} q38a_bq_weight;

/* Bytes of the three repacked planes of an n x k weight: out[0] lo, out[1] hi, out[2] scales. */
int q38a_bq_repacked_bytes(int bits, int n, int k, size_t out[3]);

/* Host-side repack of a weight from the reference file planes (docs/FORMAT.md 2.2-2.5: 16 x 64
 * slabs of 32 lanes, lo / hi planes, scales in 64-column blocks) into the q38a layout. All
 * pointers are host memory; ref_hi is null for bits 4. n must be a multiple of 64 (the file's
 * slab width), k of 64. Bits 8 (the format's lm_head width) is not supported. */
int q38a_bq_repack(int bits, int n, int k, const uint8_t* ref_lo, const uint8_t* ref_hi, const uint16_t* ref_scales,
                   uint8_t* lo, uint8_t* hi, uint16_t* scales);

/* Epilogues (reference kernels.h:75-80 Epilogue; SwiGLU is not on this path). */
enum { Q38A_EPI_STORE_BF16 = 0, Q38A_EPI_RESIDUAL = 2, Q38A_EPI_STORE_F32 = 3 };

/* Mirrors reference kernels.h:92-104 GemmEpilogue. */
typedef struct q38a_gemm_epilogue {
  int kind;
  void* out;            /* bf16 (STORE_BF16) or float (STORE_F32), row stride ldo elements */
  int ldo;
  int n_store;          /* columns of C to store (0 = w.rows) */
  float* residual;      /* RESIDUAL: [M][n] fp32, += C */
  uint16_t* xbf;        /* RESIDUAL: [M][n] bf16(residual) */
  float* partials_out;  /* RESIDUAL: [M][n / 128] sums of squares of the new residual */
  /* Row scale of a folded RMSNorm (STORE_*): rs = 1 / sqrt(sum(partials_in[row][0 .. hidden/128))
   * / hidden + eps); null = 1. */
  const float* partials_in;
  int hidden;
  float eps;
} q38a_gemm_epilogue;

/* Split-K workspace (reference kernels.h:106-111 GemmWorkspace): partial tiles and per-tile
 * arrival counters. Counters must be zero before first use; every launch leaves them zero. */
typedef struct q38a_gemm_workspace {
  float* partials;
  size_t partial_floats;
  int* counters;
  int num_counters;
} q38a_gemm_workspace;

/* C[M][N] = A[M][K] . W^T with A bf16 [M][K] (row stride K), fp32 accumulation, then the epilogue.
 * Replaces reference kernels.h:120-121 qgemm (src/kernels/qgemm.cu:573-616). Small M splits K over
 * several workgroups (deterministic reduction through `ws`). */
int q38a_qgemm(const uint16_t* a, int m, const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
               const q38a_gemm_workspace* ws, void* stream);

/* The attention layers' in-projection (reference model_runner.cpp:316-338: qgemm with the
 * StoreBF16 epilogue into proj, then qk_norm_rope_append) in one launch: W is the [q | gate | k | v]
 * weight (nq + nq + 2 nkv heads of 256 rows), ep a STORE_BF16 epilogue whose out is proj. The
 * epilogue stores the gate columns into proj (what attention reads) and runs the fused
 * norm / RoPE / append on the q, k and v tiles straight from LDS: q goes to append->q_out, k and v to
 * the cache; the q, k and v columns of proj are not written. When m is large enough for the
 * 256 x 256-tile GEMM to fill the GPU (2,048 rows of the in-projection), the call instead runs that
 * GEMM into proj (every column) and then the append launch, which is faster there. Either way the
 * results are bit-identical to q38a_qgemm followed by q38a_qk_norm_rope_append (append->proj and
 * ld_proj must describe ep->out).
 * No counterpart in the reference (SURVEY: the producer side of the attention path). */
int q38a_qgemm_qkv_append(const uint16_t* a, int m, const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
                          const q38a_gemm_workspace* ws, const q38a_qk_norm_rope_params* append,
                          const q38a_batch_desc* batch, const q38a_kv_cache_desc* kv, void* stream);

/* The attention layers' o-projection after split-KV decode (unfused reference: the decode merge into
 * attn->out, then qgemm on it, model_runner.cpp:351-357): attn and batch are those of the preceding
 * q38a_attention_decode_partials (same split scratch, same batch); runs the gated merge kernel into
 * attn->out, then q38a_qgemm with A = attn->out. w->k must be nq * 256. The result is bit-identical
 * to q38a_attention_decode followed by q38a_qgemm. */
int q38a_qgemm_merge_oproj(const q38a_attention_params* attn, const q38a_batch_desc* batch, const q38a_bq_weight* w,
                           const q38a_gemm_epilogue* ep, const q38a_gemm_workspace* ws, void* stream);

/* As q38a_qgemm_merge_oproj, but for batches the small-M GEMM kernel takes (up to 32 rows) the merge
 * runs inside the GEMM's A staging and attn->out is not written (reference OPTIMIZATION_PLAN.md:202-203,
 * "attention split-merge into the o-projection's A loader"); larger batches as q38a_qgemm_merge_oproj.
 * The merged A rows are the merge kernel's bits, but the GEMM is the split-K kernel, so at <= 8 rows
 * (where q38a_qgemm takes the wide-tile kernel) the results differ from q38a_qgemm_merge_oproj's in
 * the fp32 summation order (both within the GEMM's tolerance of the exact product). Measured slower
 * than the two launches at batch 8 (every GEMM workgroup repeats the merge of its A rows), so it is
 * not the default. */
int q38a_qgemm_merge_oproj_in_loader(const q38a_attention_params* attn, const q38a_batch_desc* batch,
                                     const q38a_bq_weight* w, const q38a_gemm_epilogue* ep,
                                     const q38a_gemm_workspace* ws, void* stream);

/* Floats of split-K partials and counters q38a_qgemm / q38a_qgemm_qkv_append may use for an
 * (m, n, k) problem: out[0] partial floats, out[1] counters. */
int q38a_qgemm_workspace_size(int m, int n, int k, size_t out[2]);

#ifdef __cplusplus
}
#endif

#endif /* Q38A_GEMM_H */
