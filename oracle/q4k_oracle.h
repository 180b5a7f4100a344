/*
 * q4k_oracle.h - CPU oracle for the Q4_K / Q6_K quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; nothing in the product (sera.c_amd/, include/) links,
 * loads or calls it. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may use it.
 *
 * It restates, in plain C99 with IEEE float/double arithmetic and no FMA
 * contraction (built with -ffp-contract=off), the arithmetic of the
 * reference (luca-saggese/sera.c) on this path:
 *
 *   fp16 <-> fp32 ............ src/q3_quant.c:18-42 (half->float, exact),
 *                              tools/qwen3_q4.py:94-130 (numpy bit tricks),
 *                              IEEE round-to-nearest-even (__float2half_rn)
 *   Q4_K block + dequant ..... src/q3_quant.h:28-33, src/q3_quant.c:44-76
 *   Q4_K quantizer ........... tools/qwen3_q4.py:316-481 (vectorized numpy
 *                              quantize_q4_k_matrix, numpy 2.x dtype rules)
 *   Q8_1 row quantizer ....... cuda/mmq/quantize.cu:4-48 (MMVQ activations)
 *   Q8_1 MMQ DS4 quantizer ... cuda/mmq/quantize.cu:271-367 (MMQ activations)
 *   per-32 int32 dots ........ cuda/mmq/vecdotq.cuh:505-527, mmq.cuh:1404-1476
 *   MMVQ output formula ...... cuda/mmq/vecdotq.cuh:505-527,864-908
 *   MMQ output formula ....... cuda/mmq/mmq.cuh:2269-2283,1440-1472
 *   dequant x fp32 GEMM ...... tests/test_q3_q4_linear.cu:236-277
 *   Q6_K block + dequant ..... src/q3_quant.c:78-103 (q6k_oracle.c)
 *   Q8_1 MMQ D4 quantizer .... cuda/mmq/quantize.cu:271-367 (Q6_K MMQ)
 *   Q6_K output formula ...... cuda/mmq/vecdotq.cuh:624-643,956-980 (MMVQ),
 *                              cuda/mmq/mmq.cuh:2687-2786 (MMQ)
 *
 * Pinning status of every function is listed in the comment above it and in
 * tests/test_oracle.py, which holds the checks.
 *
 * Layouts used by this oracle (all little-endian, row-major):
 *   W   : uint8 [N][K/256][144]            GGUF Q4_K super-blocks
 *   X   : float [M][K]
 *   xq  : int8  [M][K]                     Q8_1 quants
 *   xd  : uint16[M][K/32]                  fp16 bits of the Q8_1 scale d
 *   xs  : uint16[M][K/32]                  fp16 bits of the Q8_1 sum
 *   Y   : double[M][N]
 */
#ifndef SERA_Q4K_ORACLE_H
#define SERA_Q4K_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_Q4K_BYTES 144
#define ORC_QK8 32

/* fp16 bits -> float, exact. Restates src/q3_quant.c:18-42. */
float orc_h2f(uint16_t h);

/* float -> fp16 bits, IEEE round-to-nearest-even with subnormals, overflow
 * to inf, NaN kept NaN. Semantics of CUDA/HIP __float2half_rn. */
uint16_t orc_f2h(float f);

/* numpy bit-trick conversions of tools/qwen3_q4.py:94-111 and :114-130. */
uint16_t orc_np_f32_to_f16(float f);
float orc_np_f16_to_f32(uint16_t h);

/* Array forms of the four conversions above (n values). */
void orc_h2f_n(const uint16_t *h, size_t n, float *out);
void orc_f2h_n(const float *f, size_t n, uint16_t *out);
void orc_np_f32_to_f16_n(const float *f, size_t n, uint16_t *out);
void orc_np_f16_to_f32_n(const uint16_t *h, size_t n, float *out);

/* 6-bit scale/min of sub-block j (0..7). src/q3_quant.c:44-55. */
void orc_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* Q4_K dequant of `nblocks` consecutive super-blocks to 256*nblocks floats,
 * with the reference's fp32 expression order (d*sc)*q - (dmin*m).
 * src/q3_quant.c:57-76. */
void orc_dequant_q4k(const uint8_t *blocks, size_t nblocks, float *out);

/* Q4_K quantizer: float [rows][K] -> uint8 [rows][K/256][144].
 * Restates tools/qwen3_q4.py:316-481 (quantize_q4_k_matrix) including the
 * numpy 2.x float32/float64 promotion and pairwise-summation order.
 * Returns 0, or -1 when K % 256 != 0. */
int orc_quantize_q4k(const float *x, int64_t rows, int64_t K, uint8_t *out);

/* Q8_1 activation quantizers, one row of K values (K % 32 == 0).
 * orc_q8_1_row: cuda/mmq/quantize.cu:4-48   d = amax/127, q = roundf(x/d)
 * orc_q8_1_mmq: cuda/mmq/quantize.cu:271-367 d_inv = 127/amax,
 *               q = roundf(x*d_inv), d = 1/d_inv                         */
void orc_q8_1_row(const float *x, int64_t K, int8_t *qs, uint16_t *d, uint16_t *s);
void orc_q8_1_mmq(const float *x, int64_t K, int8_t *qs, uint16_t *d, uint16_t *s);

/* Exact per-32 integer dots I[m][n][b] = sum_{k in b} q4[n][k]*q8[m][k]. */
void orc_subblock_dots(const uint8_t *W, const int8_t *xq, int64_t M, int64_t N,
                       int64_t K, int32_t *I);

/* Per-32 sums of the Q8_1 quants, S[m][b] = sum_{k in b} q8[m][k]. */
void orc_q8_sums(const int8_t *xq, int64_t M, int64_t K, int32_t *S);

/* MMVQ-faithful output, accumulated in double:
 *   y = sum_blk [ d * sum_b sc_b*d8_b*I_b  -  dmin * sum_b m_b*d8_b*S_b ]
 * with d8_b the fp16 Q8_1 scale of the row quantizer. */
void orc_gemm_mmvq(const uint8_t *W, const int8_t *xq, const uint16_t *xd,
                   int64_t M, int64_t N, int64_t K, double *Y);

/* MMQ-faithful output, accumulated in double:
 *   y = sum_b [ fp16(d*sc_b) * d8_b * I_b  +  fp16(-dmin*m_b) * s8_b ]
 * with d8_b, s8_b the fp16 scale and fp16 sum of the DS4 quantizer. */
void orc_gemm_mmq(const uint8_t *W, const int8_t *xq, const uint16_t *xd,
                  const uint16_t *xs, int64_t M, int64_t N, int64_t K, double *Y);

/* Plain oracle of the reference test: dequantized W (fp32) x fp32 X,
 * double accumulation (tests/test_q3_q4_linear.cu:236-277). */
void orc_gemm_dequant(const uint8_t *W, const float *X, int64_t M, int64_t N,
                      int64_t K, double *Y);

/* ---- Q6_K (q6k_oracle.c): W is uint8 [N][K/256][210] GGUF Q6_K ---- */
#define ORC_Q6K_BYTES 210

/* One block -> q[256] = quant - 32, sc[16] int8 group scales, d fp32.
 * src/q3_quant.c:78-103. */
void orc_q6k_unpack(const uint8_t *blk, int8_t *q, int8_t *sc, float *d);

/* Q6_K dequant, (d*sc)*q in fp32 (src/q3_quant.c:78-103). */
void orc_dequant_q6k(const uint8_t *blocks, size_t nblocks, float *out);

/* Q8_1 MMQ quantizer, D4 layout (the one the reference uses for Q6_K):
 * quants as orc_q8_1_mmq, fp32 scale d = 1/d_inv per 32 values, no sum.
 * cuda/mmq/quantize.cu:271-367, cuda/mmq/mmq.cuh:64-103. */
void orc_q8_1_mmq_d4(const float *x, int64_t K, int8_t *qs, float *d);

/* Exact per-16 dots I[m][n][g] = sum (q-32)*q8 over group g (K/16 per row). */
void orc_q6k_group_dots(const uint8_t *W, const int8_t *xq, int64_t M, int64_t N, int64_t K,
                        int32_t *I);

/* y = sum_blk d * sum_g sc_g * d8[g/2] * I_g in double, d8 floats [M][K/32]
 * (fp16 row-quantizer scales for MMVQ, fp32 D4 scales for MMQ). */
void orc_gemm_q6k(const uint8_t *W, const int8_t *xq, const float *d8, int64_t M, int64_t N,
                  int64_t K, double *Y);

/* Dequantized Q6_K W (fp32) x fp32 X, double accumulation. */
void orc_gemm_dequant_q6k(const uint8_t *W, const float *X, int64_t M, int64_t N, int64_t K,
                          double *Y);

#ifdef __cplusplus
}
#endif

#endif
