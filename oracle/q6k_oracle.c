/*
 * q6k_oracle.c - CPU oracle for the Q6_K quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see q4k_oracle.h, which declares these
 * functions). Build with -ffp-contract=off: every float/double operation is
 * one IEEE operation, as written.
 *
 * GGUF Q6_K super-block, 256 weights in 210 bytes (src/q3_quant.h:26,
 * cuda/mmq/ggml-common.h:348-357 block_q6_K):
 *   bytes   0-127  ql[128]  low 4 bits of each 6-bit quant
 *   bytes 128-191  qh[64]   high 2 bits, four quants per byte
 *   bytes 192-207  sc[16]   int8 scale of each 16-wide group
 *   bytes 208-209  d        fp16 super-block scale
 * Weight e = 128*j + 32*k + l (j in 0..1, k in 0..3, l in 0..31):
 *   q = (low nibble of ql[64j + 32*(k&1) + l] for k < 2, high nibble for
 *        k >= 2) | ((qh[32j + l] >> 2k) & 3) << 4, value q - 32 in [-32, 31]
 *   group g = e / 16 = 8j + 2k + l/16, weight = d * sc[g] * (q - 32)
 * (src/q3_quant.c:78-103; the group index is its sc0[is + 2k] with
 * is = l/16 and sc0 advanced by 8 per 128 weights).
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void orc_q6k_unpack(const uint8_t *blk, int8_t *q, int8_t *sc, float *d) {
    const uint8_t *ql = blk, *qh = blk + 128;
    for (int j = 0; j < 2; j++)
        for (int k = 0; k < 4; k++)
            for (int l = 0; l < 32; l++) {
                const uint8_t lo = ql[64 * j + 32 * (k & 1) + l];
                const int nib = k < 2 ? (lo & 0xf) : (lo >> 4);
                const int hi = (qh[32 * j + l] >> (2 * k)) & 3;
                q[128 * j + 32 * k + l] = (int8_t)((nib | (hi << 4)) - 32);
            }
    for (int g = 0; g < 16; g++) sc[g] = (int8_t)blk[192 + g];
    *d = orc_h2f(rd16(blk + 208));
}

/* src/q3_quant.c:78-103: out = d * (float)sc * (float)q, left to right in
 * fp32, i.e. (d*sc)*q with one rounding per multiply. */
void orc_dequant_q6k(const uint8_t *blocks, size_t nblocks, float *out) {
    int8_t q[256], sc[16];
    float d;
    for (size_t b = 0; b < nblocks; b++) {
        orc_q6k_unpack(blocks + b * ORC_Q6K_BYTES, q, sc, &d);
        for (int e = 0; e < 256; e++) {
            const float dsc = d * (float)sc[e / 16];
            out[b * 256 + e] = dsc * (float)q[e];
        }
    }
}

/* cuda/mmq/quantize.cu:271-367 with the D4 layout the reference selects for
 * Q6_K (mmq.cuh:64-103, cuda/q3_mmq.cu:303-316): the quants are those of
 * the DS4 quantizer (d_inv = 127/amax, q = roundf(x*d_inv)); the scale is
 * stored as the fp32 d = 1/d_inv, no sum. amax == 0 gives q = 0, d = 0. */
void orc_q8_1_mmq_d4(const float *x, int64_t K, int8_t *qs, float *d) {
    for (int64_t ib = 0; ib < K / 32; ib++) {
        const float *xb = x + ib * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            const float ax = fabsf(xb[i]);
            if (ax > amax) amax = ax;
        }
        int8_t *q = qs + ib * 32;
        if (amax == 0.0f) {
            for (int i = 0; i < 32; i++) q[i] = 0;
            d[ib] = 0.0f;
        } else {
            const float d_inv = 127.0f / amax;
            for (int i = 0; i < 32; i++) q[i] = (int8_t)roundf(xb[i] * d_inv);
            d[ib] = 1.0f / d_inv;
        }
    }
}

/* Exact per-16 integer dots I[m][n][g] = sum_{e in group g} (q_e - 32) * q8_e,
 * the integer each 16-wide group contributes in the reference's MMQ
 * (mmq.cuh:2554-2555 stores q - 32 per byte; one tile_A x tile_B product is
 * one group, :2770-2775) and MMVQ (vecdotq.cuh:624-643, four quants per dp4a). */
void orc_q6k_group_dots(const uint8_t *W, const int8_t *xq, int64_t M, int64_t N, int64_t K,
                        int32_t *I) {
    const int64_t nb = K / ORC_QK_K, ng = K / 16;
    int8_t q[256], sc[16];
    float d;
    for (int64_t n = 0; n < N; n++)
        for (int64_t ib = 0; ib < nb; ib++) {
            orc_q6k_unpack(W + (n * nb + ib) * ORC_Q6K_BYTES, q, sc, &d);
            for (int64_t m = 0; m < M; m++) {
                const int8_t *x = xq + m * K + ib * 256;
                for (int g = 0; g < 16; g++) {
                    int32_t acc = 0;
                    for (int i = 0; i < 16; i++) acc += (int32_t)q[16 * g + i] * (int32_t)x[16 * g + i];
                    I[(m * N + n) * ng + ib * 16 + g] = acc;
                }
            }
        }
}

/* Q6_K output formula shared by both reference paths, accumulated in double:
 *   y = sum_blk d * sum_{g=0..15} sc_g * d8[g/2] * I_g
 * MMVQ (vecdotq.cuh:624-643,956-980): d8 = the fp16 scale of the row Q8_1
 * quantizer; each dp4a of four quants is multiplied by its group's scale
 * and by d8, and the thread's sum by d.
 * MMQ (mmq.cuh:2687-2786, the tensor-core branch): d8 = the fp32 D4 scale;
 * (C0*sc_2b + C1*sc_2b+1) * d8_b per 32-wide step (:2775), times d per
 * 128 weights (:2784).
 * The caller passes d8 as floats [M][K/32]. */
void orc_gemm_q6k(const uint8_t *W, const int8_t *xq, const float *d8, int64_t M, int64_t N,
                  int64_t K, double *Y) {
    const int64_t nb = K / ORC_QK_K, ns = K / 32;
    int8_t q[256], sc[16];
    float d;
    for (int64_t m = 0; m < M; m++) for (int64_t n = 0; n < N; n++) Y[m * N + n] = 0.0;
    for (int64_t n = 0; n < N; n++)
        for (int64_t ib = 0; ib < nb; ib++) {
            orc_q6k_unpack(W + (n * nb + ib) * ORC_Q6K_BYTES, q, sc, &d);
            for (int64_t m = 0; m < M; m++) {
                const int8_t *x = xq + m * K + ib * 256;
                double s = 0.0;
                for (int g = 0; g < 16; g++) {
                    int32_t acc = 0;
                    for (int i = 0; i < 16; i++) acc += (int32_t)q[16 * g + i] * (int32_t)x[16 * g + i];
                    s += (double)sc[g] * (double)d8[m * ns + ib * 8 + g / 2] * (double)acc;
                }
                Y[m * N + n] += (double)d * s;
            }
        }
}

/* Dequantized W (fp32, the reference's expression order) times fp32 X,
 * double accumulation (tests/test_q3_q4_linear.cu:236-277 with the Q6_K
 * dequant). */
void orc_gemm_dequant_q6k(const uint8_t *W, const float *X, int64_t M, int64_t N, int64_t K,
                          double *Y) {
    const int64_t nb = K / ORC_QK_K;
    float *row = (float *)malloc((size_t)K * sizeof(float));
    if (!row) return;
    for (int64_t n = 0; n < N; n++) {
        orc_dequant_q6k(W + n * nb * ORC_Q6K_BYTES, (size_t)nb, row);
        for (int64_t m = 0; m < M; m++) {
            double acc = 0.0;
            const float *x = X + m * K;
            for (int64_t k = 0; k < K; k++) acc += (double)row[k] * (double)x[k];
            Y[m * N + n] = acc;
        }
    }
    free(row);
}
