/*
 * q4k_oracle.c - CPU oracle for the Q4_K quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see q4k_oracle.h). Build with
 * -ffp-contract=off: every float/double operation below is one IEEE
 * operation, as written, with no fused multiply-add.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp16 <-> fp32                                                       */
/* ------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* src/q3_quant.c:18-42: sign, 5-bit exponent, 10-bit fraction; subnormal
 * halves are renormalised, exponent 31 maps to inf/NaN. */
float orc_h2f(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t f = h & 0x3ffu;
    uint32_t v;
    if (e == 0) {
        if (f == 0) {
            v = sign;
        } else {
            int shift = 0;
            while (!(f & 0x400u)) { f <<= 1; shift++; }
            f &= 0x3ffu;
            v = sign | ((uint32_t)(113 - shift) << 23) | (f << 13);
        }
    } else if (e == 0x1fu) {
        v = sign | 0x7f800000u | (f << 13);
    } else {
        v = sign | ((e + 112u) << 23) | (f << 13);
    }
    return u2f(v);
}

/* IEEE binary32 -> binary16, round to nearest, ties to even. */
uint16_t orc_f2h(float fl) {
    uint32_t x = f2u(fl);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                 /* inf or NaN */
        return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    }
    int e = (int)(ax >> 23) - 127;           /* unbiased exponent */
    uint32_t mant = (ax & 0x7fffffu) | (ax >= 0x00800000u ? 0x800000u : 0u);
    if (ax < 0x00800000u) e = -126;          /* fp32 subnormal */
    /* Target: value = mant * 2^(e-23). Half normal needs e >= -14. */
    int shift;                               /* right shift of the 24-bit mant */
    uint32_t hexp;
    if (e >= -14) {
        if (e > 15) return sign | 0x7c00u;   /* overflow */
        shift = 13;
        hexp = (uint32_t)(e + 15);
    } else {
        shift = 13 + (-14 - e);              /* subnormal half */
        hexp = 0;
        if (shift > 24) return sign;         /* rounds to zero (below half of min subnormal) */
    }
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) q++;
    uint32_t out;
    if (hexp == 0) {
        out = q;                              /* q <= 0x400 -> may become min normal */
    } else {
        /* q has implicit bit at 0x400; carry may bump the exponent */
        out = (hexp << 10) + (q - 0x400u);
        if (q & 0x800u) out = ((hexp + 1) << 10); /* mantissa overflow after rounding */
    }
    if (out >= 0x7c00u) out = 0x7c00u;
    return (uint16_t)(sign | out);
}

/* tools/qwen3_q4.py:94-111 (f32_to_f16), restated on one value. */
uint16_t orc_np_f32_to_f16(float x) {
    uint32_t bits = f2u(x);
    uint32_t sign = bits & 0x80000000u;
    uint32_t shl1_w = bits + bits;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    float base = fabsf(x) * u2f(0x77800000u) /* 2^112 */;
    base = base * u2f(0x08800000u) /* 2^-110 */;
    base = u2f((bias >> 1) + 0x07800000u) + base;
    uint32_t out = f2u(base);
    uint32_t exp_bits = (out >> 13) & 0x00007C00u;
    uint32_t mantissa_bits = out & 0x00000FFFu;
    uint16_t nonsign = (uint16_t)(exp_bits + mantissa_bits);
    uint16_t r = (shl1_w > 0xFF000000u) ? (uint16_t)0x7E00u : nonsign;
    return (uint16_t)((sign >> 16) | r);
}

/* tools/qwen3_q4.py:114-130 (f16_to_f32), restated on one value. */
float orc_np_f16_to_f32(uint16_t h) {
    uint32_t w = (uint32_t)h << 16;
    uint32_t sign = w & 0x80000000u;
    uint32_t two_w = w + w;
    uint32_t exp_offset = 0xE0u << 23;
    float normalized = u2f((two_w >> 4) + exp_offset) * u2f(0x07800000u) /* 2^-112 */;
    float denormalized = u2f((two_w >> 17) | (126u << 23)) - 0.5f;
    uint32_t r = sign | (two_w < (1u << 27) ? f2u(denormalized) : f2u(normalized));
    return u2f(r);
}

void orc_h2f_n(const uint16_t *h, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_h2f(h[i]);
}
void orc_f2h_n(const float *f, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f2h(f[i]);
}
void orc_np_f32_to_f16_n(const float *f, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_np_f32_to_f16(f[i]);
}
void orc_np_f16_to_f32_n(const uint16_t *h, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_np_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------ */
/* Q4_K layout and dequant                                             */
/* ------------------------------------------------------------------ */

void orc_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63u;
        *m = s[j + 4] & 63u;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xfu) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/q3_quant.c:57-76. Sub-block j uses qs[(j/2)*32 + l]: low nibble for
 * even j, high nibble for odd j. */
void orc_dequant_q4k(const uint8_t *blocks, size_t nblocks, float *out) {
    for (size_t ib = 0; ib < nblocks; ib++) {
        const uint8_t *b = blocks + ib * ORC_Q4K_BYTES;
        const float d = orc_h2f(rd16(b));
        const float dmin = orc_h2f(rd16(b + 2));
        const uint8_t *scales = b + 4;
        const uint8_t *q = b + 16;
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            orc_scale_min_k4(j, scales, &sc, &m);
            const float d1 = d * (float)sc;
            const float m1 = dmin * (float)m;
            const uint8_t *qq = q + (j / 2) * 32;
            for (int l = 0; l < 32; l++) {
                const unsigned nib = (j & 1) ? (qq[l] >> 4) : (qq[l] & 0xfu);
                *out++ = d1 * (float)nib - m1;
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* Q4_K quantizer (tools/qwen3_q4.py:316-481)                           */
/* ------------------------------------------------------------------ */

/* numpy add.reduce over 32 contiguous values: identity 0 + pairwise sum
 * with 8 accumulators (numpy loops_utils pairwise_sum, n <= 128). */
static float np_sum32f(const float *a) {
    float r[8];
    for (int j = 0; j < 8; j++) r[j] = a[j];
    for (int i = 8; i < 32; i += 8)
        for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    return 0.0f + res;
}

static double np_sum32d(const double *a) {
    double r[8];
    for (int j = 0; j < 8; j++) r[j] = a[j];
    for (int i = 8; i < 32; i += 8)
        for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    return 0.0 + res;
}

/* _nearest_int_vec: float32(v) + 1.5*2^23, mantissa bits - 2^22. */
static int32_t nearest_int_f32(float v) {
    float t = v + 12582912.0f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007FFFFF) - 0x00400000;
}

static int32_t clip_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* _make_qkx2_quants_vec for one row of 32 (tools/qwen3_q4.py:326-389),
 * nmax=15, rmin=-1, rdelta=0.1, nstep=20. min_v starts as float32 and
 * becomes float64 after the first np.where(better, this_min, min_v); the
 * flag `min_is_f64` tracks which arithmetic the numpy expressions use. */
static void make_qkx2_32(const float *x, const float *w, uint8_t *L,
                         double *out_min, double *out_scale) {
    const int nmax = 15;
    float min_f = x[0], max_f = x[0];
    for (int i = 1; i < 32; i++) {
        if (x[i] < min_f) min_f = x[i];
        if (x[i] > max_f) max_f = x[i];
    }
    const float sum_w = np_sum32f(w);
    float wx[32];
    for (int i = 0; i < 32; i++) wx[i] = w[i] * x[i];
    const float sum_x = np_sum32f(wx);

    if (min_f > 0.0f) min_f = 0.0f;
    const int eq = (max_f == min_f);
    const float max_safe = eq ? (min_f + 1.0f) : max_f;

    float iscale_f = 15.0f / (max_safe - min_f);
    float scale_f = 1.0f / iscale_f;
    uint8_t Laux[32];
    double tmp[32];
    for (int i = 0; i < 32; i++) {
        int32_t l = nearest_int_f32(iscale_f * (x[i] - min_f));
        l = clip_i32(l, 0, nmax);
        L[i] = (uint8_t)l;
        const double diff = ((double)scale_f * (double)l + (double)min_f) - (double)x[i];
        tmp[i] = ((double)w[i] * diff) * diff;
    }
    double best_error = np_sum32d(tmp);
    double scale = (double)scale_f;   /* dtype becomes f64 at the first where() */
    double min_v = (double)min_f;
    int min_is_f64 = 0;

    for (int istep = 0; istep <= 20; istep++) {
        const double c = (-1.0 + 0.1 * (double)istep) + (double)nmax;
        float iscale;
        if (!min_is_f64) {
            iscale = (float)c / (max_safe - min_f);
        } else {
            iscale = (float)(c / ((double)max_safe - min_v));
        }
        double sl[32], sl2[32], sxl[32];
        for (int i = 0; i < 32; i++) {
            float z;
            if (!min_is_f64) z = iscale * (x[i] - min_f);
            else z = (float)((double)iscale * ((double)x[i] - min_v));
            int32_t l = nearest_int_f32(z);
            l = clip_i32(l, 0, nmax);
            Laux[i] = (uint8_t)l;
            const double wl = (double)w[i] * (double)l;
            sl[i] = wl;
            sl2[i] = wl * (double)l;
            sxl[i] = wl * (double)x[i];
        }
        const double sum_l = np_sum32d(sl);
        const double sum_l2 = np_sum32d(sl2);
        const double sum_xl = np_sum32d(sxl);
        const double D = (double)sum_w * sum_l2 - sum_l * sum_l;
        const int Dpos = D > 0.0;
        const double Dsafe = Dpos ? D : 1.0;
        double this_scale = Dpos ? ((double)sum_w * sum_xl - (double)sum_x * sum_l) / Dsafe : 0.0;
        double this_min = Dpos ? (sum_l2 * (double)sum_x - sum_l * sum_xl) / Dsafe : 0.0;
        const int mpos = this_min > 0.0;
        if (mpos) {
            this_min = 0.0;
            this_scale = sum_xl / (sum_l2 > 0.0 ? sum_l2 : 1.0);
        }
        for (int i = 0; i < 32; i++) {
            const double e = ((this_scale * (double)Laux[i]) + this_min) - (double)x[i];
            tmp[i] = (double)w[i] * (e * e);
        }
        const double cur_error = np_sum32d(tmp);
        if (cur_error < best_error) {
            memcpy(L, Laux, 32);
            best_error = cur_error;
            scale = this_scale;
            min_v = this_min;
        }
        min_is_f64 = 1;   /* np.where(better, this_min, min_v) is float64 */
    }
    if (eq) {
        memset(L, 0, 32);
        scale = 0.0;
    }
    *out_min = -min_v;
    *out_scale = scale;
}

int orc_quantize_q4k(const float *xin, int64_t rows, int64_t K, uint8_t *out) {
    if (K % ORC_QK_K) return -1;
    const int64_t nb = K / ORC_QK_K;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t ib = 0; ib < nb; ib++) {
            const float *x = xin + r * K + ib * ORC_QK_K;
            uint8_t *y = out + (r * nb + ib) * ORC_Q4K_BYTES;
            uint8_t L[256];
            double mins[8], scales[8];
            for (int j = 0; j < 8; j++) {
                const float *xj = x + 32 * j;
                float sq[32], w[32];
                for (int i = 0; i < 32; i++) sq[i] = xj[i] * xj[i];
                const float sum_x2 = np_sum32f(sq);
                const float av_x = sqrtf(sum_x2 / 32.0f);
                for (int i = 0; i < 32; i++) w[i] = av_x + fabsf(xj[i]);
                make_qkx2_32(xj, w, L + 32 * j, &mins[j], &scales[j]);
            }
            double max_scale = scales[0], max_min = mins[0];
            for (int j = 1; j < 8; j++) {
                if (scales[j] > max_scale) max_scale = scales[j];
                if (mins[j] > max_min) max_min = mins[j];
            }
            const double inv_scale = max_scale > 0.0 ? 63.0 / max_scale : 0.0;
            const double inv_min = max_min > 0.0 ? 63.0 / max_min : 0.0;
            uint8_t so[12];
            memset(so, 0, sizeof(so));
            for (int j = 0; j < 8; j++) {
                int32_t ls = (int32_t)nearbyint(inv_scale * scales[j]);
                int32_t lm = (int32_t)nearbyint(inv_min * mins[j]);
                ls = clip_i32(ls, 0, 63);
                lm = clip_i32(lm, 0, 63);
                if (j < 4) {
                    so[j] = (uint8_t)ls;
                    so[j + 4] = (uint8_t)lm;
                } else {
                    so[j + 4] = (uint8_t)((ls & 0x0F) | ((lm & 0x0F) << 4));
                    so[j - 4] |= (uint8_t)(((ls >> 4) << 6) & 0xC0);
                    so[j] |= (uint8_t)(((lm >> 4) << 6) & 0xC0);
                }
            }
            const uint16_t dh = orc_np_f32_to_f16((float)(max_scale / 63.0));
            const uint16_t mh = orc_np_f32_to_f16((float)(max_min / 63.0));
            y[0] = (uint8_t)(dh & 0xff); y[1] = (uint8_t)(dh >> 8);
            y[2] = (uint8_t)(mh & 0xff); y[3] = (uint8_t)(mh >> 8);
            memcpy(y + 4, so, 12);
            const float d_f = orc_np_f16_to_f32(dh);
            const float dmin_f = orc_np_f16_to_f32(mh);
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                orc_scale_min_k4(j, so, &sc, &m);
                const float dd = d_f * (float)sc;
                const float dm = dmin_f * (float)m;
                if (dd == 0.0f) continue;            /* keep L from the search */
                for (int i = 0; i < 32; i++) {
                    int32_t l = nearest_int_f32((x[32 * j + i] + dm) / dd);
                    L[32 * j + i] = (uint8_t)clip_i32(l, 0, 15);
                }
            }
            for (int p = 0; p < 4; p++)
                for (int l = 0; l < 32; l++)
                    y[16 + p * 32 + l] = (uint8_t)(L[64 * p + l] | (L[64 * p + 32 + l] << 4));
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Q8_1 activation quantizers                                          */
/* ------------------------------------------------------------------ */

/* cuda/mmq/quantize.cu:4-48. 32 lanes hold one value each; amax and sum
 * come from an xor butterfly over offsets 16,8,4,2,1 (lane 0's value). */
void orc_q8_1_row(const float *x, int64_t K, int8_t *qs, uint16_t *d, uint16_t *s) {
    for (int64_t ib = 0; ib < K / 32; ib++) {
        const float *xb = x + ib * 32;
        float a[32], amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            a[i] = xb[i];
            const float ax = fabsf(xb[i]);
            if (ax > amax) amax = ax;
        }
        for (int off = 16; off >= 1; off >>= 1)
            for (int i = 0; i < off; i++) a[i] = a[i] + a[i + off];
        const float sum = a[0];
        const float dd = amax / 127.0f;
        for (int i = 0; i < 32; i++) {
            const float q = (amax == 0.0f) ? 0.0f : roundf(xb[i] / dd);
            qs[ib * 32 + i] = (int8_t)q;
        }
        d[ib] = orc_f2h(dd);
        s[ib] = orc_f2h(sum);
    }
}

/* cuda/mmq/quantize.cu:271-367, DS4 layout. 8 threads hold 4 values each;
 * a thread sums ((x0+x1)+x2)+x3, then xor 4,2,1 across the 8 threads. */
void orc_q8_1_mmq(const float *x, int64_t K, int8_t *qs, uint16_t *d, uint16_t *s) {
    for (int64_t ib = 0; ib < K / 32; ib++) {
        const float *xb = x + ib * 32;
        float t[8], amax = 0.0f;
        for (int th = 0; th < 8; th++) {
            const float *v = xb + 4 * th;
            t[th] = ((v[0] + v[1]) + v[2]) + v[3];
            for (int i = 0; i < 4; i++) {
                const float ax = fabsf(v[i]);
                if (ax > amax) amax = ax;
            }
        }
        for (int off = 4; off >= 1; off >>= 1)
            for (int i = 0; i < off; i++) t[i] = t[i] + t[i + off];
        const float sum = t[0];
        int8_t *q = qs + ib * 32;
        float dd;
        if (amax == 0.0f) {
            /* d_inv = inf, x*inf = NaN -> 0 on conversion, d = 1/inf = 0 */
            for (int i = 0; i < 32; i++) q[i] = 0;
            dd = 0.0f;
        } else {
            const float d_inv = 127.0f / amax;
            for (int i = 0; i < 32; i++) q[i] = (int8_t)roundf(xb[i] * d_inv);
            dd = 1.0f / d_inv;
        }
        d[ib] = orc_f2h(dd);
        s[ib] = orc_f2h(sum);
    }
}

/* ------------------------------------------------------------------ */
/* Integer dots and output formulas                                    */
/* ------------------------------------------------------------------ */

static void unpack_q4(const uint8_t *blk, uint8_t *q4 /* [256] */) {
    const uint8_t *qs = blk + 16;
    for (int j = 0; j < 8; j++)
        for (int l = 0; l < 32; l++) {
            const uint8_t v = qs[(j / 2) * 32 + l];
            q4[32 * j + l] = (j & 1) ? (uint8_t)(v >> 4) : (uint8_t)(v & 0xf);
        }
}

void orc_subblock_dots(const uint8_t *W, const int8_t *xq, int64_t M, int64_t N,
                       int64_t K, int32_t *I) {
    const int64_t nb = K / ORC_QK_K, ns = K / 32;
    uint8_t q4[256];
    for (int64_t n = 0; n < N; n++) {
        for (int64_t ib = 0; ib < nb; ib++) {
            unpack_q4(W + (n * nb + ib) * ORC_Q4K_BYTES, q4);
            for (int64_t m = 0; m < M; m++) {
                const int8_t *x = xq + m * K + ib * 256;
                for (int j = 0; j < 8; j++) {
                    int32_t acc = 0;
                    for (int l = 0; l < 32; l++) acc += (int32_t)q4[32 * j + l] * (int32_t)x[32 * j + l];
                    I[(m * N + n) * ns + ib * 8 + j] = acc;
                }
            }
        }
    }
}

void orc_q8_sums(const int8_t *xq, int64_t M, int64_t K, int32_t *S) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t b = 0; b < K / 32; b++) {
            int32_t acc = 0;
            for (int l = 0; l < 32; l++) acc += xq[m * K + b * 32 + l];
            S[m * (K / 32) + b] = acc;
        }
}

void orc_gemm_mmvq(const uint8_t *W, const int8_t *xq, const uint16_t *xd,
                   int64_t M, int64_t N, int64_t K, double *Y) {
    const int64_t nb = K / ORC_QK_K, ns = K / 32;
    uint8_t q4[256];
    for (int64_t m = 0; m < M; m++) for (int64_t n = 0; n < N; n++) Y[m * N + n] = 0.0;
    for (int64_t n = 0; n < N; n++) {
        for (int64_t ib = 0; ib < nb; ib++) {
            const uint8_t *blk = W + (n * nb + ib) * ORC_Q4K_BYTES;
            unpack_q4(blk, q4);
            const double d = orc_h2f(rd16(blk));
            const double dmin = orc_h2f(rd16(blk + 2));
            for (int64_t m = 0; m < M; m++) {
                const int8_t *x = xq + m * K + ib * 256;
                double sd = 0.0, sm = 0.0;
                for (int j = 0; j < 8; j++) {
                    uint8_t sc, mn;
                    orc_scale_min_k4(j, blk + 4, &sc, &mn);
                    int32_t I = 0, S = 0;
                    for (int l = 0; l < 32; l++) {
                        I += (int32_t)q4[32 * j + l] * (int32_t)x[32 * j + l];
                        S += x[32 * j + l];
                    }
                    const double d8 = orc_h2f(xd[m * ns + ib * 8 + j]);
                    sd += (double)sc * d8 * (double)I;
                    sm += (double)mn * d8 * (double)S;
                }
                Y[m * N + n] += d * sd - dmin * sm;
            }
        }
    }
}

void orc_gemm_mmq(const uint8_t *W, const int8_t *xq, const uint16_t *xd,
                  const uint16_t *xs, int64_t M, int64_t N, int64_t K, double *Y) {
    const int64_t nb = K / ORC_QK_K, ns = K / 32;
    uint8_t q4[256];
    for (int64_t m = 0; m < M; m++) for (int64_t n = 0; n < N; n++) Y[m * N + n] = 0.0;
    for (int64_t n = 0; n < N; n++) {
        for (int64_t ib = 0; ib < nb; ib++) {
            const uint8_t *blk = W + (n * nb + ib) * ORC_Q4K_BYTES;
            unpack_q4(blk, q4);
            const float d = orc_h2f(rd16(blk));
            const float dmin = orc_h2f(rd16(blk + 2));
            for (int j = 0; j < 8; j++) {
                uint8_t sc, mn;
                orc_scale_min_k4(j, blk + 4, &sc, &mn);
                /* half2 products of mmq.cuh:2278-2282: exact in fp32, then RNE to fp16 */
                const double dsc = orc_h2f(orc_f2h(d * (float)sc));
                const double dmm = orc_h2f(orc_f2h(-dmin * (float)mn));
                for (int64_t m = 0; m < M; m++) {
                    const int8_t *x = xq + m * K + ib * 256 + 32 * j;
                    int32_t I = 0;
                    for (int l = 0; l < 32; l++) I += (int32_t)q4[32 * j + l] * (int32_t)x[l];
                    const double d8 = orc_h2f(xd[m * ns + ib * 8 + j]);
                    const double s8 = orc_h2f(xs[m * ns + ib * 8 + j]);
                    Y[m * N + n] += dsc * d8 * (double)I + dmm * s8;
                }
            }
        }
    }
}

void orc_gemm_dequant(const uint8_t *W, const float *X, int64_t M, int64_t N,
                      int64_t K, double *Y) {
    const int64_t nb = K / ORC_QK_K;
    float *row = (float *)malloc((size_t)K * sizeof(float));
    if (!row) return;
    for (int64_t n = 0; n < N; n++) {
        orc_dequant_q4k(W + n * nb * ORC_Q4K_BYTES, (size_t)nb, row);
        for (int64_t m = 0; m < M; m++) {
            double acc = 0.0;
            const float *x = X + m * K;
            for (int64_t k = 0; k < K; k++) acc += (double)row[k] * (double)x[k];
            Y[m * N + n] = acc;
        }
    }
    free(row);
}
