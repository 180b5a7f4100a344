/*
 * q4k_aux.hip - the non-GEMM device work of the path:
 *
 *  - sera_q4k_quantize_kernel: fp32 weights -> GGUF Q4_K bytes on the GPU,
 *    the repo's quantizer of tools/qwen3_q4.py:316-481
 *    (quantize_q4_k_matrix) with its exact numpy float32/float64 arithmetic
 *    and pairwise-summation order; used to build the seeded synthetic
 *    weights resident in HBM.
 *  - sera_q4k_dequant_kernel: device twin of the CPU dequant,
 *    w = (d*sc)*q - (dmin*m) in fp32 (src/q3_quant.c:57-76,
 *    cuda/q3_cuda_primitives.cu:13-95), one thread per weight.
 *  - sera_q4k_subblock_dots_kernel: the exact int32 I_b = sum q4*q8 of
 *    every (token, row, 32-wide sub-block), computed with the same
 *    v_dot4_i32_i8 / nibble unpack the MMVQ kernel uses; exposed so tests
 *    can check the integer dots bit for bit.
 *
 * All float arithmetic in this file is uncontracted (no fused multiply-add)
 * so that it rounds exactly like the expressions it restates.
 */
#include "sera_launch.h"

/* No floating-point contraction in this file: the values here must follow
 * the reference's separately rounded multiplies and adds (hipcc fuses a * b
 * + c into one FMA by default, and the _rn intrinsics are plain operators
 * that do not prevent it). Explicit fmaf calls are unaffected. */
#pragma clang fp contract(off)

/* numpy add.reduce over 32 values: 0 + pairwise sum with 8 accumulators. */
template <typename T>
__device__ __forceinline__ T np_pairwise32(const T *a) {
#pragma clang fp contract(off)
    T r[8];
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = a[j];
#pragma unroll
    for (int i = 8; i < 32; i += 8)
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    const T res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    return (T)0 + res;
}

__device__ __forceinline__ int nearest_int_f32(float v) {
#pragma clang fp contract(off)
    const float t = v + 12582912.0f;
    return (__float_as_int(t) & 0x007FFFFF) - 0x00400000;
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* tools/qwen3_q4.py:94-111, f32_to_f16 bit trick (equals IEEE RNE). */
__device__ __forceinline__ uint32_t np_f32_to_f16(float x) {
#pragma clang fp contract(off)
    const uint32_t bits = __float_as_uint(x);
    const uint32_t sign = bits & 0x80000000u;
    const uint32_t shl1_w = bits + bits;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    float base = fabsf(x) * __uint_as_float(0x77800000u);
    base = base * __uint_as_float(0x08800000u);
    base = __uint_as_float((bias >> 1) + 0x07800000u) + base;
    const uint32_t out = __float_as_uint(base);
    const uint32_t nonsign = (((out >> 13) & 0x00007C00u) + (out & 0x00000FFFu)) & 0xffffu;
    const uint32_t r = (shl1_w > 0xFF000000u) ? 0x7E00u : nonsign;
    return (sign >> 16) | r;
}

/* _make_qkx2_quants_vec on one row of 32 (tools/qwen3_q4.py:326-389). The
 * running min is float32 until the first np.where(better, this_min, min_v),
 * float64 afterwards; every expression follows the dtype numpy gives it. */
__device__ void make_qkx2_32(const float *x, const float *w, uint8_t *L,
                             double *out_min, double *out_scale) {
#pragma clang fp contract(off)
    const int nmax = 15;
    float min_f = x[0], max_f = x[0];
#pragma unroll
    for (int i = 1; i < 32; i++) {
        min_f = x[i] < min_f ? x[i] : min_f;
        max_f = x[i] > max_f ? x[i] : max_f;
    }
    const float sum_w = np_pairwise32<float>(w);
    float wx[32];
#pragma unroll
    for (int i = 0; i < 32; i++) wx[i] = w[i] * x[i];
    const float sum_x = np_pairwise32<float>(wx);
    if (min_f > 0.0f) min_f = 0.0f;
    const bool eq = (max_f == min_f);
    const float max_safe = eq ? (min_f + 1.0f) : max_f;

    const float iscale0 = 15.0f / (max_safe - min_f);
    const float scale_f = 1.0f / iscale0;
    double tmp[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int l = clampi(nearest_int_f32(iscale0 * (x[i] - min_f)), 0, nmax);
        L[i] = (uint8_t)l;
        const double diff = ((double)scale_f * (double)l + (double)min_f) - (double)x[i];
        tmp[i] = ((double)w[i] * diff) * diff;
    }
    double best_error = np_pairwise32<double>(tmp);
    double scale = (double)scale_f;
    double min_v = (double)min_f;

    for (int istep = 0; istep <= 20; istep++) {
        const double c = (-1.0 + 0.1 * (double)istep) + (double)nmax;
        const float iscale = istep == 0 ? (float)c / (max_safe - min_f)
                                        : (float)(c / ((double)max_safe - min_v));
        uint8_t Laux[32];
        double sl[32], sl2[32], sxl[32];
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float z = istep == 0 ? iscale * (x[i] - min_f)
                                       : (float)((double)iscale * ((double)x[i] - min_v));
            const int l = clampi(nearest_int_f32(z), 0, nmax);
            Laux[i] = (uint8_t)l;
            const double wl = (double)w[i] * (double)l;
            sl[i] = wl;
            sl2[i] = wl * (double)l;
            sxl[i] = wl * (double)x[i];
        }
        const double sum_l = np_pairwise32<double>(sl);
        const double sum_l2 = np_pairwise32<double>(sl2);
        const double sum_xl = np_pairwise32<double>(sxl);
        const double D = (double)sum_w * sum_l2 - sum_l * sum_l;
        const bool Dpos = D > 0.0;
        const double Dsafe = Dpos ? D : 1.0;
        double this_scale = Dpos ? ((double)sum_w * sum_xl - (double)sum_x * sum_l) / Dsafe : 0.0;
        double this_min = Dpos ? (sum_l2 * (double)sum_x - sum_l * sum_xl) / Dsafe : 0.0;
        if (this_min > 0.0) {
            this_min = 0.0;
            this_scale = sum_xl / (sum_l2 > 0.0 ? sum_l2 : 1.0);
        }
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const double e = ((this_scale * (double)Laux[i]) + this_min) - (double)x[i];
            tmp[i] = (double)w[i] * (e * e);
        }
        const double cur_error = np_pairwise32<double>(tmp);
        if (cur_error < best_error) {
#pragma unroll
            for (int i = 0; i < 32; i++) L[i] = Laux[i];
            best_error = cur_error;
            scale = this_scale;
            min_v = this_min;
        }
    }
    if (eq) {
#pragma unroll
        for (int i = 0; i < 32; i++) L[i] = 0;
        scale = 0.0;
    }
    *out_min = -min_v;
    *out_scale = scale;
}

/* 64 threads = 8 super-blocks x 8 sub-blocks; thread (sb, j) owns sub-block
 * j of super-block sb. grid.x covers rows*K/256 super-blocks. */
__global__ __launch_bounds__(64) void sera_q4k_quantize_kernel(
        const float *__restrict__ xin, int64_t nblocks_total, uint8_t *__restrict__ out) {
#pragma clang fp contract(off)
    __shared__ double s_scale[8][8], s_min[8][8];
    __shared__ uint8_t s_L[8][8][32];
    const int sb = threadIdx.x >> 3, j = threadIdx.x & 7;
    const int64_t gb = (int64_t)blockIdx.x * 8 + sb;
    const bool valid = gb < nblocks_total;
    const float *x = xin + (valid ? gb : 0) * Q4K_QK + 32 * j;

    float xv[32], wv[32], sq[32];
#pragma unroll
    for (int i = 0; i < 32; i++) xv[i] = x[i];
#pragma unroll
    for (int i = 0; i < 32; i++) sq[i] = xv[i] * xv[i];
    const float sum_x2 = np_pairwise32<float>(sq);
    const float av_x = sqrtf(sum_x2 / 32.0f);
#pragma unroll
    for (int i = 0; i < 32; i++) wv[i] = av_x + fabsf(xv[i]);
    uint8_t L[32];
    double mn, sc;
    make_qkx2_32(xv, wv, L, &mn, &sc);
    s_scale[sb][j] = sc;
    s_min[sb][j] = mn;
    __syncthreads();

    double max_scale = s_scale[sb][0], max_min = s_min[sb][0];
    for (int t = 1; t < 8; t++) {
        max_scale = s_scale[sb][t] > max_scale ? s_scale[sb][t] : max_scale;
        max_min = s_min[sb][t] > max_min ? s_min[sb][t] : max_min;
    }
    const double inv_scale = max_scale > 0.0 ? 63.0 / max_scale : 0.0;
    const double inv_min = max_min > 0.0 ? 63.0 / max_min : 0.0;
    uint8_t so[12];
    for (int t = 0; t < 12; t++) so[t] = 0;
    for (int t = 0; t < 8; t++) {
        const int ls = clampi((int)rint(inv_scale * s_scale[sb][t]), 0, 63);
        const int lm = clampi((int)rint(inv_min * s_min[sb][t]), 0, 63);
        if (t < 4) {
            so[t] = (uint8_t)ls;
            so[t + 4] = (uint8_t)lm;
        } else {
            so[t + 4] = (uint8_t)((ls & 0x0F) | ((lm & 0x0F) << 4));
            so[t - 4] |= (uint8_t)(((ls >> 4) << 6) & 0xC0);
            so[t] |= (uint8_t)(((lm >> 4) << 6) & 0xC0);
        }
    }
    const uint32_t dh = np_f32_to_f16((float)(max_scale / 63.0));
    const uint32_t mh = np_f32_to_f16((float)(max_min / 63.0));
    const float d_f = h2f_bits(dh), dmin_f = h2f_bits(mh);
    uint32_t s0 = so[0] | (so[1] << 8) | (so[2] << 16) | ((uint32_t)so[3] << 24);
    uint32_t s1 = so[4] | (so[5] << 8) | (so[6] << 16) | ((uint32_t)so[7] << 24);
    uint32_t s2 = so[8] | (so[9] << 8) | (so[10] << 16) | ((uint32_t)so[11] << 24);
    uint32_t scj, mj;
    q4k_scale_min(j, s0, s1, s2, &scj, &mj);
    const float dd = d_f * (float)scj;
    const float dm = dmin_f * (float)mj;
    if (dd != 0.0f) {
#pragma unroll
        for (int i = 0; i < 32; i++) L[i] = (uint8_t)clampi(nearest_int_f32((xv[i] + dm) / dd), 0, 15);
    }
#pragma unroll
    for (int i = 0; i < 32; i++) s_L[sb][j][i] = L[i];
    __syncthreads();
    if (!valid) return;
    uint8_t *y = out + gb * Q4K_BLOCK_BYTES;
    if (j == 0) {
        uint4 hv;
        hv.x = dh | (mh << 16);
        hv.y = s0; hv.z = s1; hv.w = s2;
        *(uint4 *)y = hv;
    }
    if ((j & 1) == 0) {
        /* bytes (j/2)*32 + l: low nibble sub-block j, high nibble j+1 */
        uint8_t *q = y + 16 + (j >> 1) * 32;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; e++)
                v |= (uint32_t)(s_L[sb][j][i + e] | (s_L[sb][j + 1][i + e] << 4)) << (8 * e);
            *(uint32_t *)(q + i) = v;
        }
    }
}

/* One thread per weight, (d*sc)*q - (dmin*m) rounded step by step. out is
 * row-major [N][K]: weight i sits in block i / 256 of row order, read from
 * the GGUF bytes (tiled = 0) or from its place in the tiled layout of a
 * matrix with nkb super-blocks per row. */
__global__ __launch_bounds__(256) void sera_q4k_dequant_kernel(
        const uint8_t *__restrict__ W, int64_t nweights, float *__restrict__ out, int tiled, int64_t nkb) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nweights) return;
    const int64_t blk = i >> 8;
    const uint8_t *b = W + (tiled ? q4k_block_offset(1, (size_t)(blk / nkb), (size_t)(blk % nkb), (size_t)nkb)
                                  : (size_t)blk * Q4K_BLOCK_BYTES);
    const int e = (int)(i & 255), j = e >> 5, l = e & 31;
    const uint4 hv = *(const uint4 *)b;
    const float d = h2f_bits(hv.x & 0xffffu), dmin = h2f_bits(hv.x >> 16);
    uint32_t sc, m;
    q4k_scale_min(j, hv.y, hv.z, hv.w, &sc, &m);
    const uint8_t qb = b[16 + (j >> 1) * 32 + l];
    const uint32_t q = (j & 1) ? (qb >> 4) : (qb & 0xfu);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)m;
    out[i] = d1 * (float)q - m1;
}

/* I[m][n][b] for the row-layout stage: one thread per (m, n, super-block),
 * 8 sub-blocks each, through the v_dot4 path of the MMVQ kernel. */
__global__ __launch_bounds__(256) void sera_q4k_subblock_dots_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, int32_t *__restrict__ I,
        int M, int N, int K) {
    const int nb = K / Q4K_QK;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)M * N * nb) return;
    const int blk = (int)(idx % nb);
    const int n = (int)((idx / nb) % N);
    const int m = (int)(idx / ((int64_t)nb * N));
    const uint8_t *b = W + ((size_t)n * nb + blk) * Q4K_BLOCK_BYTES;
    const int8_t *x = xq + (size_t)m * K + (size_t)blk * Q4K_QK;
    for (int j2 = 0; j2 < 4; j2++) {
        int ia = 0, ib = 0;
        for (int h = 0; h < 2; h++) {
            const uint4 qv = *(const uint4 *)(b + 16 + 32 * j2 + 16 * h);
            const int4 xa = *(const int4 *)(x + 64 * j2 + 16 * h);
            const int4 xb = *(const int4 *)(x + 64 * j2 + 32 + 16 * h);
            ia = __builtin_amdgcn_sdot4((int)(qv.x & 0x0F0F0F0Fu), xa.x, ia, false);
            ia = __builtin_amdgcn_sdot4((int)(qv.y & 0x0F0F0F0Fu), xa.y, ia, false);
            ia = __builtin_amdgcn_sdot4((int)(qv.z & 0x0F0F0F0Fu), xa.z, ia, false);
            ia = __builtin_amdgcn_sdot4((int)(qv.w & 0x0F0F0F0Fu), xa.w, ia, false);
            ib = __builtin_amdgcn_sdot4((int)((qv.x >> 4) & 0x0F0F0F0Fu), xb.x, ib, false);
            ib = __builtin_amdgcn_sdot4((int)((qv.y >> 4) & 0x0F0F0F0Fu), xb.y, ib, false);
            ib = __builtin_amdgcn_sdot4((int)((qv.z >> 4) & 0x0F0F0F0Fu), xb.z, ib, false);
            ib = __builtin_amdgcn_sdot4((int)((qv.w >> 4) & 0x0F0F0F0Fu), xb.w, ib, false);
        }
        int32_t *o = I + ((size_t)m * N + n) * (K / 32) + (size_t)blk * 8 + 2 * j2;
        o[0] = ia;
        o[1] = ib;
    }
}

/* GGUF Q4_K rows [row0, row0 + rows) (back to back at src) into the tiled
 * layout of a matrix of nkb super-blocks per row. The 144-byte blocks move
 * whole, as nine 16-byte pieces: thread (row r, block b, piece c) copies
 * one piece. Reads are contiguous; a 16-row group's writes land in one
 * 16 x nkb x 144-byte run. rows and row0 are multiples of 16. */
__global__ __launch_bounds__(256) void sera_q4k_tile_kernel(const uint4 *__restrict__ src, uint8_t *__restrict__ dst,
                                                            uint64_t row0, uint64_t rows, uint64_t nkb) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nkb * 9) return;
    const uint64_t rb = i / 9;                  /* r * nkb + b within the source rows */
    const int c = (int)(i - rb * 9);
    const uint64_t r = rb / nkb, b = rb - r * nkb;
    *(uint4 *)(dst + q4k_block_offset(1, row0 + r, b, nkb) + 16 * c) = src[i];
}

extern "C" hipError_t sera_launch_q4k_tile(const void *src, void *dst, uint64_t row0, uint64_t rows, uint64_t nkb,
                                           hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const uint64_t threads = rows * nkb * 9;
    hipLaunchKernelGGL(sera_q4k_tile_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       (const uint4 *)src, (uint8_t *)dst, row0, rows, nkb);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q4k_quantize(const float *x, int64_t rows, int64_t K, void *out,
                                               hipStream_t s) {
    const int64_t nblocks = rows * (K / Q4K_QK);
    hipLaunchKernelGGL(sera_q4k_quantize_kernel, dim3((unsigned)((nblocks + 7) / 8)), dim3(64), 0, s,
                       x, nblocks, (uint8_t *)out);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q4k_dequant(const void *W, int64_t nblocks, float *out, hipStream_t s) {
    const int64_t n = nblocks * Q4K_QK;
    hipLaunchKernelGGL(sera_q4k_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)W, n, out, 0, (int64_t)1);
    return hipGetLastError();
}

/* The whole N x K matrix in the tiled layout, out row-major. */
extern "C" hipError_t sera_launch_q4k_dequant_tiled(const void *W, int64_t N, int64_t K, float *out, hipStream_t s) {
    const int64_t n = N * K;
    hipLaunchKernelGGL(sera_q4k_dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)W, n, out, 1, K / Q4K_QK);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q4k_subblock_dots(const void *W, const int8_t *xq, int32_t *I,
                                                    int M, int N, int K, hipStream_t s) {
    const int64_t n = (int64_t)M * N * (K / Q4K_QK);
    hipLaunchKernelGGL(sera_q4k_subblock_dots_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)W, xq, I, M, N, K);
    return hipGetLastError();
}
