/*
 * q4k_mmvq.hip - Q4_K x Q8_1 matrix-vector kernel for M <= 8 (decode).
 *
 * Arithmetic of the reference MMVQ (cuda/mmq/vecdotq.cuh:505-527,864-908):
 *   y[c][n] = sum_blk ( d * sum_b sc_b * d8_b * I_b  -  dmin * sum_b m_b * d8_b * S_b )
 * with I_b = sum of q4*q8 over sub-block b (exact int32, v_dot4_i32_i8) and
 * S_b = sum of q8 over b (precomputed by the row quantizer into dsf).
 *
 * gfx950 mapping (wave64, HBM-bound):
 *   - a Q4_K super-block is 9 x 16 bytes: header (d, dmin, 12 scale bytes)
 *     and 8 pieces of 16 qs bytes. Eight lanes ("a group") take one block:
 *     lane p loads qs piece p with one 16-byte load and the header with a
 *     second 16-byte load (all 8 lanes hit the same address). Piece p holds
 *     elements 16h..16h+15 (h = p&1) of sub-blocks 2*(p>>1) (low nibbles)
 *     and 2*(p>>1)+1 (high nibbles).
 *   - a wave covers RPW weight rows; the 8/RPW groups of a row walk its
 *     blocks with stride 8/RPW, so one wave-wide load touches 8 blocks,
 *     RPW rows x (8/RPW) consecutive blocks each.
 *   - nibbles are unpacked in registers (and/shift), dotted with v_dot4,
 *     scaled in fp32; the per-row partials are reduced across the row's
 *     lanes with xor shuffles (DPP/ds_swizzle) and one lane stores.
 */
#include "q4k_common.h"

template <int NCOLS, int RPW, int UNROLL>
__global__ __launch_bounds__(256) void sera_q4k_mmvq_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
        const float4 *__restrict__ dsf, float *__restrict__ y, int N, int K) {
    constexpr int LPR = 64 / RPW;     /* lanes per row */
    constexpr int GPR = LPR / 8;      /* 8-lane groups per row */
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int p = lane & 7;           /* qs piece */
    const int j2 = p >> 1;            /* sub-block pair */
    const int h = p & 1;              /* element half */
    const int gi = (lane >> 3) % GPR; /* group index within the row */
    const int row = (blockIdx.x * 4 + wave) * RPW + lane / LPR;
    if (row >= N) return;             /* whole row-group leaves together */

    const int nb = K / Q4K_QK;
    const uint8_t *wrow = W + (size_t)row * nb * Q4K_BLOCK_BYTES;

    float acc[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; c++) acc[c] = 0.0f;

    for (int blk0 = gi; blk0 < nb; blk0 += GPR * UNROLL) {
        uint4 hdr[UNROLL], qv[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int blk = blk0 + u * GPR;
            if (blk < nb) {
                const uint8_t *b = wrow + (size_t)blk * Q4K_BLOCK_BYTES;
                hdr[u] = *(const uint4 *)b;
                qv[u] = *(const uint4 *)(b + 16 + 16 * p);
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; u++) {
            const int blk = blk0 + u * GPR;
            if (blk >= nb) break;
            const float d = h2f_bits(hdr[u].x & 0xffffu);
            const float dmin = h2f_bits(hdr[u].x >> 16);
            uint32_t scA, mA, scB, mB;
            q4k_scale_min(2 * j2, hdr[u].y, hdr[u].z, hdr[u].w, &scA, &mA);
            q4k_scale_min(2 * j2 + 1, hdr[u].y, hdr[u].z, hdr[u].w, &scB, &mB);
            const int lo0 = qv[u].x & 0x0F0F0F0F, hi0 = (qv[u].x >> 4) & 0x0F0F0F0F;
            const int lo1 = qv[u].y & 0x0F0F0F0F, hi1 = (qv[u].y >> 4) & 0x0F0F0F0F;
            const int lo2 = qv[u].z & 0x0F0F0F0F, hi2 = (qv[u].z >> 4) & 0x0F0F0F0F;
            const int lo3 = qv[u].w & 0x0F0F0F0F, hi3 = (qv[u].w >> 4) & 0x0F0F0F0F;
            const float mh = (float)(h ? mB : mA);
            const size_t koff = (size_t)blk * Q4K_QK + 64 * j2 + 16 * h;
#pragma unroll
            for (int c = 0; c < NCOLS; c++) {
                const int8_t *xr = xq + (size_t)c * K + koff;
                const int4 xa = *(const int4 *)xr;
                const int4 xb = *(const int4 *)(xr + 32);
                const float4 f = dsf[(size_t)c * (K / 64) + blk * 4 + j2];
                int ia = __builtin_amdgcn_sdot4(lo0, xa.x, 0, false);
                ia = __builtin_amdgcn_sdot4(lo1, xa.y, ia, false);
                ia = __builtin_amdgcn_sdot4(lo2, xa.z, ia, false);
                ia = __builtin_amdgcn_sdot4(lo3, xa.w, ia, false);
                int ib = __builtin_amdgcn_sdot4(hi0, xb.x, 0, false);
                ib = __builtin_amdgcn_sdot4(hi1, xb.y, ib, false);
                ib = __builtin_amdgcn_sdot4(hi2, xb.z, ib, false);
                ib = __builtin_amdgcn_sdot4(hi3, xb.w, ib, false);
                const float sumd = f.x * (float)(ia * (int)scA) + f.y * (float)(ib * (int)scB);
                const float summ = (h ? f.w : f.z) * mh;
                acc[c] += d * sumd - dmin * summ;
            }
        }
    }

#pragma unroll
    for (int c = 0; c < NCOLS; c++) {
        float v = acc[c];
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[c] = v;
    }
    if ((lane % LPR) == 0) {
#pragma unroll
        for (int c = 0; c < NCOLS; c++) y[(size_t)c * N + row] = acc[c];
    }
}

template <int NCOLS, int RPW>
static hipError_t launch_mmvq(const uint8_t *W, const int8_t *xq, const float4 *dsf,
                              float *y, int N, int K, hipStream_t s) {
    const int rows_per_wg = 4 * RPW;
    dim3 grid((N + rows_per_wg - 1) / rows_per_wg);
    hipLaunchKernelGGL((sera_q4k_mmvq_kernel<NCOLS, RPW, 4>), grid, dim3(256), 0, s,
                       W, xq, dsf, y, N, K);
    return hipGetLastError();
}

/* Rows per wave: the largest of 8/4/2/1 that still gives >= 4096 waves
 * (16 per CU on 256 CUs), so short-N shapes split each row across more
 * lanes instead of leaving CUs idle. */
extern "C" int sera_mmvq_rows_per_wave(int N, int K) {
    (void)K;
    int rpw = 8;
    while (rpw > 1 && (N + rpw - 1) / rpw < 4096) rpw >>= 1;
    return rpw;
}

template <int NCOLS>
static hipError_t dispatch_rpw(int rpw, const uint8_t *W, const int8_t *xq, const float4 *dsf,
                               float *y, int N, int K, hipStream_t s) {
    switch (rpw) {
        case 8: return launch_mmvq<NCOLS, 8>(W, xq, dsf, y, N, K, s);
        case 4: return launch_mmvq<NCOLS, 4>(W, xq, dsf, y, N, K, s);
        case 2: return launch_mmvq<NCOLS, 2>(W, xq, dsf, y, N, K, s);
        default: return launch_mmvq<NCOLS, 1>(W, xq, dsf, y, N, K, s);
    }
}

extern "C" hipError_t sera_launch_q4k_mmvq(const void *W, const void *stage, float *y,
                                           int M, int N, int K, int rpw, hipStream_t s) {
    const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const float4 *dsf = (const float4 *)(base + L.dsf);
    const uint8_t *w = (const uint8_t *)W;
    if (rpw <= 0) rpw = sera_mmvq_rows_per_wave(N, K);
    switch (M) {
        case 1: return dispatch_rpw<1>(rpw, w, xq, dsf, y, N, K, s);
        case 2: return dispatch_rpw<2>(rpw, w, xq, dsf, y, N, K, s);
        case 3: return dispatch_rpw<3>(rpw, w, xq, dsf, y, N, K, s);
        case 4: return dispatch_rpw<4>(rpw, w, xq, dsf, y, N, K, s);
        case 5: return dispatch_rpw<5>(rpw, w, xq, dsf, y, N, K, s);
        case 6: return dispatch_rpw<6>(rpw, w, xq, dsf, y, N, K, s);
        case 7: return dispatch_rpw<7>(rpw, w, xq, dsf, y, N, K, s);
        case 8: return dispatch_rpw<8>(rpw, w, xq, dsf, y, N, K, s);
        default: return hipErrorInvalidValue;
    }
}
