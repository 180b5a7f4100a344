/*
 * q4k_mmq.hip - Q4_K x Q8_1 tiled GEMM on CDNA4 int8 MFMA (prefill, M > 8).
 *
 * Arithmetic of the reference MMQ (cuda/mmq/mmq.cuh:2269-2283 stores the
 * fp16 products (d*sc_b, -dmin*m_b) per row and sub-block; :1440-1472 adds
 * dmA.x*dsB.x*I_b and dmA.y*dsB.y per 32-wide sub-block):
 *   y[m][n] = sum_b  fp16(d*sc_b) * d8[m][b] * I[m][n][b]
 *                  + fp16(-dmin*m_b) * s8[m][b]
 * with d8, s8 the fp16 scale and fp16 sum of the DS4 Q8_1 quantizer.
 *
 * gfx950 mapping:
 *   - workgroup = 4 waves, tile 128 weight rows x BM tokens; each wave owns
 *     32 weight rows and all BM tokens (BM/32 column tiles of 32).
 *   - K advances one super-block (256) per step. The BM x 256 int8
 *     activation tile and its (d, sum) pairs are staged in LDS (double
 *     buffered, rows padded to 272 bytes so 16-byte reads of 16 consecutive
 *     tokens hit distinct banks). Weights are NOT staged: each lane loads
 *     its own row's 16-byte qs pieces straight into registers (the A operand
 *     of v_mfma_i32_32x32x32_i8 is 16 consecutive int8 of one row) and
 *     unpacks nibbles in registers; one 16-byte piece feeds the two
 *     sub-blocks that share it (low/high nibbles).
 *   - one v_mfma_i32_32x32x32_i8 per (sub-block, column tile) gives the
 *     exact int32 I_b for a 32x32 tile; the fp32 epilogue applies
 *     fp16(d*sc_b)*d8 per element (VALU).
 *   - the min term is a plain matrix product over the sub-block index:
 *     [rows x 8] fp16(-dmin*m_b) times [8 x tokens] fp16 s8, done per
 *     super-block by one v_mfma_f32_32x32x8_f16 that accumulates into the
 *     same fp32 tile (fp16 x fp16 products are exact in fp32).
 *   - the tile index is remapped so that the workgroups one XCD runs share
 *     weight rows (column tiles vary fastest within an XCD's range).
 *   - split-K: with few tiles, gridDim.y > 1 splits the super-blocks; each
 *     split writes fp32 partials that a second kernel sums in a fixed order
 *     (deterministic, no atomics).
 */
#include "q4k_common.h"

#define MMQ_BN 128
#define MMQ_XROW 272          /* LDS bytes per staged token row (256 + 16 pad) */

template <int BM>
struct MmqSmem {
    int8_t xs[2][BM][MMQ_XROW];
    uint32_t xds[2][BM][8];          /* half2 (d, sum) per token and sub-block */
    float sw[2][4][8][32];           /* fp16(d*sc) as float, per wave/sub-block/row */
};

__device__ __forceinline__ v4i unpack_nib(uint4 q, int hi) {
    const int s = hi ? 4 : 0;
    v4i a;
    a.x = (int)((q.x >> s) & 0x0F0F0F0Fu);
    a.y = (int)((q.y >> s) & 0x0F0F0F0Fu);
    a.z = (int)((q.z >> s) & 0x0F0F0F0Fu);
    a.w = (int)((q.w >> s) & 0x0F0F0F0Fu);
    return a;
}

/* Tile order: consecutive workgroup ids go to consecutive XCDs (8 on
 * MI355X). Give each XCD a contiguous run of tiles, column tiles fastest,
 * so the workgroups resident on one XCD reuse the same weight rows in L2. */
__device__ __forceinline__ int mmq_tile_of(int wg, int ntiles) {
    const int nx = 8;
    const int full = (ntiles / nx) * nx;
    if (wg >= full) return wg;
    const int per = ntiles / nx;
    return (wg % nx) * per + wg / nx;
}

template <int BM>
__global__ __launch_bounds__(256, 2) void sera_q4k_mmq_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, float *__restrict__ y, float *__restrict__ partial,
        int M, int N, int K, int kb_per_split) {
    constexpr int CT = BM / 32;              /* 32-token column tiles per wave */
    __shared__ MmqSmem<BM> sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int h = lane >> 5;

    const int ncol_tiles = (M + BM - 1) / BM;
    const int nrow_tiles = (N + MMQ_BN - 1) / MMQ_BN;
    const int tile = mmq_tile_of(blockIdx.x, ncol_tiles * nrow_tiles);
    const int rt = tile / ncol_tiles;
    const int ct = tile % ncol_tiles;
    const int n0 = rt * MMQ_BN;
    const int m0 = ct * BM;

    const int nkb_total = K / Q4K_QK;
    const int kb_begin = blockIdx.y * kb_per_split;
    const int kb_end = min(nkb_total, kb_begin + kb_per_split);
    const int nkb = kb_end - kb_begin;

    /* This lane's weight row for the A operand (row l32 of the wave's 32). */
    int wrow = n0 + wave * 32 + l32;
    if (wrow > N - 1) wrow = N - 1;          /* clamp; rows >= N are never stored */
    const uint8_t *wbase = W + (size_t)wrow * nkb_total * Q4K_BLOCK_BYTES;

    /* --- activation staging: BM tokens x 256 int8 + BM x 8 half2 per step --- */
    constexpr int XCH = BM * 16 / 256;       /* 16-byte chunks per thread */
    auto load_x = [&](int kb, uint4 *xr, uint4 &dr) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i;
            const int tok = c >> 4, piece = c & 15;
            xr[i] = *(const uint4 *)(xq + (size_t)(m0 + tok) * K + (size_t)kb * Q4K_QK + 16 * piece);
        }
        if (tid < BM * 2) {
            const int tok = tid >> 1, part = tid & 1;
            dr = *(const uint4 *)(xds + (size_t)(m0 + tok) * (K / 32) + kb * 8 + 4 * part);
        }
    };
    auto store_x = [&](int buf, const uint4 *xr, const uint4 &dr) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i;
            const int tok = c >> 4, piece = c & 15;
            *(uint4 *)&sm.xs[buf][tok][16 * piece] = xr[i];
        }
        if (tid < BM * 2) {
            const int tok = tid >> 1, part = tid & 1;
            *(uint4 *)&sm.xds[buf][tok][4 * part] = dr;
        }
    };
    /* --- weights: header + 4 qs pieces of 16 bytes (elements 16h..16h+15 of
     *     every sub-block pair) for this lane's row --- */
    auto load_w = [&](int kb, uint4 &hdr, uint4 *q) {
        const uint8_t *b = wbase + (size_t)kb * Q4K_BLOCK_BYTES;
        hdr = *(const uint4 *)b;
#pragma unroll
        for (int j2 = 0; j2 < 4; j2++) q[j2] = *(const uint4 *)(b + 16 + 32 * j2 + 16 * h);
    };
    /* fp16(d*sc_b) to LDS for the epilogue; fp16(-dmin*m_b) for b = 4h..4h+3
     * returned as the A operand of the min-term MFMA. */
    auto scales_w = [&](int buf, const uint4 &hdr) -> v4h {
        const f16 d = (f16)h2f_bits(hdr.x & 0xffffu);
        const f16 ndmin = -(f16)h2f_bits(hdr.x >> 16);
        v4h mw;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t sc, mn;
            q4k_scale_min(4 * h + e, hdr.y, hdr.z, hdr.w, &sc, &mn);
            const f16 dsc = d * (f16)(float)sc;      /* fp16 product, RNE */
            sm.sw[buf][wave][4 * h + e][l32] = (float)dsc;
            mw[e] = ndmin * (f16)(float)mn;
        }
        return mw;
    };

    v16f acc[CT];
#pragma unroll
    for (int t = 0; t < CT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    uint4 xr[XCH], dr = make_uint4(0, 0, 0, 0);
    uint4 hdr, qw[4], hdr_n, qw_n[4];

    if (nkb > 0) {
        load_x(kb_begin, xr, dr);
        store_x(0, xr, dr);
        load_w(kb_begin, hdr, qw);
    }
    v4h mw = scales_w(0, hdr);
    __syncthreads();

    for (int it = 0; it < nkb; it++) {
        const int buf = it & 1;
        const bool more = it + 1 < nkb;
        if (more) {
            load_x(kb_begin + it + 1, xr, dr);
            load_w(kb_begin + it + 1, hdr_n, qw_n);
        }
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const v4i A = unpack_nib(qw[b >> 1], b & 1);
            float sw[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 s4 = *(const float4 *)&sm.sw[buf][wave][b][8 * q + 4 * h];
                sw[4 * q + 0] = s4.x; sw[4 * q + 1] = s4.y;
                sw[4 * q + 2] = s4.z; sw[4 * q + 3] = s4.w;
            }
#pragma unroll
            for (int t = 0; t < CT; t++) {
                const int tok = 32 * t + l32;
                const v4i B = *(const v4i *)&sm.xs[buf][tok][32 * b + 16 * h];
                const v16i zero = {};
                const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, zero, 0, 0, 0);
                const float d8 = h2f_bits(sm.xds[buf][tok][b] & 0xffffu);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] = fmaf((float)I[r], sw[r] * d8, acc[t][r]);
            }
        }
        /* min term of this super-block: [32 rows x 8] x [8 x 32 tokens] */
#pragma unroll
        for (int t = 0; t < CT; t++) {
            const int tok = 32 * t + l32;
            const uint4 s = *(const uint4 *)&sm.xds[buf][tok][4 * h];
            v4h bs;
            bs[0] = (f16)h2f_bits(s.x >> 16);
            bs[1] = (f16)h2f_bits(s.y >> 16);
            bs[2] = (f16)h2f_bits(s.z >> 16);
            bs[3] = (f16)h2f_bits(s.w >> 16);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(mw, bs, acc[t], 0, 0, 0);
        }
        if (more) {
            store_x(buf ^ 1, xr, dr);
            hdr = hdr_n;
#pragma unroll
            for (int j2 = 0; j2 < 4; j2++) qw[j2] = qw_n[j2];
            mw = scales_w(buf ^ 1, hdr);
        }
        __syncthreads();
    }

    /* Store: lane holds token m0+32t+l32, rows n0+32*wave+8q+4h+{0..3}. */
    float *out = partial ? partial + (size_t)blockIdx.y * M * N : y;
#pragma unroll
    for (int t = 0; t < CT; t++) {
        const int m = m0 + 32 * t + l32;
        if (m >= M) continue;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int n = n0 + 32 * wave + 8 * q + 4 * h;
            float *dst = out + (size_t)m * N + n;
            if (n + 3 < N) {
                *(float4 *)dst = make_float4(acc[t][4 * q], acc[t][4 * q + 1],
                                             acc[t][4 * q + 2], acc[t][4 * q + 3]);
            } else {
                for (int e = 0; e < 4; e++)
                    if (n + e < N) dst[e] = acc[t][4 * q + e];
            }
        }
    }
}

/* Sums the split-K partials in split order: y = ((p0 + p1) + p2) + ... */
__global__ __launch_bounds__(256) void sera_splitk_reduce_kernel(
        const float4 *__restrict__ partial, float4 *__restrict__ y, size_t n4, int splits) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float4 s = partial[i];
    for (int k = 1; k < splits; k++) {
        const float4 v = partial[(size_t)k * n4 + i];
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    y[i] = s;
}

/* Column-tile width for M tokens: the smallest of 32/64/128 that covers M
 * in the fewest tiles. */
extern "C" int sera_mmq_bm(int M) {
    if (M <= 32) return 32;
    if (M <= 64) return 64;
    return 128;
}

/* Split-K factor: enough workgroups to give every CU at least two, but
 * never fewer than 2 super-blocks per split. */
extern "C" int sera_mmq_splits(int M, int N, int K) {
    const int bm = sera_mmq_bm(M);
    const int tiles = ((M + bm - 1) / bm) * ((N + MMQ_BN - 1) / MMQ_BN);
    const int nkb = K / Q4K_QK;
    int s = 1;
    while (tiles * s < 512 && nkb / (s * 2) >= 2 && s < 16) s *= 2;
    return s;
}

/* Rows of the MMQ activation stage: M rounded up to the column tile. */
extern "C" int sera_mmq_padded_rows(int M) {
    const int bm = sera_mmq_bm(M);
    return (M + bm - 1) / bm * bm;
}

template <int BM>
static hipError_t launch_mmq_bm(const uint8_t *W, const int8_t *xq, const uint32_t *xds, float *y,
                                float *partial, int M, int N, int K, int splits, hipStream_t s) {
    const int tiles = ((M + BM - 1) / BM) * ((N + MMQ_BN - 1) / MMQ_BN);
    const int nkb = K / Q4K_QK;
    const int per = (nkb + splits - 1) / splits;
    dim3 grid(tiles, splits);
    hipLaunchKernelGGL((sera_q4k_mmq_kernel<BM>), grid, dim3(256), 0, s, W, xq, xds, y,
                       splits > 1 ? partial : nullptr, M, N, K, per);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    const size_t n4 = (size_t)M * N / 4;
    hipLaunchKernelGGL(sera_splitk_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       (const float4 *)partial, (float4 *)y, n4, splits);
    return hipGetLastError();
}

/* partial: M*N*splits floats of scratch when splits > 1 (M*N % 4 == 0). */
extern "C" hipError_t sera_launch_q4k_mmq(const void *W, const void *stage, float *y, float *partial,
                                          int M, int N, int K, int splits, hipStream_t s) {
    const int Mpad = sera_mmq_padded_rows(M);
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const uint32_t *xds = (const uint32_t *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    switch (sera_mmq_bm(M)) {
        case 32: return launch_mmq_bm<32>(w, xq, xds, y, partial, M, N, K, splits, s);
        case 64: return launch_mmq_bm<64>(w, xq, xds, y, partial, M, N, K, splits, s);
        default: return launch_mmq_bm<128>(w, xq, xds, y, partial, M, N, K, splits, s);
    }
}
