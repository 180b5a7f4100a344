/*
 * q4k_skinny.hip - Q4_K x Q8_1 for few tokens (M <= 16) on int8 MFMA.
 *
 * One v_mfma_i32_16x16x32_i8 gives the exact int32 dot I_b of one 32-wide
 * sub-block for 16 tokens x 16 weight rows. Tokens are the A operand,
 * weights the B operand, so in the 16x16 result a lane owns one weight row
 * and four tokens: lane l holds row l%16 and tokens 4*(l/16) + r, r = 0..3.
 * Tokens past M compute on a copy of the last token and are never stored.
 *
 * Two output formulas, chosen at compile time so each path keeps the
 * reference's arithmetic:
 *   MMVQ (row stage; cuda/mmq/vecdotq.cuh:505-527,864-908):
 *     y = sum_b (d*sc_b) * d8_b * I_b  -  sum_b (dmin*m_b) * (d8_b*S_b)
 *     with d*sc_b and dmin*m_b exact in fp32 and d8_b*S_b from the stage;
 *     the min term runs as fp32 fmas on the vector ALU.
 *   MMQ (MMQ stage; cuda/mmq/mmq.cuh:2269-2283,1440-1472):
 *     y = sum_b fp16(d*sc_b) * d8_b * I_b  +  sum_b fp16(-dmin*m_b) * s8_b
 *     the min term is a rank-8 product, one v_mfma_f32_16x16x16_f16 per
 *     16-row tile (fp16 x fp16 products are exact in fp32).
 *
 * Work split, as the MMQ kernel: a workgroup is 4 waves along N, each wave
 * CT tiles of 16 weight rows, so 64*CT rows per workgroup; all waves walk K
 * together. Per 256-wide K step the 16 tokens' quants go global -> LDS with
 * 16-byte direct-to-LDS loads (one per thread, XOR-swizzled 16-byte columns
 * so the 8-byte A reads of 16 tokens spread over the banks) and their
 * scales through registers; weights go HBM -> registers one step ahead
 * (per lane and row tile: the 16-byte header and four 8-byte nibble pieces
 * of its k-octet). gridDim.y > 1 splits K; partials then go through the
 * split-K reduce kernel.
 */
#include "q4k_common.h"

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void sk_lds_void;
typedef __attribute__((address_space(1))) const void sk_global_cvoid;

struct SkinnySmem {
    alignas(16) int8_t xs[2][16][Q4K_QK];   /* quants; piece c of token t at column c ^ t */
    alignas(16) float d8[2][8][16];         /* d8 as float, [sub-block][token] */
    alignas(16) float mn[2][8][16];         /* MMVQ: d8*S; MMQ: s8 as float */
};

__device__ __forceinline__ h2 sk_as_h2(uint32_t u) {
    union { uint32_t u; h2 h; } c;
    c.u = u;
    return c.h;
}

/* FORM 0 = MMVQ formula on a row stage, 1 = MMQ formula on an MMQ stage. */
template <int FORM, int CT>
__global__ __launch_bounds__(256) void sera_q4k_skinny_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const void *__restrict__ xsc,
        float *__restrict__ y, float *__restrict__ partial, int M, int N, int K, int kb_per_split, int accum) {
    __shared__ SkinnySmem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 15;          /* B: weight row in a tile; A: token */
    const int gk = lane >> 4;         /* k-octet; result tokens 4*gk .. 4*gk+3 */
    const int nkb_total = K / Q4K_QK;
    const int kb_begin = blockIdx.y * kb_per_split;
    const int kb_end = min(nkb_total, kb_begin + kb_per_split);
    const int nkb = kb_end - kb_begin;
    const int n0 = blockIdx.x * (64 * CT) + 16 * CT * wave;

    const uint8_t *wrow[CT];
    bool row_ok[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) {
        int row = n0 + 16 * c + j;
        row_ok[c] = row < N;
        if (!row_ok[c]) row = N - 1;  /* clamp; never stored */
        wrow[c] = W + (size_t)row * nkb_total * Q4K_BLOCK_BYTES;
    }

    /* --- activations: quants by direct-to-LDS loads, scales by registers --- */
    auto issue_x = [&](int kb, int buf) {
        const int t = tid >> 4, col = tid & 15;              /* LDS piece (t, col) */
        const int ts = min(t, M - 1);                        /* tokens past M copy the last one */
        const int8_t *src = xq + (size_t)ts * K + (size_t)kb * Q4K_QK + 16 * (col ^ t);
        __builtin_amdgcn_global_load_lds((sk_global_cvoid *)src, (sk_lds_void *)&sm.xs[buf][0][wave * 1024], 16, 0, 0);
    };
    auto load_sc = [&](int kb, v4u &sr) {
        if (FORM == 0) {
            /* dsf float4 [M][K/64]: thread = token t x pair p */
            const int t = min(tid >> 2, M - 1), p = tid & 3;
            if (tid < 64) sr = *(const v4u *)((const uint8_t *)xsc + ((size_t)t * (K / 64) + 4 * kb + p) * 16);
        } else {
            /* ds half2 [Mpad][K/32]: thread = token t x sub-block b */
            const int t = min(tid >> 3, M - 1), b = tid & 7;
            if (tid < 128) sr.x = ((const uint32_t *)xsc)[(size_t)t * (K / 32) + 8 * kb + b];
        }
    };
    auto store_sc = [&](int buf, const v4u &sr) {
        if (FORM == 0) {
            if (tid < 64) {
                const int t = tid >> 2, p = tid & 3;
                sm.d8[buf][2 * p][t] = __uint_as_float(sr.x);
                sm.d8[buf][2 * p + 1][t] = __uint_as_float(sr.y);
                sm.mn[buf][2 * p][t] = __uint_as_float(sr.z);
                sm.mn[buf][2 * p + 1][t] = __uint_as_float(sr.w);
            }
        } else {
            if (tid < 128) {
                const int t = tid >> 3, b = tid & 7;
                sm.d8[buf][b][t] = h2f_bits(sr.x & 0xffffu);
                sm.mn[buf][b][t] = h2f_bits(sr.x >> 16);
            }
        }
    };
    /* --- weights: header and four 8-byte nibble pieces per row tile --- */
    struct WRegs {
        v4u hd[CT];
        v2u qp[CT][4];
    };
    auto load_w = [&](int kb, WRegs &wr) {
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const uint8_t *bp = wrow[c] + (size_t)kb * Q4K_BLOCK_BYTES;
            wr.hd[c] = *(const v4u *)bp;
#pragma unroll
            for (int p = 0; p < 4; p++) wr.qp[c][p] = *(const v2u *)(bp + 16 + 32 * p + 8 * gk);
        }
    };

    v4f acc[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) acc[c] = (v4f){0.f, 0.f, 0.f, 0.f};
    v4u sr = {0u, 0u, 0u, 0u};
    WRegs wr;
    if (nkb > 0) {
        issue_x(kb_begin, 0);
        load_sc(kb_begin, sr);
        store_sc(0, sr);
        load_w(kb_begin, wr);
    }
    __builtin_amdgcn_s_waitcnt(0);   /* this thread's loads to LDS have landed */
    __syncthreads();

    for (int it = 0; it < nkb; it++) {
        const int buf = it & 1;
        const bool more = it + 1 < nkb;
        if (more) {
            issue_x(kb_begin + it + 1, buf ^ 1);   /* buffer last read one step ago, freed by the barrier */
            load_sc(kb_begin + it + 1, sr);
        }
        /* the 8-byte A fragments (token j, k-octet gk) of the eight sub-blocks */
        v2i A[8];
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int piece = 2 * b + (gk >> 1);
            A[b] = *(const v2i *)&sm.xs[buf][j][16 * (piece ^ j) + 8 * (gk & 1)];
        }
#pragma unroll
        for (int c = 0; c < CT; c++) {
            /* (scale, min) of the eight sub-blocks, four at a time
             * (src/q3_quant.c:44-55) */
            const v4u hd = wr.hd[c];
            const uint32_t sc03 = hd.y & 0x3F3F3F3Fu;
            const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
            const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
            const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
            float swb[8], mwb[8];
            if (FORM == 0) {
                const float d = h2f_bits(hd.x & 0xffffu), dmin = h2f_bits(hd.x >> 16);
#pragma unroll
                for (int b = 0; b < 8; b++) {
                    const uint32_t scw = b < 4 ? sc03 : sc47, mw = b < 4 ? m03 : m47;
                    const int sh = 8 * (b & 3);
                    swb[b] = d * (float)((scw >> sh) & 0xffu);       /* exact: fp16 x 6-bit */
                    mwb[b] = -dmin * (float)((mw >> sh) & 0xffu);
                }
            } else {
                /* fp16(d*sc) and fp16(-dmin*m), one RNE rounding each: the
                 * 6-bit value v sits under exponent byte 0x64 (fp16 1024 + v)
                 * and the subtraction of 1024 is exact */
                const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
                const h2 dd = sk_as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x01000100u));
                const h2 nm = -sk_as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x03020302u));
                const uint32_t src[4] = {sc03, sc47, m03, m47};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const h2 lo = sk_as_h2(__builtin_amdgcn_perm(0x64646464u, src[q], 0x04010400u)) - bias;
                    const h2 hi = sk_as_h2(__builtin_amdgcn_perm(0x64646464u, src[q], 0x04030402u)) - bias;
                    const h2 a = lo * (q < 2 ? dd : nm), e = hi * (q < 2 ? dd : nm);
                    float *dst = q < 2 ? swb : mwb;
                    const int b0 = 4 * (q & 1);
                    dst[b0] = (float)a.x; dst[b0 + 1] = (float)a.y;
                    dst[b0 + 2] = (float)e.x; dst[b0 + 3] = (float)e.y;
                }
            }
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t sh = (b & 1) ? 4u : 0u;
                const v2u q = wr.qp[c][b >> 1];
                v2i Bw;
                Bw.x = (int)((q.x >> sh) & 0x0F0F0F0Fu);
                Bw.y = (int)((q.y >> sh) & 0x0F0F0F0Fu);
                const v4f d8 = *(const v4f *)&sm.d8[buf][b][4 * gk];
                const v4i zero = {0, 0, 0, 0};
                const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    __builtin_bit_cast(long, A[b]), __builtin_bit_cast(long, Bw), zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[c][r] = fmaf((float)I[r], d8[r] * swb[b], acc[c][r]);
            }
            /* min term: acc[t][n] += sum_b mn[b][t] * mwb_n[b], a rank-8 product */
            if (FORM == 0) {
#pragma unroll
                for (int b = 0; b < 8; b++) {
                    const v4f dS = *(const v4f *)&sm.mn[buf][b][4 * gk];
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[c][r] = fmaf(dS[r], mwb[b], acc[c][r]);
                }
            } else {
                /* lane group gk holds k = 4gk..4gk+3: sub-blocks 0..7 in
                 * groups 0-1, zeros in groups 2-3 */
                v4h a, bm;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int b = (4 * gk + e) & 7;
                    a[e] = gk < 2 ? (_Float16)sm.mn[buf][b][j] : (_Float16)0.0f;
                    bm[e] = gk < 2 ? (_Float16)mwb[b] : (_Float16)0.0f;
                }
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, bm, acc[c], 0, 0, 0);
            }
        }
        if (more) {
            load_w(kb_begin + it + 1, wr);
            store_sc(buf ^ 1, sr);
        }
        __builtin_amdgcn_s_waitcnt(0);   /* this thread's loads to LDS have landed */
        __syncthreads();
    }

    float *out = partial ? partial + (size_t)blockIdx.y * M * N : y;
#pragma unroll
    for (int c = 0; c < CT; c++) {
        if (!row_ok[c]) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 4 * gk + r;
            if (t < M) {
                float *dst = out + (size_t)t * N + n0 + 16 * c + j;
                *dst = !partial && accum ? *dst + acc[c][r] : acc[c][r];
            }
        }
    }
}

extern "C" hipError_t sera_launch_splitk_reduce_acc(const float *partial, float *y, size_t n, int splits, int accum,
                                                    hipStream_t s);
extern "C" int sera_mmq_padded_rows(int M);

#define SK_CT 2   /* 16-row tiles per wave: 128 weight rows per workgroup */

/* Split count for the few-token kernel: fill the chip with workgroups, keep
 * at least 4 super-blocks per split. */
extern "C" int sera_skinny_splits(int M, int N, int K) {
    (void)M;
    const int wgs = (N + 64 * SK_CT - 1) / (64 * SK_CT);
    const int nkb = K / Q4K_QK;
    int s = 1;
    while (wgs * s < 1024 && nkb / (s * 2) >= 4 && s < 16) s *= 2;
    return s;
}

template <int FORM>
static hipError_t launch_skinny(const uint8_t *W, const int8_t *xq, const void *xsc, float *y, float *partial,
                                int M, int N, int K, int splits, int accum, hipStream_t s) {
    const int nkb = K / Q4K_QK;
    const int per = (nkb + splits - 1) / splits;
    dim3 grid((N + 64 * SK_CT - 1) / (64 * SK_CT), splits);
    hipLaunchKernelGGL((sera_q4k_skinny_kernel<FORM, SK_CT>), grid, dim3(256), 0, s, W, xq, xsc, y,
                       splits > 1 ? partial : nullptr, M, N, K, per, accum);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q4k_skinny_acc(int form, const void *W, const void *stage, float *y,
                                                 float *partial, int M, int N, int K, int splits, int accum,
                                                 hipStream_t s);

/* form 0: row stage (MMVQ formula), form 1: MMQ stage (MMQ formula).
 * partial: splits*M*N floats when splits > 1 (M*N % 4 == 0). */
extern "C" hipError_t sera_launch_q4k_skinny(int form, const void *W, const void *stage, float *y, float *partial,
                                             int M, int N, int K, int splits, hipStream_t s) {
    return sera_launch_q4k_skinny_acc(form, W, stage, y, partial, M, N, K, splits, 0, s);
}

/* accum != 0 adds the product to y. */
extern "C" hipError_t sera_launch_q4k_skinny_acc(int form, const void *W, const void *stage, float *y,
                                                 float *partial, int M, int N, int K, int splits, int accum,
                                                 hipStream_t s) {
    const char *base = (const char *)stage;
    const uint8_t *w = (const uint8_t *)W;
    hipError_t e;
    if (form == 0) {
        const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
        e = launch_skinny<0>(w, (const int8_t *)(base + L.qs), base + L.dsf, y, partial, M, N, K, splits, accum, s);
    } else {
        const sera_stage_layout L = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K);
        e = launch_skinny<1>(w, (const int8_t *)(base + L.qs), base + L.ds, y, partial, M, N, K, splits, accum, s);
    }
    if (e != hipSuccess || splits <= 1) return e;
    return sera_launch_splitk_reduce_acc(partial, y, (size_t)M * N, splits, accum, s);
}
