/*
 * q4k_skinny.hip - Q4_K x Q8_1 for few tokens (M <= 16) on int8 MFMA.
 *
 * One v_mfma_i32_16x16x32_i8 gives the exact int32 dot I_b of one 32-wide
 * sub-block for 16 tokens x 16 weight rows. Tokens are the A operand (rows
 * beyond M read as zero), weights the B operand, so in the 16x16 result a
 * lane owns one weight row and four tokens: lane l holds row l%16 and tokens
 * 4*(l/16) + r, r = 0..3.
 *
 * Two output formulas, chosen at compile time so each path keeps the
 * reference's arithmetic:
 *   MMVQ (M <= 8, row stage; cuda/mmq/vecdotq.cuh:505-527,864-908):
 *     y = sum_b (d*sc_b) * d8_b * I_b  -  sum_b (dmin*m_b) * (d8_b*S_b)
 *     with d*sc_b and dmin*m_b exact in fp32 and d8_b*S_b from the stage.
 *   MMQ (M > 8, MMQ stage; cuda/mmq/mmq.cuh:2269-2283,1440-1472):
 *     y = sum_b fp16(d*sc_b) * d8_b * I_b  +  sum_b fp16(-dmin*m_b) * s8_b
 * The min term is a rank-8 product over the sub-block index: fp32 fmas on
 * the vector ALU for MMVQ, one v_mfma_f32_16x16x16_f16 for MMQ (fp16
 * operands, products exact in fp32).
 *
 * Work split: a workgroup is WGN x WGK waves. The WGN waves along N each own
 * 16 weight rows; the WGK waves along K take interleaved super-blocks and
 * run independently until their partial sums meet in LDS, in a fixed
 * order, at the end. Per super-block a lane loads, one super-block ahead,
 * its row's 16-byte header and the four 8-byte nibble pieces of its k-octet
 * (B), the 8-byte k-octets of its token for the eight sub-blocks (A), and
 * one word of the 16 tokens' scales, which the wave transposes through its
 * own double-buffered LDS tile (no workgroup barrier in the loop).
 * gridDim.y > 1 splits K further; partials then go through the split-K
 * reduce kernel.
 */
#include "q4k_common.h"

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

/* Per-wave LDS: the 16 tokens' scales of one super-block, double buffered.
 * d8[b][t] = d8 of token t, sub-block b; mn[b][t] = d8*S (MMVQ) or s8 (MMQ). */
struct SkinnyWaveSmem {
    alignas(16) float d8[2][8][16];
    alignas(16) float mn[2][8][16];
};

__device__ __forceinline__ h2 sk_as_h2(uint32_t u) {
    union { uint32_t u; h2 h; } c;
    c.u = u;
    return c.h;
}

/* FORM 0 = MMVQ formula on a row stage, 1 = MMQ formula on an MMQ stage. */
template <int FORM, int WGN, int WGK>
__global__ __launch_bounds__(256) void sera_q4k_skinny_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const void *__restrict__ xsc,
        float *__restrict__ y, float *__restrict__ partial, int M, int N, int K, int kb_per_split) {
    static_assert(WGN * WGK == 4, "4 waves");
    __shared__ SkinnyWaveSmem wsm[4];
    __shared__ __attribute__((aligned(16))) float red[WGK > 1 ? WGK - 1 : 1][WGN][64][4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave % WGN, wk = wave / WGN;
    const int j = lane & 15;          /* B: weight row; A: token */
    const int gk = lane >> 4;         /* k-octet; result tokens 4*gk .. 4*gk+3 */
    SkinnyWaveSmem &sm = wsm[wave];
    const int nkb_total = K / Q4K_QK;
    const int kb_begin = blockIdx.y * kb_per_split;
    const int kb_end = min(nkb_total, kb_begin + kb_per_split);
    /* this wave's super-blocks: kb_begin + wk, + WGK, ... */
    const int nmine = kb_end - kb_begin - wk > 0 ? (kb_end - kb_begin - wk + WGK - 1) / WGK : 0;

    int row = blockIdx.x * (16 * WGN) + 16 * wn + j;
    const bool row_ok = row < N;
    if (!row_ok) row = N - 1;         /* clamp; never stored */
    const uint8_t *wrow = W + (size_t)row * nkb_total * Q4K_BLOCK_BYTES;
    /* Activation loads go through buffer resources sized to the M real
     * tokens: a token >= M reads as zero, without a branch. */
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(xq), (short)0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(xsc), (short)0, FORM == 0 ? M * (K / 64) * 16 : M * (K / 32) * 4, 0x00020000);

    /* One super-block's operands in registers: weight header and nibble
     * pieces of row `row`, the A fragments of token j (k-octet gk of each
     * sub-block), and one scale word for the LDS scale tile. */
    struct Regs {
        v4u hd;
        v2u qp[4];
        v2i xa[8];
        v4f f;
    };
    auto load = [&](int i, Regs &r) {
        const int kb = kb_begin + wk + i * WGK;
        const uint8_t *bp = wrow + (size_t)kb * Q4K_BLOCK_BYTES;
        r.hd = *(const v4u *)bp;
#pragma unroll
        for (int p = 0; p < 4; p++) r.qp[p] = *(const v2u *)(bp + 16 + 32 * p + 8 * gk);
        const int vx = j * K + 8 * gk;                 /* token j, k-octet gk */
#pragma unroll
        for (int b = 0; b < 8; b++)
            r.xa[b] = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rx, vx, kb * Q4K_QK + 32 * b, 0));
        const int t = lane >> 2, p = lane & 3;         /* token t x pair p */
        if (FORM == 0) {
            /* dsf float4 [M][K/64] */
            r.f = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, (t * (K / 64) + 4 * kb + p) * 16, 0, 0));
        } else {
            /* ds half2 [Mpad][K/32]: sub-blocks 2p, 2p+1 */
            const v2u h = __builtin_amdgcn_raw_buffer_load_b64(rs, (t * (K / 32) + 8 * kb + 2 * p) * 4, 0, 0);
            r.f = (v4f){__uint_as_float(h.x), __uint_as_float(h.y), 0.f, 0.f};
        }
    };
    auto store_scales = [&](int buf, const Regs &r) {
        const int t = lane >> 2, p = lane & 3;
        if (FORM == 0) {
            sm.d8[buf][2 * p][t] = r.f.x;
            sm.d8[buf][2 * p + 1][t] = r.f.y;
            sm.mn[buf][2 * p][t] = r.f.z;
            sm.mn[buf][2 * p + 1][t] = r.f.w;
        } else {
            const uint32_t h0 = __float_as_uint(r.f.x), h1 = __float_as_uint(r.f.y);
            sm.d8[buf][2 * p][t] = h2f_bits(h0 & 0xffffu);
            sm.mn[buf][2 * p][t] = h2f_bits(h0 >> 16);
            sm.d8[buf][2 * p + 1][t] = h2f_bits(h1 & 0xffffu);
            sm.mn[buf][2 * p + 1][t] = h2f_bits(h1 >> 16);
        }
    };

    v4f acc = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Regs &r, int buf) {
        /* the wave's own scale writes precede these reads in LDS order */
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    /* (scale, min) of the eight sub-blocks, four at a time
     * (src/q3_quant.c:44-55) */
    const v4u hd = r.hd;
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
        /* fp16(d*sc) and fp16(-dmin*m), one RNE rounding each: the 6-bit
         * value v sits under exponent byte 0x64 (fp16 1024 + v) and the
         * subtraction of 1024 is exact */
        const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 dd = sk_as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x01000100u));
        const h2 nm = -sk_as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x03020302u));
        const uint32_t src[4] = {sc03, sc47, m03, m47};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const h2 lo = sk_as_h2(__builtin_amdgcn_perm(0x64646464u, src[q], 0x04010400u)) - bias;
            const h2 hi = sk_as_h2(__builtin_amdgcn_perm(0x64646464u, src[q], 0x04030402u)) - bias;
            const h2 a = lo * (q < 2 ? dd : nm), c = hi * (q < 2 ? dd : nm);
            float *dst = q < 2 ? swb : mwb;
            const int b0 = 4 * (q & 1);
            dst[b0] = (float)a.x; dst[b0 + 1] = (float)a.y;
            dst[b0 + 2] = (float)c.x; dst[b0 + 3] = (float)c.y;
        }
    }

#pragma unroll
    for (int b = 0; b < 8; b++) {
        const uint32_t sh = (b & 1) ? 4u : 0u;
        const v2u q = r.qp[b >> 1];
        v2i Bw;
        Bw.x = (int)((q.x >> sh) & 0x0F0F0F0Fu);
        Bw.y = (int)((q.y >> sh) & 0x0F0F0F0Fu);
        const v4f d8 = *(const v4f *)&sm.d8[buf][b][4 * gk];
        const v4i zero = {0, 0, 0, 0};
        const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(
            __builtin_bit_cast(long, r.xa[b]), __builtin_bit_cast(long, Bw), zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = fmaf((float)I[r], d8[r] * swb[b], acc[r]);
    }

    /* min term: acc[t][n] += sum_b mn[b][t] * mwb_n[b], a rank-8 product */
    if (FORM == 0) {
        /* fp32 on the vector ALU: d8*S of the lane's four tokens per sub-block */
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const v4f dS = *(const v4f *)&sm.mn[buf][b][4 * gk];
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = fmaf(dS[r], mwb[b], acc[r]);
        }
    } else {
        /* one fp16 16x16x16 product (fp16 x fp16 products are exact in
         * fp32); lane group gk holds k = 4gk..4gk+3: sub-blocks 0..7 in
         * groups 0-1, zeros in groups 2-3 */
        v4h a, bm;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int b = (4 * gk + e) & 7;
            a[e] = gk < 2 ? (_Float16)sm.mn[buf][b][j] : (_Float16)0.0f;
            bm[e] = gk < 2 ? (_Float16)mwb[b] : (_Float16)0.0f;
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, bm, acc, 0, 0, 0);
    }
    };

    /* software pipeline, one super-block ahead; the prefetch index is
     * clamped so the loads stay unconditional (the extra load at the end is
     * in bounds and unused) */
    Regs ra, rb;
    if (nmine > 0) {
        load(0, ra);
        store_scales(0, ra);
        for (int i = 0; i < nmine; i += 2) {
            load(min(i + 1, nmine - 1), rb);
            compute(ra, 0);
            store_scales(1, rb);                 /* buffer 1: last read two steps ago */
            if (i + 1 >= nmine) break;
            load(min(i + 2, nmine - 1), ra);
            compute(rb, 1);
            store_scales(0, ra);
        }
    }

    /* waves along K meet in LDS, fixed order */
    if (WGK > 1) {
        if (wk > 0) *(v4f *)&red[wk - 1][wn][lane][0] = acc;
        __syncthreads();
        if (wk == 0) {
#pragma unroll
            for (int u = 1; u < WGK; u++) acc += *(const v4f *)&red[u - 1][wn][lane][0];
        }
    }
    if (wk == 0 && row_ok) {
        float *out = partial ? partial + (size_t)blockIdx.y * M * N : y;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = 4 * gk + r;
            if (t < M) out[(size_t)t * N + row] = acc[r];
        }
    }
}

extern "C" hipError_t sera_launch_splitk_reduce(const float *partial, float *y, size_t n, int splits,
                                                hipStream_t s);
extern "C" int sera_mmq_padded_rows(int M);

/* Split count for the skinny kernel: fill the chip with workgroups, keep at
 * least 2 super-blocks per (split, K-wave). */
extern "C" int sera_skinny_splits(int M, int N, int K) {
    (void)M;
    const int wgs = (N + 15) / 16;   /* WGN = 1, WGK = 4 */
    const int nkb = K / Q4K_QK;
    int s = 1;
    while (wgs * s < 1024 && nkb / (s * 2) >= 8 && s < 8) s *= 2;
    return s;
}

template <int FORM, int WGN, int WGK>
static hipError_t launch_skinny(const uint8_t *W, const int8_t *xq, const void *xsc, float *y, float *partial,
                                int M, int N, int K, int splits, hipStream_t s) {
    const int nkb = K / Q4K_QK;
    const int per = (nkb + splits - 1) / splits;
    dim3 grid((N + 16 * WGN - 1) / (16 * WGN), splits);
    hipLaunchKernelGGL((sera_q4k_skinny_kernel<FORM, WGN, WGK>), grid, dim3(256), 0, s, W, xq, xsc, y,
                       splits > 1 ? partial : nullptr, M, N, K, per);
    return hipGetLastError();
}

/* form 0: row stage (MMVQ formula), form 1: MMQ stage (MMQ formula).
 * partial: splits*M*N floats when splits > 1 (M*N % 4 == 0). */
extern "C" hipError_t sera_launch_q4k_skinny(int form, const void *W, const void *stage, float *y, float *partial,
                                             int M, int N, int K, int splits, hipStream_t s) {
    const char *base = (const char *)stage;
    const uint8_t *w = (const uint8_t *)W;
    hipError_t e;
    if (form == 0) {
        const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
        e = launch_skinny<0, 1, 4>(w, (const int8_t *)(base + L.qs), base + L.dsf, y, partial, M, N, K, splits, s);
    } else {
        const sera_stage_layout L = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K);
        e = launch_skinny<1, 1, 4>(w, (const int8_t *)(base + L.qs), base + L.ds, y, partial, M, N, K, splits, s);
    }
    if (e != hipSuccess || splits <= 1) return e;
    return sera_launch_splitk_reduce(partial, y, (size_t)M * N, splits, s);
}
