/*
 * q4k_fewtok.hip - Q4_K x Q8_1 for 1..16 tokens on int8 MFMA: the MMVQ
 * path's kernel from 4 tokens up (MMVQ formula on the row stage) and the
 * MMQ path's kernel up to 16 tokens (MMQ formula on the MMQ stage).
 *
 * Arithmetic, per output and 32-wide sub-block b with I_b the exact int32
 * dot of the sub-block:
 *   MMVQ (cuda/mmq/vecdotq.cuh:505-527,864-908):
 *     y = sum_b (d*sc_b) * d8_b * I_b  -  sum_b (dmin*m_b) * (d8_b*S_b)
 *     with d*sc_b and dmin*m_b exact in fp32, d8_b and d8_b*S_b from the row
 *     stage (dsf);
 *   MMQ (cuda/mmq/mmq.cuh:2269-2283,1440-1472):
 *     y = sum_b fp16(d*sc_b) * d8_b * I_b  +  fp16(-dmin*m_b) * s8_b
 *     with d8_b and s8_b (the fp16 sum of x) from the MMQ stage (ds).
 *
 * gfx950 mapping:
 *   - One v_mfma_i32_16x16x64_i8 computes the int32 dots of TWO sub-blocks
 *     for 8 tokens x 16 weight rows. Its 64-wide K is split in four lane
 *     groups g of 16: groups 0-1 carry sub-block sa, groups 2-3 sub-block
 *     sb. A rows 0-7 are the tokens on sa (zero in groups 2-3), rows 8-15
 *     the tokens on sb (zero in groups 0-1), so result rows 0-7 are I_sa and
 *     rows 8-15 are I_sb: every lane's four results are real dots, and the
 *     fp32 epilogue runs on no padding. 9-16 tokens are two groups of 8
 *     sharing the weight registers.
 *   - Weights are B. Lane (n = lane & 15, g = lane >> 4) owns weight row n
 *     and loads, per super-block, the 16-byte header and the 16-byte pieces
 *     at 16 + 64 j + 16 g (j = 0, 1): nibble bytes of pair 2j + (g >> 1),
 *     half g & 1. Across the wave one load instruction reads 64 contiguous
 *     bytes of each of 16 rows. The low nibbles feed the MFMA of sub-blocks
 *     (4j, 4j+2), the high nibbles (4j+1, 4j+3).
 *   - The min term is a rank-8 fp32 product, two v_mfma_f32_16x16x4_f32 per
 *     super-block and token group into the same accumulator (A = the tokens'
 *     d8*S or s8, zero rows 8-15; B = the row's -dmin*m product).
 *   - Workgroup: NW waves, one 16-row tile each, over one chunk of K. The
 *     chunk's activations (quants with 16-byte columns XOR-swizzled by
 *     token, the two scale factors transposed to [super-block][sub-block]
 *     [token]) are staged in LDS once; after that one barrier each wave runs
 *     on its own, with its next super-block's weights in flight while it
 *     computes the current one.
 *   - gridDim.y > 1 splits K. Each split stores its partial tile with
 *     device-scope (write-through) stores, waits for them and bumps the row
 *     group's counter; the split that completes the count sums all partials
 *     in split order (device-scope loads), stores y and resets the counter.
 *     One launch, no workgroup waits on another, and results repeat bit for
 *     bit.
 */
#include "sera_launch.h"

typedef uint32_t ft_v4u __attribute__((ext_vector_type(4)));
typedef float ft_v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void ft_lds_void;
typedef __attribute__((address_space(1))) const void ft_global_cvoid;

#define SERA_FEWTOK_MAX_TOKENS 16
#define SERA_FEWTOK_LDS_CHUNK_TOKENS 320   /* chunk x staged tokens: 40 super-blocks of 8, 20 of 16 */

/* LDS bytes of a workgroup for `chunk` super-blocks of `tok` staged tokens:
 * quants, d8, the min-term activation factor, and a 16-byte zero operand. */
static inline size_t fewtok_lds_bytes(int chunk, int tok) {
    return (size_t)chunk * tok * (Q4K_QK + 2 * 8 * sizeof(float)) + 16;
}

struct FewtokW {
    ft_v4u hd;      /* d | dmin, 12 scale bytes */
    ft_v4u q[2];    /* nibble bytes at 16 + 64 j + 16 g */
};

/* TG token groups of 8 (M <= 8 TG), FORM 0: MMVQ formula on a row stage
 * (dsf: d8, d8*S as fp32); FORM 1: MMQ formula on an MMQ stage (ds: fp16
 * d8, fp16 sum of x), cuda/mmq/mmq.cuh:2269-2283,1440-1472:
 *   y = sum_b fp16(d*sc_b) * d8_b * I_b + fp16(-dmin*m_b) * s8_b */
template <int NW, int TG, int FORM>
__global__ __launch_bounds__(NW * 64) void sera_q4k_fewtok_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const void *__restrict__ xsc,
        float *__restrict__ y, float *__restrict__ slots, int *__restrict__ counters, int M, int N, int K,
        int chunk, int accum) {
    constexpr int TOK = 8 * TG;                          /* staged tokens */
    extern __shared__ __attribute__((aligned(16))) uint8_t ft_smem[];
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;          /* B column (weight row), A row */
    const int g = lane >> 4;          /* 16-wide K group */
    const int hq = g & 1;
    const int nkb = K / Q4K_QK;
    const int kb0 = blockIdx.y * chunk;
    const int C = min(nkb - kb0, chunk);
    /* LDS: quants [u][t][256] | d8 [u][b][t] | min factor [u][b][t] | zero */
    int8_t *xs = (int8_t *)ft_smem;
    float *d8s = (float *)(ft_smem + (size_t)chunk * TOK * Q4K_QK);
    float *mns = d8s + (size_t)chunk * 8 * TOK;
    uint8_t *zero = (uint8_t *)(mns + (size_t)chunk * 8 * TOK);

    constexpr int RW = 16 * NW;       /* weight rows per workgroup */
    int row = blockIdx.x * RW + 16 * wave + n;
    const bool row_ok = row < N;
    if (!row_ok) row = N - 1;         /* clamp; never stored */
    const uint8_t *wr = W + ((size_t)row * nkb + kb0) * Q4K_BLOCK_BYTES;
    /* super-block u of the chunk; u past the chunk re-reads the last one
     * (its contribution is scaled by zero), so the loop has no branches
     * around loads and the compiler's load counting stays exact */
    auto load = [&](int u, FewtokW &w) {
        const uint8_t *b = wr + (size_t)min(u, C - 1) * Q4K_BLOCK_BYTES;
        w.hd = *(const ft_v4u *)b;
        w.q[0] = *(const ft_v4u *)(b + 16 + 16 * g);
        w.q[1] = *(const ft_v4u *)(b + 80 + 16 * g);
    };
    FewtokW wa, wb;
    load(0, wa);    /* in flight during the activation staging */

    /* --- stage the chunk's activations --- */
    {
        /* quants: 16-byte piece (u, token t, column c) at LDS column c ^ t;
         * one wave-instruction writes 1 KB; tokens past M copy the last */
        const int pieces = C * TOK * 16;
        for (int base = wave * 64; base < pieces; base += NW * 64) {
            const int q = min(base + lane, pieces - 1);
            const int u = q / (TOK * 16), t = (q >> 4) % TOK, col = q & 15;
            const int8_t *src = xq + (size_t)min(t, M - 1) * K + (size_t)(kb0 + u) * Q4K_QK + 16 * (col ^ t);
            __builtin_amdgcn_global_load_lds((ft_global_cvoid *)src, (ft_lds_void *)(xs + (size_t)base * 16), 16, 0, 0);
        }
        /* scales, transposed to [u][sub-block][token]: all loads first, then
         * the LDS writes. FORM 0: float4 (d_2p, d_2p+1, dS_2p, dS_2p+1) per
         * token and sub-block pair; FORM 1: four half2 (d8, s8) per token
         * and sub-block quad. (Four-byte loads straight to LDS, each lane
         * picking its slot's float, measured 1-2% slower for FORM 0.) */
        constexpr int ITEMS = (SERA_FEWTOK_LDS_CHUNK_TOKENS / TOK) * TOK * (FORM == 0 ? 4 : 2);
        constexpr int SCR = (ITEMS + NW * 64 - 1) / (NW * 64);
        const int items = C * TOK * (FORM == 0 ? 4 : 2);
        ft_v4u f[SCR];
#pragma unroll
        for (int r = 0; r < SCR; r++) {
            const int i = min(tid + r * NW * 64, items - 1);
            if (FORM == 0) {
                const int u = i / (TOK * 4), t = (i >> 2) % TOK, p = i & 3;
                f[r] = ((const ft_v4u *)xsc)[(size_t)min(t, M - 1) * (K / 64) + (size_t)(kb0 + u) * 4 + p];
            } else {
                const int u = i / (TOK * 2), t = (i >> 1) % TOK, p = i & 1;
                f[r] = ((const ft_v4u *)xsc)[(size_t)min(t, M - 1) * (K / 128) + (size_t)(kb0 + u) * 2 + p];
            }
        }
#pragma unroll
        for (int r = 0; r < SCR; r++) {
            const int i = tid + r * NW * 64;
            if (i < items) {
                if (FORM == 0) {
                    const int u = i / (TOK * 4), t = (i >> 2) % TOK, p = i & 3;
                    float *d8u = d8s + u * 8 * TOK, *mnu = mns + u * 8 * TOK;
                    d8u[(2 * p) * TOK + t] = __uint_as_float(f[r].x);
                    d8u[(2 * p + 1) * TOK + t] = __uint_as_float(f[r].y);
                    mnu[(2 * p) * TOK + t] = __uint_as_float(f[r].z);
                    mnu[(2 * p + 1) * TOK + t] = __uint_as_float(f[r].w);
                } else {
                    const int u = i / (TOK * 2), t = (i >> 1) % TOK, p = i & 1;
                    float *d8u = d8s + u * 8 * TOK, *mnu = mns + u * 8 * TOK;
                    const uint32_t ds[4] = {f[r].x, f[r].y, f[r].z, f[r].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        d8u[(4 * p + e) * TOK + t] = h2f_bits(ds[e] & 0xffffu);
                        mnu[(4 * p + e) * TOK + t] = h2f_bits(ds[e] >> 16);
                    }
                }
            }
        }
        if (tid == 0) *(ft_v4u *)zero = (ft_v4u){0u, 0u, 0u, 0u};
    }
    __builtin_amdgcn_s_waitcnt(0);    /* this thread's loads to LDS have landed */
    __syncthreads();

    /* A operand offsets: lane (row i = n, group g) is real when (i < 8) ==
     * (g < 2): token 8 tg + (i & 7) on sub-block 4j + 2 (i >> 3) + h, 16
     * bytes at k-half hq; other lanes read the zero operand */
    int aoff[TG][4];
    bool m_real[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
        const int t = 8 * tg + (n & 7);
        const bool a_real = ((n < 8) == (g < 2)) && t < M;
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int sbk = 4 * (jh >> 1) + 2 * (n >> 3) + (jh & 1);
            aoff[tg][jh] = a_real ? t * Q4K_QK + 16 * ((2 * sbk + hq) ^ t) : -1;
        }
        m_real[tg] = n < 8 && 8 * tg + n < M;
    }
    const int sg = g >> 1;            /* result sub-block: 4j + 2 sg + h */
    const int tq = 4 * hq;            /* result tokens 8 tg + tq .. + 3 */
    ft_v4f acc[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[tg] = (ft_v4f){0.f, 0.f, 0.f, 0.f};
    const v4i magic = sera_magic_seed<4>();

    auto compute = [&](int u, const FewtokW &w) {
        const float live = u < C ? 1.0f : 0.0f;
        const int uu = min(u, C - 1);
        const int8_t *xu = xs + (size_t)uu * TOK * Q4K_QK;
        const float *d8u = d8s + uu * 8 * TOK, *mnu = mns + uu * 8 * TOK;
        /* (scale, min) bytes of sub-blocks 0-3 and 4-7 (src/q3_quant.c:44-55) */
        const ft_v4u hd = w.hd;
        const uint32_t sc03 = hd.y & 0x3F3F3F3Fu;
        const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        /* sub-block scale and min products: FORM 0 exact in fp32 (d*sc,
         * -dmin*m); FORM 1 one fp16 rounding each, as the reference's half2
         * store (d, dmin) * (1, -1) * (sc, m) */
        auto scale = [&](uint32_t v) -> float {
            if (FORM == 0) return h2f_bits(hd.x & 0xffffu) * (float)v;
            return (float)((_Float16)v * (_Float16)h2f_bits(hd.x & 0xffffu));
        };
        auto minp = [&](uint32_t v) -> float {
            if (FORM == 0) return -h2f_bits(hd.x >> 16) * (float)v;
            return (float)((_Float16)v * (_Float16)(-h2f_bits(hd.x >> 16)));
        };
        /* min term: lane (n, g) gives A[n][g] and B[g][n] for sub-blocks g
         * and 4 + g (A: FORM 0 d8*S, FORM 1 the fp16 sum of x) */
        const float bm0 = live * minp((m03 >> (8 * g)) & 0xffu);
        const float bm1 = live * minp((m47 >> (8 * g)) & 0xffu);
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const float am0 = m_real[tg] ? mnu[g * TOK + 8 * tg + n] : 0.0f;
            const float am1 = m_real[tg] ? mnu[(4 + g) * TOK + 8 * tg + n] : 0.0f;
            acc[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, bm0, acc[tg], 0, 0, 0);
            acc[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, bm1, acc[tg], 0, 0, 0);
        }
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int j = jh >> 1, h = jh & 1;
            const int sbl = 4 * j + 2 * sg + h;
            const float swb = live * scale(((j ? sc47 : sc03) >> (8 * (2 * sg + h))) & 0xffu);
            const float nswb = -SERA_MAGIC_F * swb;
            const ft_v4u q = w.q[j];
            v4i B;
            B.x = (int)((q.x >> (4 * h)) & 0x0F0F0F0Fu);
            B.y = (int)((q.y >> (4 * h)) & 0x0F0F0F0Fu);
            B.z = (int)((q.z >> (4 * h)) & 0x0F0F0F0Fu);
            B.w = (int)((q.w >> (4 * h)) & 0x0F0F0F0Fu);
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                const v4i A = *(const v4i *)(aoff[tg][jh] >= 0 ? (const void *)(xu + aoff[tg][jh])
                                                               : (const void *)zero);
                const ft_v4f D8 = *(const ft_v4f *)&d8u[sbl * TOK + 8 * tg + tq];
                /* magic-seeded: (I * scale) rounded once, then * d8 into acc */
                const v4i F = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, magic, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[tg][r] = fmaf(scaled_dot(F[r], swb, nswb), D8[r], acc[tg][r]);
            }
        }
    };
    /* One super-block in flight, issued before the current one's compute
     * (the scheduling barriers keep each load group ahead of the compute it
     * overlaps). Measured against two in flight (the next two issued after
     * each compute): 4-6% faster at 4-8 tokens (gate/up 19.6 -> 18.5 us,
     * down 25.3 -> 23.9), equal at 16; deeper prefetch, in groups of 2-5
     * super-blocks or only before the staging, was slower at every size. */
    for (int u0 = 0; u0 < C; u0 += 2) {
        load(u0 + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
        compute(u0, wa);
        __builtin_amdgcn_sched_barrier(0);
        load(u0 + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        compute(u0 + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
    }
    /* lanes g and g ^ 2 hold the two sub-block halves of the same outputs */
#pragma unroll
    for (int tg = 0; tg < TG; tg++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[tg][r] += __shfl_xor(acc[tg][r], 32, 64);
    const bool owner = g < 2 && row_ok;

    if (gridDim.y > 1) {
        /* split K: this split's partial of the tile goes to slots[split][t][row]
         * with device-scope stores, so the hand-off needs no cache-wide fence */
        const int S = gridDim.y;
        if (owner) {
            float *mine = slots + (size_t)blockIdx.y * M * N;
#pragma unroll
            for (int tg = 0; tg < TG; tg++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = 8 * tg + tq + r;
                    if (t < M)
                        __hip_atomic_store(&mine[(size_t)t * N + row], acc[tg][r], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     S - 1;
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (owner) {
#pragma unroll
            for (int tg = 0; tg < TG; tg++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = 8 * tg + tq + r;
                    if (t >= M) continue;
                    const size_t at = (size_t)t * N + row;
                    float v = __hip_atomic_load(&slots[at], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    for (int k = 1; k < S; k++)
                        v += __hip_atomic_load(&slots[(size_t)k * M * N + at], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    acc[tg][r] = v;
                }
        }
    }
    if (owner) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = 8 * tg + tq + r;
                if (t < M) {
                    float *dst = y + (size_t)t * N + row;
                    *dst = accum ? *dst + acc[tg][r] : acc[tg][r];
                }
            }
    }
}

/* Workgroup shape and K chunk for M tokens of an N x K matrix, from sweeps
 * on MI355X over the Qwen3-32B projections (weights streamed from HBM): 8
 * waves (128 rows) for the large matrices, 4 otherwise, and enough K splits
 * to give the chip about 192 (8 waves) or 256 (4 waves) workgroups, with
 * chunks of at least 5 super-blocks (below that the LDS staging dominates)
 * and at most 20. The kernel takes chunks of up to 320 / staged tokens
 * super-blocks (40 for 8 tokens, 20 for 16): up to 100 KB of LDS, one 8-wave
 * workgroup per CU. The 20-block chunk at 16 tokens (one split on gate/up and
 * the LM head) measured 23-24 and 112-120 us against 31-34 and 146-155 us
 * with the earlier 10-block cap and its second split. */
extern "C" void sera_fewtok_plan(int M, int N, int K, int *nwave, int *chunk) {
    const int nw = (N >= 16384 || K >= 16384) ? 8 : 4;
    const int groups = (N + 16 * nw - 1) / (16 * nw);
    const int nkb = K / Q4K_QK;
    /* planned chunks stay within 20 super-blocks, the range measured on the
     * Qwen3-32B shapes; longer ones (up to the LDS limit) only on request */
    const int maxc = 20;
    const int target = nw == 8 ? 192 : 256;
    int s = (target + groups - 1) / groups;
    if (s > 16) s = 16;
    if (s > nkb / 5) s = nkb / 5;   /* chunks of at least 5 super-blocks: staging amortised */
    if (s < 1) s = 1;
    int c = (nkb + s - 1) / s;
    if (c > maxc) c = maxc;   /* more splits when K is long */
    *nwave = nw;
    *chunk = c;
}

/* Largest chunk for M tokens. */
extern "C" int sera_fewtok_max_chunk(int M) { return SERA_FEWTOK_LDS_CHUNK_TOKENS / (M > 8 ? 16 : 8); }

/* Row groups (counters needed when K is split) of the planned launch. */
extern "C" int sera_fewtok_groups(int M, int N, int K) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    return (N + 16 * nw - 1) / (16 * nw);
}

/* Splits of K (grid rows) for a chunk (0 = planned). */
extern "C" int sera_fewtok_splits(int M, int N, int K, int chunk) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    const int nkb = K / Q4K_QK;
    return (nkb + c - 1) / c;
}


template <int NW, int TG, int FORM>
static hipError_t launch_fewtok(const uint8_t *W, const int8_t *xq, const void *xsc, float *y, float *slots,
                                int *counters, int M, int N, int K, int chunk, int accum, hipStream_t s) {
    const int nkb = K / Q4K_QK;
    const int splits = (nkb + chunk - 1) / chunk;
    dim3 grid((N + 16 * NW - 1) / (16 * NW), splits);
    hipLaunchKernelGGL((sera_q4k_fewtok_kernel<NW, TG, FORM>), grid, dim3(NW * 64), fewtok_lds_bytes(chunk, 8 * TG),
                       s, W, xq, xsc, y, slots, counters, M, N, K, chunk, accum);
    return hipGetLastError();
}

template <int TG, int FORM>
static hipError_t launch_fewtok_nw(int nw, const uint8_t *W, const int8_t *xq, const void *xsc, float *y,
                                   float *slots, int *counters, int M, int N, int K, int chunk, int accum,
                                   hipStream_t s) {
    if (nw == 8) return launch_fewtok<8, TG, FORM>(W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, s);
    return launch_fewtok<4, TG, FORM>(W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, s);
}

/* y (+)= X . W^T for 1 <= M <= 16. form 0: row stage, MMVQ formula (M <= 8);
 * form 1: MMQ stage, MMQ formula. chunk: super-blocks per workgroup
 * (1..sera_fewtok_max_chunk(M), 0 = planned); when it splits K, slots holds
 * splits*M*N floats and counters sera_fewtok_groups() ints, zero on entry
 * and zero again after the kernel. */
extern "C" hipError_t sera_launch_q4k_fewtok_acc(int form, const void *W, const void *stage, float *y, float *slots,
                                                 int *counters, int M, int N, int K, int chunk, int accum,
                                                 hipStream_t s) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    if (c > sera_fewtok_max_chunk(M)) return hipErrorInvalidValue;   /* the LDS staging is sized for this */
    const char *base = (const char *)stage;
    const uint8_t *w = (const uint8_t *)W;
    if (form == 0) {
        const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
        return launch_fewtok_nw<1, 0>(nw, w, (const int8_t *)(base + L.qs), base + L.dsf, y, slots, counters, M, N,
                                      K, c, accum, s);
    }
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K);
    if (M > 8)
        return launch_fewtok_nw<2, 1>(nw, w, (const int8_t *)(base + L.qs), base + L.ds, y, slots, counters, M, N, K,
                                      c, accum, s);
    return launch_fewtok_nw<1, 1>(nw, w, (const int8_t *)(base + L.qs), base + L.ds, y, slots, counters, M, N, K, c,
                                  accum, s);
}
