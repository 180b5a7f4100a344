/*
 * q4k_fewtok.hip - Q4_K x Q8_1 for 1..8 tokens on int8 MFMA, the MMVQ path's
 * kernel from 4 tokens up.
 *
 * Arithmetic of the reference MMVQ (cuda/mmq/vecdotq.cuh:505-527,864-908):
 *   y[t][n] = sum_b (d*sc_b) * d8_b * I_b  -  sum_b (dmin*m_b) * (d8_b*S_b)
 * with I_b the exact int32 dot of sub-block b, d*sc_b and dmin*m_b exact in
 * fp32, d8_b and d8_b*S_b from the row stage (dsf).
 *
 * gfx950 mapping:
 *   - One v_mfma_i32_16x16x64_i8 computes the int32 dots of TWO sub-blocks
 *     for 8 tokens x 16 weight rows. Its 64-wide K is split in four lane
 *     groups g of 16: groups 0-1 carry sub-block sa, groups 2-3 sub-block
 *     sb. A rows 0-7 are the tokens on sa (zero in groups 2-3), rows 8-15
 *     the tokens on sb (zero in groups 0-1), so result rows 0-7 are I_sa and
 *     rows 8-15 are I_sb: every lane's four results are real dots, and the
 *     fp32 epilogue runs on no padding.
 *   - Weights are B. Lane (n = lane & 15, g = lane >> 4) owns weight row n
 *     and loads, per super-block, the 16-byte header and the 16-byte pieces
 *     at 16 + 64 j + 16 g (j = 0, 1): nibble bytes of pair 2j + (g >> 1),
 *     half g & 1. Across the wave one load instruction reads 64 contiguous
 *     bytes of each of 16 rows, which streams from HBM as fast as a plain
 *     copy (32-byte pieces per row measured 30% slower). The low nibbles
 *     feed the MFMA of sub-blocks (4j, 4j+2), the high nibbles (4j+1, 4j+3).
 *   - The min term is a rank-8 fp32 product, two v_mfma_f32_16x16x4_f32 per
 *     super-block into the same accumulator (A = d8*S of tokens 0-7, zero
 *     rows 8-15; B = -dmin*m of the row).
 *   - Workgroup: NW waves, one 16-row tile each, over one chunk of K (at
 *     most SERA_FEWTOK_MAX_CHUNK super-blocks). The chunk's activations
 *     (quants with 16-byte columns XOR-swizzled by token, d8 and d8*S
 *     transposed to [super-block][sub-block][token]) are staged in LDS once;
 *     after that one barrier each wave runs on its own, with its next
 *     super-block's weights in flight while it computes the current one.
 *   - gridDim.y > 1 splits K. Each split stores its partial tile with
 *     device-scope (write-through) stores, waits for them and bumps the row
 *     group's counter; the split that completes the count sums all partials
 *     in split order (device-scope loads), stores y and resets the counter.
 *     One launch, no workgroup waits on another, and results repeat bit for
 *     bit.
 */
#include "q4k_common.h"

typedef uint32_t ft_v4u __attribute__((ext_vector_type(4)));
typedef float ft_v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void ft_lds_void;
typedef __attribute__((address_space(1))) const void ft_global_cvoid;

#define SERA_FEWTOK_MAX_TOKENS 8
#define SERA_FEWTOK_MAX_CHUNK 20                      /* super-blocks per workgroup: 51 KB of LDS */
#define SERA_FEWTOK_QS_BYTES (SERA_FEWTOK_MAX_TOKENS * Q4K_QK)   /* quants of one super-block */
#define SERA_FEWTOK_SC_FLOATS (8 * SERA_FEWTOK_MAX_TOKENS)       /* [sub-block][token] */

/* LDS bytes of a workgroup for `chunk` super-blocks: quants, d8, d8*S, and
 * a 16-byte zero operand. */
static inline size_t fewtok_lds_bytes(int chunk) {
    return (size_t)chunk * (SERA_FEWTOK_QS_BYTES + 2 * SERA_FEWTOK_SC_FLOATS * sizeof(float)) + 16;
}

struct FewtokW {
    ft_v4u hd;      /* d | dmin, 12 scale bytes */
    ft_v4u q[2];    /* nibble bytes at 16 + 64 j + 16 g */
};

template <int NW>
__global__ __launch_bounds__(NW * 64) void sera_q4k_fewtok_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const float4 *__restrict__ dsf,
        float *__restrict__ y, float *__restrict__ slots, int *__restrict__ counters, int M, int N, int K,
        int chunk, int accum) {
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
    int8_t *xs = (int8_t *)ft_smem;
    float *d8s = (float *)(ft_smem + (size_t)chunk * SERA_FEWTOK_QS_BYTES);
    float *dSs = d8s + (size_t)chunk * SERA_FEWTOK_SC_FLOATS;
    uint8_t *zero = (uint8_t *)(dSs + (size_t)chunk * SERA_FEWTOK_SC_FLOATS);

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
    FewtokW w0, w1;
    load(0, w0);
    load(1, w1);

    /* --- stage the chunk's activations --- */
    {
        /* quants: 16-byte piece (u, token t, column c) at LDS column c ^ t;
         * one wave-instruction writes 1 KB; tokens past M copy the last */
        const int pieces = C * (SERA_FEWTOK_QS_BYTES / 16);
        for (int base = wave * 64; base < pieces; base += NW * 64) {
            const int q = min(base + lane, pieces - 1);
            const int u = q >> 7, t = (q >> 4) & 7, col = q & 15;
            const int8_t *src = xq + (size_t)min(t, M - 1) * K + (size_t)(kb0 + u) * Q4K_QK + 16 * (col ^ t);
            __builtin_amdgcn_global_load_lds((ft_global_cvoid *)src, (ft_lds_void *)(xs + (size_t)base * 16), 16, 0, 0);
        }
        /* d8 and d8*S: float4 (d_2p, d_2p+1, dS_2p, dS_2p+1) per token and
         * sub-block pair, all loads first, then the transposed LDS writes */
        constexpr int SCR = (SERA_FEWTOK_MAX_CHUNK * 32 + NW * 64 - 1) / (NW * 64);
        float4 f[SCR];
#pragma unroll
        for (int r = 0; r < SCR; r++) {
            const int i = min(tid + r * NW * 64, C * 32 - 1);
            const int u = i >> 5, t = (i >> 2) & 7, p = i & 3;
            f[r] = dsf[(size_t)min(t, M - 1) * (K / 64) + (size_t)(kb0 + u) * 4 + p];
        }
#pragma unroll
        for (int r = 0; r < SCR; r++) {
            const int i = tid + r * NW * 64;
            if (i < C * 32) {
                const int u = i >> 5, t = (i >> 2) & 7, p = i & 3;
                float *d8u = d8s + u * SERA_FEWTOK_SC_FLOATS, *dSu = dSs + u * SERA_FEWTOK_SC_FLOATS;
                d8u[(2 * p) * 8 + t] = f[r].x;
                d8u[(2 * p + 1) * 8 + t] = f[r].y;
                dSu[(2 * p) * 8 + t] = f[r].z;
                dSu[(2 * p + 1) * 8 + t] = f[r].w;
            }
        }
        if (tid == 0) *(ft_v4u *)zero = (ft_v4u){0u, 0u, 0u, 0u};
    }
    __builtin_amdgcn_s_waitcnt(0);    /* this thread's loads to LDS have landed */
    __syncthreads();

    /* A operand offsets: lane (row i = n, group g) is real when (i < 8) ==
     * (g < 2): token i & 7 on sub-block 4j + 2 (i >> 3) + h, 16 bytes at
     * k-half hq; other lanes read the zero operand */
    const int ti = n & 7;
    const bool a_real = ((n < 8) == (g < 2)) && ti < M;
    int aoff[4];
#pragma unroll
    for (int jh = 0; jh < 4; jh++) {
        const int sbk = 4 * (jh >> 1) + 2 * (n >> 3) + (jh & 1);
        aoff[jh] = a_real ? ti * Q4K_QK + 16 * ((2 * sbk + hq) ^ ti) : -1;
    }
    const int sg = g >> 1;            /* result sub-block: 4j + 2 sg + h */
    const int tq = 4 * hq;            /* result tokens tq .. tq + 3 */
    const bool m_real = n < 8 && n < M;
    ft_v4f acc = {0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int u, const FewtokW &w) {
        const float live = u < C ? 1.0f : 0.0f;
        const int uu = min(u, C - 1);
        const int8_t *xu = xs + (size_t)uu * SERA_FEWTOK_QS_BYTES;
        const float *d8u = d8s + uu * SERA_FEWTOK_SC_FLOATS, *dSu = dSs + uu * SERA_FEWTOK_SC_FLOATS;
        v4i A[4];
        ft_v4f D8[4];
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            A[jh] = *(const v4i *)(aoff[jh] >= 0 ? (const void *)(xu + aoff[jh]) : (const void *)zero);
            D8[jh] = *(const ft_v4f *)&d8u[(4 * (jh >> 1) + 2 * sg + (jh & 1)) * 8 + tq];
        }
        const float am0 = m_real ? dSu[g * 8 + n] : 0.0f;
        const float am1 = m_real ? dSu[(4 + g) * 8 + n] : 0.0f;
        /* (scale, min) bytes of sub-blocks 0-3 and 4-7 (src/q3_quant.c:44-55) */
        const ft_v4u hd = w.hd;
        const uint32_t sc03 = hd.y & 0x3F3F3F3Fu;
        const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        const float d = live * h2f_bits(hd.x & 0xffffu);
        const float ndmin = -live * h2f_bits(hd.x >> 16);
        /* min term: lane (n, g) gives A[n][g] and B[g][n] for sub-blocks g
         * and 4 + g */
        const float bm0 = ndmin * (float)((m03 >> (8 * g)) & 0xffu);
        const float bm1 = ndmin * (float)((m47 >> (8 * g)) & 0xffu);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(am0, bm0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(am1, bm1, acc, 0, 0, 0);
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int j = jh >> 1, h = jh & 1;
            const float swb = d * (float)(((j ? sc47 : sc03) >> (8 * (2 * sg + h))) & 0xffu);
            const ft_v4u q = w.q[j];
            v4i B;
            B.x = (int)((q.x >> (4 * h)) & 0x0F0F0F0Fu);
            B.y = (int)((q.y >> (4 * h)) & 0x0F0F0F0Fu);
            B.z = (int)((q.z >> (4 * h)) & 0x0F0F0F0Fu);
            B.w = (int)((q.w >> (4 * h)) & 0x0F0F0F0Fu);
            const v4i I = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[jh], B, (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = fmaf((float)I[r], D8[jh][r] * swb, acc[r]);
        }
    };
    for (int u0 = 0; u0 < C; u0 += 2) {
        compute(u0, w0);
        load(u0 + 2, w0);
        compute(u0 + 1, w1);
        load(u0 + 3, w1);
    }
    /* lanes g and g ^ 2 hold the two sub-block halves of the same outputs */
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] += __shfl_xor(acc[r], 32, 64);
    const bool owner = g < 2 && row_ok;

    if (gridDim.y > 1) {
        /* split K: this split's partial of the tile goes to slots[split][t][row]
         * with device-scope stores, so the hand-off needs no cache-wide fence */
        const int S = gridDim.y;
        if (owner) {
            float *mine = slots + (size_t)blockIdx.y * M * N;
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (tq + r < M)
                    __hip_atomic_store(&mine[(size_t)(tq + r) * N + row], acc[r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
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
            for (int r = 0; r < 4; r++) {
                if (tq + r >= M) continue;
                const size_t at = (size_t)(tq + r) * N + row;
                float v = __hip_atomic_load(&slots[at], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int k = 1; k < S; k++)
                    v += __hip_atomic_load(&slots[(size_t)k * M * N + at], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                acc[r] = v;
            }
        }
    }
    if (owner) {
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (tq + r < M) {
                float *dst = y + (size_t)(tq + r) * N + row;
                *dst = accum ? *dst + acc[r] : acc[r];
            }
    }
}

/* Workgroup shape and K chunk for M tokens of an N x K matrix, from sweeps
 * on MI355X over the Qwen3-32B projections: 8 waves (128 rows) for the
 * large matrices, 4 otherwise, and enough K splits to give the chip about
 * 192 (8 waves) or 256 (4 waves) workgroups. */
extern "C" void sera_fewtok_plan(int M, int N, int K, int *nwave, int *chunk) {
    (void)M;
    const int nw = (N >= 16384 || K >= 16384) ? 8 : 4;
    const int groups = (N + 16 * nw - 1) / (16 * nw);
    const int nkb = K / Q4K_QK;
    const int target = nw == 8 ? 192 : 256;
    int s = (target + groups - 1) / groups;
    if (s > 16) s = 16;
    if (s > nkb) s = nkb;
    if (s < 1) s = 1;
    int c = (nkb + s - 1) / s;
    if (c > SERA_FEWTOK_MAX_CHUNK) c = SERA_FEWTOK_MAX_CHUNK;   /* more splits when K is long */
    *nwave = nw;
    *chunk = c;
}

/* Row groups (counters needed when K is split) of the planned launch. */
extern "C" int sera_fewtok_groups(int M, int N, int K) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    return (N + 16 * nw - 1) / (16 * nw);
}

template <int NW>
static hipError_t launch_fewtok(const uint8_t *W, const int8_t *xq, const float4 *dsf, float *y, float *slots,
                                int *counters, int M, int N, int K, int chunk, int accum, hipStream_t s) {
    const int nkb = K / Q4K_QK;
    const int splits = (nkb + chunk - 1) / chunk;
    dim3 grid((N + 16 * NW - 1) / (16 * NW), splits);
    hipLaunchKernelGGL((sera_q4k_fewtok_kernel<NW>), grid, dim3(NW * 64), fewtok_lds_bytes(chunk), s, W, xq, dsf, y,
                       slots, counters, M, N, K, chunk, accum);
    return hipGetLastError();
}

/* Splits of K (grid rows) for a chunk (0 = planned). */
extern "C" int sera_fewtok_splits(int M, int N, int K, int chunk) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    const int nkb = K / Q4K_QK;
    return (nkb + c - 1) / c;
}

/* y (+)= X . W^T for 1 <= M <= 8 on a row stage. chunk: super-blocks per
 * workgroup (1..SERA_FEWTOK_MAX_CHUNK, 0 = planned); when it splits K,
 * slots holds splits*M*N floats and counters sera_fewtok_groups() ints,
 * zero on entry and zero again after the kernel. */
extern "C" hipError_t sera_launch_q4k_fewtok_acc(const void *W, const void *stage, float *y, float *slots,
                                                 int *counters, int M, int N, int K, int chunk, int accum,
                                                 hipStream_t s) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const float4 *dsf = (const float4 *)(base + L.dsf);
    const uint8_t *w = (const uint8_t *)W;
    if (nw == 8) return launch_fewtok<8>(w, xq, dsf, y, slots, counters, M, N, K, c, accum, s);
    return launch_fewtok<4>(w, xq, dsf, y, slots, counters, M, N, K, c, accum, s);
}
