/*
 * q6k_mmvq.hip - Q6_K x Q8_1 matrix-vector product for 1..8 tokens (decode).
 *
 * Arithmetic of the reference MMVQ for Q6_K (cuda/mmq/vecdotq.cuh:624-643,
 * 956-980): per group of 16 weights with int8 scale sc_g, the exact integer
 * I_g = sum (q - 32) * q8 (four quants per dp4a), then
 *   y = sum_blk d * sum_g d8[g/2] * (I_g * sc_g)
 * with d8 the fp16 scale of the row-layout Q8_1 activations.
 *
 * A Q6_K super-block is 210 bytes, so blocks (and rows) sit at 2-byte
 * alignment only and no lane can load its fields with aligned 16-byte loads.
 * gfx950 mapping:
 *   - each wave owns R whole weight rows and streams them through its own
 *     LDS double buffer in stages of 8 super-blocks (1680 bytes of a row):
 *     raw bytes go global -> LDS by 16-byte buffer loads to LDS (1 KB per
 *     wave-instruction, no registers, fully coalesced), covering each row's
 *     stage from its 16-byte-aligned start; the next stage streams in while
 *     the wave computes on the current one. No barriers: each wave waits on
 *     its own loads only.
 *   - lane = (block b of the stage, half j, l-quarter): it reads its 8-byte
 *     pieces of ql (two, each giving a low- and a high-nibble quant run),
 *     qh, the 8 group scales of its half and d from LDS as aligned dwords
 *     and funnel-shifts them into place (v_alignbit), builds the raw 6-bit
 *     quants four per dword and runs v_dot4 against its activation slice;
 *     the -32 offset is folded in as -32 * (sum of the 8 activation quants),
 *     computed once per stage and shared by all R rows.
 *   - activation slices (int8 quants and fp16 d8) are loaded once per stage
 *     and reused for the R rows.
 *   - every lane accumulates R x M fp32 partial sums, reduced over the wave
 *     with xor shuffles at the end in a fixed order (deterministic).
 * Bounds: loads go through a buffer resource whose range ends at the end of
 * the weight matrix rounded up to 16 bytes (W must be readable to that
 * boundary, as any hipMalloc allocation is), offsets are vector offsets
 * only, and slots a stage does not need are given an offset past the range
 * (they read zeros, no traffic).
 */
#include "sera_launch.h"

typedef __attribute__((address_space(3))) void q6_lds_void;
typedef unsigned q6_v4u __attribute__((ext_vector_type(4)));
#ifndef SERA_Q6S_ISSUE_ALL_MAX_M
#define SERA_Q6S_ISSUE_ALL_MAX_M 4
#endif

#define Q6K_BLOCK_BYTES 210
#define Q6K_RSRC_FLAGS 0x00020000   /* gfx9 buffer descriptor word 3: 32-bit dword format */

namespace {

constexpr int kStageBlocks = 8;
constexpr int kStageBytes = kStageBlocks * Q6K_BLOCK_BYTES;   /* 1680 = 105 x 16 */
constexpr int kWinChunks = kStageBytes / 16 + 1;              /* 106: a stage at any 16-byte phase */
constexpr int kWin = kWinChunks * 16;                         /* 1696 */
constexpr uint32_t kOutOfRange = 0x80000000u;                 /* past every resource range */

template <int R>
struct Q6Shape {
    static constexpr int SLOTS = R * kWinChunks;   /* 16-byte chunks per stage */
    static constexpr int NI = (SLOTS + 63) / 64;   /* load-to-LDS wave-instructions per stage */
    static constexpr int BUF = NI * 1024;          /* LDS bytes per stage buffer */
};

/* 8 bytes at a 2-byte-aligned LDS byte offset, as two little-endian dwords. */
__device__ __forceinline__ void lds_read8(const uint8_t *lds, uint32_t a, uint32_t &lo, uint32_t &hi) {
    const uint32_t *p = (const uint32_t *)(lds + (a & ~3u));
    const uint32_t sh = (a & 2u) * 8u;
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    lo = __builtin_amdgcn_alignbit(w1, w0, sh);
    hi = __builtin_amdgcn_alignbit(w2, w1, sh);
}

/* int8 field at bit `sh` of w, sign-extended (v_bfe_i32) */
__device__ __forceinline__ int sext8(uint32_t w, int sh) { return (int)(w << (24 - sh)) >> 24; }

__device__ __forceinline__ uint32_t lds_read16(const uint8_t *lds, uint32_t a) {
    return *(const uint16_t *)(lds + a);
}

}  // namespace

/* s_waitcnt immediate for "at most n vector-memory operations outstanding"
 * (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14). */
#define Q6_WAIT_VM(n) (((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

template <int M, int R>
__global__ __launch_bounds__(256) void sera_q6k_mmvq_kernel(
        const uint8_t *__restrict__ W, uint64_t wbytes, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, float *__restrict__ y, int N, int K, int accum) {
    using S = Q6Shape<R>;
    __shared__ __attribute__((aligned(16))) uint8_t s_buf[4][2][S::BUF];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * R;
    if (row0 >= N) return;
    const int nb = K / Q4K_QK;
    const uint64_t rb = (uint64_t)nb * Q6K_BLOCK_BYTES;
    const int nstage = (nb + kStageBlocks - 1) / kStageBlocks;

    /* resource from the wave's first row (16-byte aligned down) to the end
     * of the matrix rounded up to 16 bytes (a chunk that straddles the end
     * must not read as zero); all offsets below are relative to it */
    const uint64_t gbase = ((uint64_t)row0 * rb) & ~(uint64_t)15;
    const uint64_t rem = ((wbytes - gbase) + 15) & ~(uint64_t)15;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(W + gbase), (short)0, (int)(rem > 0x7fffffffu ? 0x7fffffffu : rem), Q6K_RSRC_FLAGS);

    /* phase of each row start within its 16-byte chunk (wave-uniform);
     * rows past N repeat row N-1 and are never stored */
    uint32_t phase[R], rowoff[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint64_t start = (uint64_t)min(row0 + r, N - 1) * rb;
        phase[r] = (uint32_t)(start & 15);
        rowoff[r] = (uint32_t)((start & ~(uint64_t)15) - gbase);
    }
    /* this lane's load slot in each wave-instruction: row sr, chunk sc */
    uint32_t slot_off[S::NI], slot_lim[S::NI];
#pragma unroll
    for (int i = 0; i < S::NI; i++) {
        const int f = 64 * i + lane;
        const int r = f / kWinChunks, c = f - r * kWinChunks;
        const int rc = r < R ? r : 0;
        uint32_t ro = rowoff[0], ph = phase[0];
#pragma unroll
        for (int q = 1; q < R; q++)
            if (rc == q) { ro = rowoff[q]; ph = phase[q]; }
        slot_off[i] = ro + 16u * (uint32_t)c;
        /* chunk c of a row is needed iff 16c < phase + stage bytes; slots past
         * the R windows are never needed */
        slot_lim[i] = f < S::SLOTS ? (ph | ((uint32_t)c << 8)) : 0xffffffffu;
    }

    auto issue = [&](int s, int buf) {
        const uint32_t bytes = (uint32_t)min(kStageBlocks, nb - s * kStageBlocks) * Q6K_BLOCK_BYTES;
#pragma unroll
        for (int i = 0; i < S::NI; i++) {
            const uint32_t ph = slot_lim[i] & 0xffu, c = slot_lim[i] >> 8;
            const bool need = slot_lim[i] != 0xffffffffu && 16u * c < ph + bytes;
            const uint32_t vo = need ? slot_off[i] + (uint32_t)s * kStageBytes : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (q6_lds_void *)&s_buf[wave][buf][1024 * i], 16, vo, 0, 0, 0);
        }
    };

    const int b = lane >> 3;           /* block of the stage */
    const int hh = (lane >> 2) & 1;    /* 128-weight half */
    const int qq = lane & 3;           /* l in [8qq, 8qq + 8) */
    const int jj = qq >> 1;            /* l / 16 */

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < M; t++) acc[r][t] = 0.0f;

    /* activation slices of this lane for stage s: quants of weights
     * 128hh + 32q + 8qq + [0, 8), q = 0..3, of block 8s + b, and the raw
     * (fp16 d8, fp16 sum) words of their Q8_1 blocks. Lanes whose block is
     * past the row end load block 8s and are zeroed through d. */
    struct Act {
        uint32_t xv[M][4][2];
        uint32_t ds[M][4];
    };
    auto load_act = [&](int s, Act &a) {
        const int kb = s * kStageBlocks + b;
        const int kbc = kb < nb ? kb : s * kStageBlocks;
#pragma unroll
        for (int t = 0; t < M; t++) {
            const int8_t *xp = xq + (size_t)t * K + (size_t)kbc * Q4K_QK + 128 * hh + 8 * qq;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint2 v = *(const uint2 *)(xp + 32 * q);
                a.xv[t][q][0] = v.x;
                a.xv[t][q][1] = v.y;
            }
            const uint4 dv = *(const uint4 *)(xds + (size_t)t * (K / 32) + kbc * 8 + 4 * hh);
            a.ds[t][0] = dv.x;
            a.ds[t][1] = dv.y;
            a.ds[t][2] = dv.z;
            a.ds[t][3] = dv.w;
        }
    };

    /* One stage: wait for its loads, read its weight fields of all R rows
     * from LDS, start the next stage's loads (into the other buffer; the
     * reads above precede them), then compute. */
    auto step = [&](int s, int buf, const Act &cur, Act &nxt) {
        const bool active = s * kStageBlocks + b < nb;
        __builtin_amdgcn_s_waitcnt(Q6_WAIT_VM(0));
        const uint8_t *lds = &s_buf[wave][buf][0];
        uint32_t qa[R][2], qb[R][2], qh[R][2], sc[R][2], db[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t base = (uint32_t)(r * kWin) + phase[r] + (uint32_t)(Q6K_BLOCK_BYTES * b);
            lds_read8(lds, base + 64 * hh + 8 * qq, qa[r][0], qa[r][1]);
            lds_read8(lds, base + 64 * hh + 32 + 8 * qq, qb[r][0], qb[r][1]);
            lds_read8(lds, base + 128 + 32 * hh + 8 * qq, qh[r][0], qh[r][1]);
            lds_read8(lds, base + 192 + 8 * hh, sc[r][0], sc[r][1]);
            db[r] = lds_read16(lds, base + 208);
        }
        if (s + 1 < nstage) {
            issue(s + 1, buf ^ 1);
            load_act(s + 1, nxt);
        }
        int corr[M][4];   /* -32 * sum of the slice's 8 quants */
#pragma unroll
        for (int t = 0; t < M; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                corr[t][q] = -__builtin_amdgcn_sdot4((int)cur.xv[t][q][0], 0x20202020,
                                                     __builtin_amdgcn_sdot4((int)cur.xv[t][q][1], 0x20202020, 0,
                                                                            false),
                                                     false);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = active ? h2f_bits(db[r]) : 0.0f;
            /* group scales of quarter q: sc[8hh + 2q + jj] */
            const int scq[4] = {sext8(sc[r][0], 8 * jj), sext8(sc[r][0], 16 + 8 * jj), sext8(sc[r][1], 8 * jj),
                                sext8(sc[r][1], 16 + 8 * jj)};
            /* raw 6-bit quants, four per dword */
            uint32_t v[4][2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                v[0][e] = (qa[r][e] & 0x0F0F0F0Fu) | ((qh[r][e] << 4) & 0x30303030u);
                v[1][e] = (qb[r][e] & 0x0F0F0F0Fu) | ((qh[r][e] << 2) & 0x30303030u);
                v[2][e] = ((qa[r][e] >> 4) & 0x0F0F0F0Fu) | (qh[r][e] & 0x30303030u);
                v[3][e] = ((qb[r][e] >> 4) & 0x0F0F0F0Fu) | ((qh[r][e] >> 2) & 0x30303030u);
            }
#pragma unroll
            for (int t = 0; t < M; t++) {
                float part = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    int I = __builtin_amdgcn_sdot4((int)v[q][0], (int)cur.xv[t][q][0], corr[t][q], false);
                    I = __builtin_amdgcn_sdot4((int)v[q][1], (int)cur.xv[t][q][1], I, false);
                    /* |I| <= 8 * 32 * 127 and |sc| <= 128: a 24-bit multiply is exact */
                    part = fmaf(h2f_bits(cur.ds[t][q] & 0xffffu), (float)__mul24(I, scq[q]), part);
                }
                acc[r][t] = fmaf(d, part, acc[r][t]);
            }
        }
    };

    Act a0, a1;
    issue(0, 0);
    load_act(0, a0);
    for (int s = 0; s < nstage; s += 2) {
        step(s, 0, a0, a1);
        if (s + 1 < nstage) step(s + 1, 1, a1, a0);
    }

    /* wave sums, fixed xor order; lane r*M + t stores (row0 + r, token t) */
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < M; t++) {
            float v = acc[r][t];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == r * M + t) mine = v;
        }
    if (lane < R * M) {
        const int r = lane / M, t = lane - (lane / M) * M;
        if (row0 + r < N) {
            float *dst = y + (size_t)t * N + row0 + r;
            *dst = accum ? *dst + mine : mine;
        }
    }
}

/* ---- split device layout --------------------------------------------------
 * The same product on the split layout (block b's ql, qh, sc at 208*b,
 * 16-byte aligned; d in a separate fp16 array). Every lane field is now an
 * aligned 16-byte load, so the kernel streams straight from HBM into
 * registers, as the Q4_K MMVQ kernel does:
 *   - a quad of lanes takes one block; lane q = (half j = q/2, l-half
 *     lh = q%2) takes weights 128j + 32k + 16lh + [0, 16), k = 0..3: ql
 *     bytes 64j + 16lh + [0, 16) (k = 0, 2) and 64j + 32 + 16lh + [0, 16)
 *     (k = 1, 3), qh bytes 128 + 32j + 16lh + [0, 16), scale bytes
 *     192 + 8j + [0, 8) (its group scales sc[8j + 2k + lh]) and d.
 *   - a wave-load covers 8 consecutive blocks of 2 rows (lanes 32-63 take
 *     the odd row); each lane walks R/2 row pairs with one activation slice
 *     per token (4 x 16 quants, the 4 fp16 d8 of its Q8_1 blocks).
 *   - NW waves split the row's groups of 8 blocks; partial sums meet in LDS
 *     and are added in wave order (deterministic).
 * Arithmetic as above: I_g exact (dot4 of the raw quants minus 32 * the
 * group's activation quant sum), y = sum_blk d * sum_g d8 * (I_g * sc_g).
 * Bounds: rows come from a buffer resource over this tile's rows; the
 * last tile is shifted back to end at row N, and R = 4 needs N >= 4 (the
 * launcher falls back to R = 2, whose odd row sits in the vector offset
 * and reads zeros past N). */
template <int M, int R, int NW>
__global__ __launch_bounds__(NW * 64) void sera_q6s_mmvq_kernel(
        const uint8_t *__restrict__ Wq, const uint16_t *__restrict__ Wd, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, float *__restrict__ y, int N, int K, int accum) {
    constexpr int HR = R / 2;
    static_assert(HR == 1 || HR == 2, "rows per workgroup 2 or 4");
    __shared__ float s_part[NW][R][M];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane & 3, g = (lane >> 2) & 7, rs = lane >> 5;
    const int j = q >> 1, lh = q & 1;
    const int tile0 = blockIdx.x * R;
    const int row0 = tile0 + R > N && N >= R ? N - R : tile0;
    const int nb = K / Q4K_QK;
    const int ngroups = (nb + 7) >> 3;
    const int rowbytes = nb * Q6K_SPLIT_QBYTES;
    const int nrows = min(R, N - row0);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(Wq + (size_t)row0 * rowbytes), (short)0, nrows * rowbytes, Q6K_RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(Wd + (size_t)row0 * nb), (short)0, (nrows * nb * 2 + 3) & ~3, Q6K_RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(xq), (short)0, M * K, Q6K_RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t *>(xds), (short)0, M * (K / 32) * 4, Q6K_RSRC_FLAGS);
    const int vo_w = rs * rowbytes + g * Q6K_SPLIT_QBYTES;
    const int vo_la = vo_w + 64 * j + 16 * lh, vo_lb = vo_la + 32;
    const int vo_qh = vo_w + 128 + 32 * j + 16 * lh, vo_sc = vo_w + 192 + 8 * j;
    const int vo_d = (rs * nb + g) * 2;
    const int vo_x = Q4K_QK * g + 128 * j + 16 * lh;
    const int vo_ds = (8 * g + 4 * j) * 4;

    float acc[HR][M];
#pragma unroll
    for (int r = 0; r < HR; r++)
#pragma unroll
        for (int t = 0; t < M; t++) acc[r][t] = 0.0f;

    for (int bg = wave; bg < ngroups; bg += NW) {
        if (bg * 8 + g >= nb) continue;
        v4i x[M][4];
        q6_v4u ds[M];
#pragma unroll
        for (int t = 0; t < M; t++) {
            const int so = t * K + bg * 8 * Q4K_QK;
#pragma unroll
            for (int k = 0; k < 4; k++)
                x[t][k] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo_x + 32 * k, so, 0));
            ds[t] = __builtin_amdgcn_raw_buffer_load_b128(rf, vo_ds, (t * (K / 32) + bg * 64) * 4, 0);
        }
        q6_v4u la[HR], lb[HR], qh[HR];
        uint32_t sc0[HR], sc1[HR], dd[HR];
#pragma unroll
        for (int r = 0; r < HR; r++) {
            const int so = 2 * r * rowbytes + bg * 8 * Q6K_SPLIT_QBYTES;
            la[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_la, so, 0);
            lb[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_lb, so, 0);
            qh[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_qh, so, 0);
            const uint2 sv = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vo_sc, so, 0));
            sc0[r] = sv.x;
            sc1[r] = sv.y;
            dd[r] = __builtin_amdgcn_raw_buffer_load_b16(rd, vo_d, (2 * r * nb + bg * 8) * 2, 0);
        }
        /* up to 4 tokens every load of the group is in flight before any
         * compute: without this fence the scheduler trades the later loads
         * for registers and the wave waits on HBM several times per group
         * (measured 20-25% slower at 1-4 tokens on down and the LM head) */
        if constexpr (M <= SERA_Q6S_ISSUE_ALL_MAX_M) __builtin_amdgcn_sched_barrier(0);
        /* -32 * (sum of each group's 16 activation quants), shared by the rows */
        int corr[M][4];
#pragma unroll
        for (int t = 0; t < M; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int m32 = (int)0xE0E0E0E0u;   /* four int8 -32 */
                int c = __builtin_amdgcn_sdot4(x[t][k].x, m32, 0, false);
                c = __builtin_amdgcn_sdot4(x[t][k].y, m32, c, false);
                c = __builtin_amdgcn_sdot4(x[t][k].z, m32, c, false);
                corr[t][k] = __builtin_amdgcn_sdot4(x[t][k].w, m32, c, false);
            }
#pragma unroll
        for (int r = 0; r < HR; r++) {
            const uint32_t A[4] = {la[r].x, la[r].y, la[r].z, la[r].w};
            const uint32_t B[4] = {lb[r].x, lb[r].y, lb[r].z, lb[r].w};
            const uint32_t H[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
            /* raw 6-bit quants of quarter k, four per dword (src/q3_quant.c:88-95) */
            uint32_t v[4][4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[0][i] = (A[i] & 0x0F0F0F0Fu) | ((H[i] << 4) & 0x30303030u);
                v[1][i] = (B[i] & 0x0F0F0F0Fu) | ((H[i] << 2) & 0x30303030u);
                v[2][i] = ((A[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u);
                v[3][i] = ((B[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u);
            }
            const int scq[4] = {sext8(sc0[r], 8 * lh), sext8(sc0[r], 16 + 8 * lh), sext8(sc1[r], 8 * lh),
                                sext8(sc1[r], 16 + 8 * lh)};
            const float d = h2f_bits(dd[r] & 0xffffu);
#pragma unroll
            for (int t = 0; t < M; t++) {
                float part = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    int I = __builtin_amdgcn_sdot4((int)v[k][0], x[t][k].x, 0, false);
                    I = __builtin_amdgcn_sdot4((int)v[k][1], x[t][k].y, I, false);
                    I = __builtin_amdgcn_sdot4((int)v[k][2], x[t][k].z, I, false);
                    I = __builtin_amdgcn_sdot4((int)v[k][3], x[t][k].w, I, false);
                    I += corr[t][k];
                    const uint32_t dw = k == 0 ? ds[t].x : k == 1 ? ds[t].y : k == 2 ? ds[t].z : ds[t].w;
                    /* |I| <= 16 * 32 * 127 and |sc| <= 128: a 24-bit multiply is exact */
                    part = fmaf(h2f_bits(dw & 0xffffu), (float)__mul24(I, scq[k]), part);
                }
                acc[r][t] = fmaf(d, part, acc[r][t]);
            }
        }
    }

    /* rows of a lane: row pair r, parity rs. HR = 2: one halving step
     * (lanes with bit 16 keep row pair 1), then xor 8..1; HR = 1: xor 16..1. */
#pragma unroll
    for (int t = 0; t < M; t++) {
        float s;
        int row;
        if constexpr (HR == 2) {
            const bool up = (lane & 16) != 0;
            const float send = up ? acc[0][t] : acc[1][t];
            s = (up ? acc[1][t] : acc[0][t]) + __shfl_xor(send, 16, 64);
            row = 2 * (up ? 1 : 0) + rs;
        } else {
            s = acc[0][t] + __shfl_xor(acc[0][t], 16, 64);
            row = rs;
        }
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
        if ((lane & 15) == 0 && (HR == 2 || (lane & 16) == 0)) s_part[wave][row][t] = s;
    }
    __syncthreads();
    if (threadIdx.x < R * M) {
        const int r = threadIdx.x / M, t = threadIdx.x % M;
        float v = s_part[0][r][t];
#pragma unroll
        for (int w = 1; w < NW; w++) v += s_part[w][r][t];
        if (row0 + r >= tile0 && row0 + r < N) {
            float *dst = y + (size_t)t * N + row0 + r;
            *dst = accum ? *dst + v : v;
        }
    }
}

template <int M, int R>
static hipError_t launch_q6s_mmvq(const uint8_t *Wq, const uint16_t *Wd, const int8_t *xq, const uint32_t *xds,
                                  float *y, int N, int K, int accum, hipStream_t s) {
    const int ngroups = (K / Q4K_QK + 7) / 8;
    const dim3 grid((N + R - 1) / R);
    switch (ngroups >= 4 ? 4 : ngroups) {
        case 1: hipLaunchKernelGGL((sera_q6s_mmvq_kernel<M, R, 1>), grid, dim3(64), 0, s, Wq, Wd, xq, xds, y, N, K,
                                   accum); break;
        case 2: hipLaunchKernelGGL((sera_q6s_mmvq_kernel<M, R, 2>), grid, dim3(128), 0, s, Wq, Wd, xq, xds, y, N,
                                   K, accum); break;
        case 3: hipLaunchKernelGGL((sera_q6s_mmvq_kernel<M, R, 3>), grid, dim3(192), 0, s, Wq, Wd, xq, xds, y, N,
                                   K, accum); break;
        default: hipLaunchKernelGGL((sera_q6s_mmvq_kernel<M, R, 4>), grid, dim3(256), 0, s, Wq, Wd, xq, xds, y, N,
                                    K, accum); break;
    }
    return hipGetLastError();
}

template <int M>
static hipError_t dispatch_q6s_r(int r, const uint8_t *Wq, const uint16_t *Wd, const int8_t *xq,
                                 const uint32_t *xds, float *y, int N, int K, int accum, hipStream_t s) {
    if (r == 4 && N >= 4) return launch_q6s_mmvq<M, 4>(Wq, Wd, xq, xds, y, N, K, accum, s);
    return launch_q6s_mmvq<M, 2>(Wq, Wd, xq, xds, y, N, K, accum, s);
}

template <int M, int R>
static hipError_t launch_q6k_mmvq(const uint8_t *W, uint64_t wbytes, const int8_t *xq, const uint32_t *xds,
                                  float *y, int N, int K, int accum, hipStream_t s) {
    const int waves = (N + R - 1) / R;
    hipLaunchKernelGGL((sera_q6k_mmvq_kernel<M, R>), dim3((waves + 3) / 4), dim3(256), 0, s, W, wbytes, xq, xds,
                       y, N, K, accum);
    return hipGetLastError();
}

/* Rows per wave: 4 where the grid stays well above the chip's wave slots,
 * fewer for short matrices and for 5-8 tokens (register budget). */
extern "C" int sera_q6k_mmvq_rows(int N, int M) {
    if (M > 4) return N >= 4096 ? 2 : 1;
    if (N >= 16384) return 4;
    return N >= 4096 ? 2 : 1;
}

template <int M>
static hipError_t dispatch_q6k_r(int r, const uint8_t *W, uint64_t wbytes, const int8_t *xq,
                                 const uint32_t *xds, float *y, int N, int K, int accum, hipStream_t s) {
    switch (r) {
        case 4: if constexpr (M <= 4) return launch_q6k_mmvq<M, 4>(W, wbytes, xq, xds, y, N, K, accum, s);
                [[fallthrough]];
        case 2: return launch_q6k_mmvq<M, 2>(W, wbytes, xq, xds, y, N, K, accum, s);
        default: return launch_q6k_mmvq<M, 1>(W, wbytes, xq, xds, y, N, K, accum, s);
    }
}

/* Rows per workgroup of the split-layout kernel (2 or 4): 4 measured
 * fastest on MI355X for 1..4 tokens on down (5120 x 25600) and the LM head
 * (151936 x 5120), and equal on v (1024 x 5120); the launcher drops to 2
 * when N < 4. */
extern "C" int sera_q6s_mmvq_rows(int N, int M) {
    (void)N;
    (void)M;
    return 4;
}

/* qtype 14: W is GGUF bytes, rows = rows per wave (1, 2, 4; 0 = built-in).
 * qtype SERA_QTYPE_Q6K_SPLIT: W is the split layout, rows = rows per
 * workgroup (2, 4; 0 = built-in). accum != 0 adds the product to y. */
extern "C" hipError_t sera_launch_q6k_mmvq_acc(uint32_t qtype, const void *W, const void *stage, float *y, int M,
                                               int N, int K, int rows, int accum, hipStream_t s) {
    const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const uint32_t *xds = (const uint32_t *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    const uint64_t nblk = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    if (qtype == SERA_QTYPE_Q6K_SPLIT) {
        const uint16_t *wd = (const uint16_t *)(w + nblk * Q6K_SPLIT_QBYTES);
        if (rows <= 0) rows = sera_q6s_mmvq_rows(N, M);
        switch (M) {
            case 1: return dispatch_q6s_r<1>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 2: return dispatch_q6s_r<2>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 3: return dispatch_q6s_r<3>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 4: return dispatch_q6s_r<4>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 5: return dispatch_q6s_r<5>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 6: return dispatch_q6s_r<6>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 7: return dispatch_q6s_r<7>(rows, w, wd, xq, xds, y, N, K, accum, s);
            case 8: return dispatch_q6s_r<8>(rows, w, wd, xq, xds, y, N, K, accum, s);
            default: return hipErrorInvalidValue;
        }
    }
    const uint64_t wbytes = nblk * Q6K_BLOCK_BYTES;
    if (rows <= 0) rows = sera_q6k_mmvq_rows(N, M);
    switch (M) {
        case 1: return dispatch_q6k_r<1>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 2: return dispatch_q6k_r<2>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 3: return dispatch_q6k_r<3>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 4: return dispatch_q6k_r<4>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 5: return dispatch_q6k_r<5>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 6: return dispatch_q6k_r<6>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 7: return dispatch_q6k_r<7>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        case 8: return dispatch_q6k_r<8>(rows, w, wbytes, xq, xds, y, N, K, accum, s);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t sera_launch_q6k_mmvq(uint32_t qtype, const void *W, const void *stage, float *y, int M, int N,
                                           int K, int rows, hipStream_t s) {
    return sera_launch_q6k_mmvq_acc(qtype, W, stage, y, M, N, K, rows, 0, s);
}
