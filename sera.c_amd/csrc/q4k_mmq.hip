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
 *   - v_mfma_i32_32x32x32_i8: one instruction is one 32-wide sub-block of a
 *     32 token x 32 weight-row tile, i.e. the exact int32 I_b. Activations
 *     are the A operand (MFMA rows = tokens), weights the B operand (MFMA
 *     columns = weight rows), so in the 32x32 result each lane owns one
 *     weight row: its sub-block scale fp16(d*sc_b) is a per-lane value the
 *     lane decodes from the block header it loaded itself, and the token
 *     scales d8 come from LDS as float4s.
 *   - the fp32 epilogue is two VALU ops per element and sub-block, with no
 *     int-to-float convert: the MFMA's int32 accumulator starts at the bit
 *     pattern of 1.5 * 2^23, so its result, read as a float, is exactly
 *     1.5 * 2^23 + I (|I| <= 32*15*127 < 2^22 keeps the exponent fixed);
 *     t = fma(F, sw, -1.5 * 2^23 * sw) is then I * sw rounded once (the
 *     offset product is exact: sw is an fp16 value), and acc = fma(t, d8,
 *     acc). This rounds each term twice where the reference rounds it once:
 *     the reference's sw * d8 is exact (two fp16 values), and its
 *     fma(sw * d8, I, sum) rounds only into the sum. Here I * sw is rounded
 *     to fp32 first (relative error at most 2^-24 per term) and then
 *     accumulated, so per-term results do not follow the reference's single
 *     rounding; they are exact whenever I * sw fits 24 bits (integer-exact
 *     inputs), and otherwise differ by about 2^-24 of the term.
 *   - the min term is a plain matrix product over the sub-block index,
 *     [tokens x 8] fp16 s8 times [8 x rows] fp16(-dmin*m_b), done once per
 *     super-block by one v_mfma_f32_32x32x16_f16 accumulating into the same
 *     fp32 tile (fp16 x fp16 products are exact in fp32).
 *   - activations (int8 quants, d8, s8) for the workgroup's tokens are
 *     staged in LDS, double buffered per 256-wide K step, rows padded to
 *     272 bytes so 16 consecutive tokens' 16-byte reads hit distinct banks.
 *     Weights are not staged: each lane loads its row's 16-byte nibble
 *     pieces straight into registers (16 consecutive int8 of one row is the
 *     B operand) and unpacks them in registers; one piece feeds the two
 *     sub-blocks that share it.
 *   - output stores: lanes 0-31 of a half-wave write 32 consecutive
 *     features of one token (coalesced 128-byte rows).
 *   - the tile index is remapped so that the workgroups one XCD runs share
 *     weight rows (token tiles vary fastest within an XCD's range).
 *   - split-K: with few tiles, gridDim.y > 1 splits the super-blocks; each
 *     split writes fp32 partials that a second kernel sums in a fixed order
 *     (deterministic, no atomics).
 */
#include "sera_launch.h"

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_cvoid_t;

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int BM, int PR>
struct alignas(16) MmqSmem {
    /* int8 quants of one 256-wide K step; the 16-byte piece c of token t
     * sits in column c ^ (t & 15), so 16 consecutive tokens reading the same
     * piece hit 16 different bank groups */
    alignas(16) int8_t xs[2][BM][Q4K_QK];
    /* d8 per [sub-block][token]: the paired tile keeps it as float; the
     * 32-row tiles keep the fp16 value itself, each 32-token group in the
     * order of the MFMA result rows a lane holds (token 8q + 4h + i at
     * 16h + 4q + i), so a lane's 16 scales are one 32-byte run */
    alignas(16) float d8[PR ? 2 : 1][8][PR ? BM : 4];
    alignas(16) _Float16 d8h[PR ? 1 : 2][8][PR ? 8 : BM];
    alignas(16) _Float16 s8[2][BM][8];       /* fp16 s8, [token][sub-block] */
    alignas(16) _Float16 zero8[8];           /* a zero min-term operand */
};

/* acc = fma(t, d8, acc) with d8 the low (HI = 0) or high half of a packed
 * fp16 pair: v_fma_mix_f32 converts the half exactly and rounds once, as
 * v_fma_f32 on the converted value would. Written with the accumulator
 * tied to the destination; left to itself the register allocator gives
 * each result a new register and copies the accumulators back per step. */
template <int HI>
__device__ __forceinline__ void fma_acc_f16(float &acc, float t, uint32_t d8pair) {
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(t), "v"(d8pair));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(t), "v"(d8pair));
}

/* Position of token tok in a 32-token group of MmqSmem::d8h. */
__device__ __forceinline__ int mmq_d8h_pos(int tok) {
    return (tok & ~31) + 16 * ((tok >> 2) & 1) + 4 * ((tok >> 3) & 3) + (tok & 3);
}

__device__ __forceinline__ v16i magic_seed() { return sera_magic_seed<16>(); }

/* Tile order: consecutive workgroup ids go to consecutive XCDs (8 on
 * MI355X). Give each XCD a contiguous run of tiles, token tiles fastest,
 * so the workgroups resident on one XCD reuse the same weight rows in L2. */
__device__ __forceinline__ int mmq_tile_of(int wg, int ntiles) {
    const int nx = 8;
    const int full = (ntiles / nx) * nx;
    if (wg >= full) return wg;
    const int per = ntiles / nx;
    return (wg % nx) * per + wg / nx;
}

__device__ __forceinline__ v4i unpack_nib(v4u q, int hi) {
    const int s = hi ? 4 : 0;
    v4i a;
    a.x = (int)((q.x >> s) & 0x0F0F0F0Fu);
    a.y = (int)((q.y >> s) & 0x0F0F0F0Fu);
    a.z = (int)((q.z >> s) & 0x0F0F0F0Fu);
    a.w = (int)((q.w >> s) & 0x0F0F0F0Fu);
    return a;
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 as_h2(uint32_t u) {
    union { uint32_t u; h2 h; } c;
    c.u = u;
    return c.h;
}

/* The eight (scale, min) pairs of a Q4_K header (dwords: d|dmin, then the
 * 12 scale bytes), as fp16 products sw[p] = (fp16(d*sc_2p), fp16(d*sc_2p+1))
 * and mw[p] = (fp16(-dmin*m_2p), fp16(-dmin*m_2p+1)), each a single
 * round-to-nearest-even rounding of the exact product as in the
 * reference's half2 scale store (cuda/mmq/mmq.cuh:2269-2283). The 6-bit
 * fields are unpacked four at a time (src/q3_quant.c:44-55); a byte v < 64
 * becomes the fp16 1024 + v by placing it under the exponent byte 0x64,
 * and subtracting 1024 is exact. */
__device__ __forceinline__ void q4k_scales_f16(v4u hd, h2 sw[4], h2 mw[4]) {
    const uint32_t sc03 = hd.y & 0x3F3F3F3Fu;
    const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
    const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 dd = as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x01000100u));       /* (d, d) */
    const h2 nm = -as_h2(__builtin_amdgcn_perm(hd.x, hd.x, 0x03020302u));      /* (-dmin, -dmin) */
    const uint32_t srcs[4] = {sc03, sc47, m03, m47};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 lo = as_h2(__builtin_amdgcn_perm(0x64646464u, srcs[i], 0x04010400u)) - bias;
        const h2 hi = as_h2(__builtin_amdgcn_perm(0x64646464u, srcs[i], 0x04030402u)) - bias;
        if (i < 2) { sw[2 * i] = lo * dd; sw[2 * i + 1] = hi * dd; }
        else       { mw[2 * (i - 2)] = lo * nm; mw[2 * (i - 2) + 1] = hi * nm; }
    }
}

/* PR = 1 is the paired 16-token tile (TT = WGT = 1): the 32 MFMA rows are
 * the 16 tokens twice, rows 0-15 on sub-block 2p and rows 16-31 on
 * sub-block 2p + 1, so the fp32 epilogue runs on no padding rows. */
template <int TT, int WGT, int WGN, int PR = 0>
struct MmqShape {
    static_assert(PR == 0 || (TT == 1 && WGT == 1), "the paired tile is one 32-row MFMA tile per wave");
    static constexpr int BMW = PR ? 16 : 32 * TT;  /* tokens per wave */
    static constexpr int BM = BMW * WGT;    /* tokens per workgroup */
    static constexpr int BN = 64 * WGN;     /* weight rows per workgroup */
    static constexpr int NACC = TT * 2 * 16; /* accumulator floats per lane */
};

/* One output tile (tokens m0.., weight rows n0..) over super-blocks
 * [kb_begin, kb_end): TT token tiles (of 32) per wave, WGT x WGN waves
 * (along tokens x rows), two 32-row weight tiles per wave. Starts and ends
 * with all threads past a barrier, so consecutive calls may restage.
 *
 * Paired tile (PR = 1, 16 tokens): for sub-blocks sa = 2p, sb = 2p + 1 two
 * MFMAs accumulate in int32. Lane (l32, h) holds the 16 nibble bytes
 * [16h, 16h + 16) of pair p of weight row l32. The first MFMA takes its
 * nibble plane h (k-half h of the B operand: sa's k 0-15 for h = 0, sb's
 * k 16-31 for h = 1), the second the other plane (sb's k 0-15, sa's k
 * 16-31). A row l32 (token l32 & 15 on sub-block 2p + (l32 >> 4)) is real
 * in k-half h exactly when its slice matches: in the first MFMA when
 * h == l32 >> 4, in the second otherwise, always reading the token's bytes
 * [16h, 16h + 16) of its sub-block; the other half is zero. Result rows
 * 0-15 are I_sa, rows 16-31 I_sb. */
template <int TT, int WGT, int WGN, int PR = 0, bool AHEAD = false>
__device__ __forceinline__ void mmq_segment(
        MmqSmem<MmqShape<TT, WGT, WGN, PR>::BM, PR> &sm, const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, int N, int K, int m0, int n0, int kb_begin, int kb_end,
        v16f (&acc)[TT][2], int tiled) {
    using S = MmqShape<TT, WGT, WGN, PR>;
    constexpr int BMW = S::BMW, BM = S::BM;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int h = lane >> 5;
    const int wt = wave % WGT;
    const int wn = wave / WGT;
    const int nkb_total = K / Q4K_QK;
    const int nkb = kb_end - kb_begin;

    /* the two weight rows this lane feeds as B operand (column l32) */
    const uint8_t *wbase[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        int row = n0 + 64 * wn + 32 * nt + l32;
        if (row > N - 1) row = N - 1;          /* clamp; rows >= N are never stored */
        wbase[nt] = W + q4k_block_offset(tiled, row, 0, nkb_total);
    }
    const int bstride = q4k_block_stride(tiled);   /* super-block to super-block of one row */

    /* --- activation staging: BM tokens x 256 int8 go global -> LDS directly
     * (16-byte loads to LDS, one KB per wave-instruction, XOR-swizzled
     * columns); d8 and s8 go through registers (fp16 -> fp32 for d8) --- */
    constexpr int XCH = BM * 16 / 256;         /* 16-byte pieces per thread */
    auto issue_x = [&](int kb, int buf) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int inst = wave + 4 * i;        /* wave-instruction index: 64 pieces each */
            const int c = inst * 64 + lane;       /* LDS piece: token c/16, column c%16 */
            const int tok = c >> 4, col = c & 15;
            /* 32-bit offset (Mpad*K < 2^31): the stream-K loop would otherwise
             * keep four 64-bit per-lane bases live across segments and spill */
            const int8_t *src = xq + (uint32_t)((m0 + tok) * K + kb * Q4K_QK + 16 * (col ^ (tok & 15)));
            __builtin_amdgcn_global_load_lds((global_cvoid_t *)src, (lds_void_t *)&sm.xs[buf][0][inst * 1024], 16, 0, 0);
        }
    };
    auto load_x = [&](int kb, v4u &dr) {
        if (tid < BM * 2) {
            const int tok = tid >> 1, part = tid & 1;
            dr = *(const v4u *)(xds + (size_t)(m0 + tok) * (K / 32) + kb * 8 + 4 * part);
        }
    };
    auto store_x = [&](int buf, const v4u &dr) {
        if (tid < BM * 2) {
            const int tok = tid >> 1, part = tid & 1;
            const uint32_t dw[4] = {dr.x, dr.y, dr.z, dr.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                union { uint16_t u; _Float16 f; } cv;
                if constexpr (PR) {
                    sm.d8[buf][4 * part + e][tok] = h2f_bits(dw[e] & 0xffffu);
                } else {
                    cv.u = (uint16_t)(dw[e] & 0xffffu);
                    sm.d8h[buf][4 * part + e][mmq_d8h_pos(tok)] = cv.f;
                }
                cv.u = (uint16_t)(dw[e] >> 16);
                sm.s8[buf][tok][4 * part + e] = cv.f;
            }
        }
    };
    /* --- weights: header + 4 qs pieces of 16 bytes per weight tile --- */
    auto load_w = [&](int kb, v4u *hdr, v4u (*q)[4]) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const uint8_t *b = wbase[nt] + (size_t)kb * bstride;
            hdr[nt] = *(const v4u *)b;
#pragma unroll
            for (int j2 = 0; j2 < 4; j2++) q[nt][j2] = *(const v4u *)(b + 16 + 32 * j2 + 16 * h);
        }
    };
    auto load_hdr = [&](int kb, v4u *hdr) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++) hdr[nt] = *(const v4u *)(wbase[nt] + (size_t)kb * bstride);
    };
    auto load_piece = [&](int kb, int j2, v4u *q) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            q[nt] = *(const v4u *)(wbase[nt] + (size_t)kb * bstride + 16 + 32 * j2 + 16 * h);
    };

#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][nt][r] = 0.0f;

    const v16i magic = magic_seed();
    v4u dr = {};
    v4u hdr[2] = {}, qw[2][4];
    /* AHEAD (one token tile per wave at 2 waves per SIMD leaves registers for
     * a second weight set): the next step's weights are issued before this
     * step's compute, so their latency hides behind it instead of behind the
     * step's barrier. */
    constexpr bool kWeightsAhead = AHEAD;
    v4u hdrn[2] = {}, qwn[2][4];
    /* Otherwise (PR = 0) the next step's weights come in piece by piece as
     * this step frees their registers: its header as soon as the scales are
     * decoded, piece 0 into a spare set at once, piece j2 + 1 into the
     * registers of piece j2 when sub-block 2 * j2 + 2 starts (pieces j2 feed
     * sub-blocks 2 * j2 and 2 * j2 + 1). Every load then has at least two
     * sub-blocks of compute to land in; the sets rotate at the step's end. */
    constexpr bool kProgressive = !AHEAD && !PR;
    v4u spare[2] = {};

    /* zero8 is the min-term A operand of the lanes (h = 1) whose k
     * positions carry no sub-block */
    if (tid == 0) *(v4u *)&sm.zero8[0] = (v4u){0u, 0u, 0u, 0u};
    if (nkb > 0) {
        issue_x(kb_begin, 0);
        load_x(kb_begin, dr);
        store_x(0, dr);
        load_w(kb_begin, hdr, qw);
    }
    __builtin_amdgcn_s_waitcnt(0);   /* this thread's loads to LDS have landed */
    __syncthreads();

    for (int it = 0; it < nkb; it++) {
        const int buf = it & 1;
        const bool more = it + 1 < nkb;
        if (more) {
            issue_x(kb_begin + it + 1, buf ^ 1);   /* buffer last read one step ago, freed by the barrier */
            load_x(kb_begin + it + 1, dr);
            if constexpr (kWeightsAhead) load_w(kb_begin + it + 1, hdrn, qwn);
        }

        /* per weight tile: fp16(d*sc_b) as fp32 for the epilogue and the
         * min-term B operand fp16(-dmin*m_b), b = 0..7 */
        h2 sw[2][4];
        v8h bmin[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            h2 mw[4];
            q4k_scales_f16(hdr[nt], sw[nt], mw);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                bmin[nt][2 * p] = mw[p].x;
                bmin[nt][2 * p + 1] = mw[p].y;
            }
        }
        /* min term of this super-block: one f16 MFMA per (token tile,
         * weight tile), after the sub-blocks */
        auto min_term = [&]() {
#pragma unroll
            for (int t = 0; t < TT; t++) {
                /* paired tile: the min term goes to rows 0-15 only (each token once) */
                const int tok = PR ? (l32 & 15) : BMW * wt + 32 * t + l32;
                const bool none = h || (PR && l32 >= 16);
                const v8h as8 =
                    *(const v8h *)(none ? (const void *)&sm.zero8[0] : (const void *)&sm.s8[buf][tok][0]);
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    acc[t][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as8, bmin[nt], acc[t][nt], 0, 0, 0);
            }
        };
        /* the next step's super-block; the last step reloads its own (in
         * bounds, unused), which keeps the prefetch free of branches */
        const int kb_next = more ? kb_begin + it + 1 : kb_begin + it;
        if constexpr (kProgressive) {
            load_hdr(kb_next, hdr);
            load_piece(kb_next, 0, spare);
        }

        if constexpr (PR) {
            const int sh = l32 >> 4;            /* this A row's sub-block of the pair */
            const int t = l32 & 15;             /* this A row's token */
#pragma unroll
            for (int p = 0; p < 4; p++) {
                v4i B0[2], B1[2];
                float swa[2], swbb[2], nswa[2], nswbb[2];
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    B0[nt] = unpack_nib(qw[nt][p], h);
                    B1[nt] = unpack_nib(qw[nt][p], 1 - h);
                    swa[nt] = (float)sw[nt][p].x;
                    swbb[nt] = (float)sw[nt][p].y;
                    nswa[nt] = -SERA_MAGIC_F * swa[nt];
                    nswbb[nt] = -SERA_MAGIC_F * swbb[nt];
                }
                const void *real = &sm.xs[buf][t][16 * ((4 * p + 2 * sh + h) ^ t)];
                const v4i A0 = *(const v4i *)(h == sh ? real : (const void *)&sm.zero8[0]);
                const v4i A1 = *(const v4i *)(h != sh ? real : (const void *)&sm.zero8[0]);
                float d8v[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4f f4 = *(const v4f *)&sm.d8[buf][2 * p + (q >> 1)][8 * (q & 1) + 4 * h];
                    d8v[4 * q] = f4.x; d8v[4 * q + 1] = f4.y; d8v[4 * q + 2] = f4.z; d8v[4 * q + 3] = f4.w;
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    v16i F = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B0[nt], magic, 0, 0, 0);
                    F = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B1[nt], F, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float t = r < 8 ? scaled_dot(F[r], swa[nt], nswa[nt])
                                              : scaled_dot(F[r], swbb[nt], nswbb[nt]);
                        acc[0][nt][r] = fmaf(t, d8v[r], acc[0][nt][r]);
                    }
                }
            }
        }
        if constexpr (!PR) {
            /* The 16 * TT MFMAs of the step in order (sub-block b, token tile
             * t, weight tile nt; nt fastest), software pipelined: MFMA i + 1
             * is issued before the epilogue of MFMA i, so the matrix unit
             * runs while the VALU consumes the previous result. */
            constexpr int NI = 8 * TT * 2;
            auto a_of = [&](int b, int t) -> v4i {
                const int tok = BMW * wt + 32 * t + l32;
                return *(const v4i *)&sm.xs[buf][tok][16 * ((2 * b + h) ^ (tok & 15))];
            };
            auto mfma_of = [&](int i) -> v16i {
                const int b = i / (2 * TT), t = (i >> 1) % TT, nt = i & 1;
                return __builtin_amdgcn_mfma_i32_32x32x32_i8(a_of(b, t), unpack_nib(qw[nt][b >> 1], b & 1), magic, 0,
                                                             0, 0);
            };
            v16i Fc = mfma_of(0);
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int b = i / (2 * TT), t = (i >> 1) % TT, nt = i & 1;
                if constexpr (kProgressive) {
                    if (i % (2 * TT) == 0 && b >= 2 && (b & 1) == 0) {
                        v4u nq[2];
                        load_piece(kb_next, b >> 1, nq);
                        qw[0][(b >> 1) - 1] = nq[0];
                        qw[1][(b >> 1) - 1] = nq[1];
                    }
                }
                v16i Fn = {};
                if (i + 1 < NI) Fn = mfma_of(i + 1);
                const float swb = (float)((b & 1) ? sw[nt][b >> 1].y : sw[nt][b >> 1].x);
                const float nswb = -SERA_MAGIC_F * swb;
                /* the lane's 16 token scales (fp16, exact as float): one
                 * 32-byte run; v_fma_mix takes each half as it is */
                const _Float16 *d8p = &sm.d8h[buf][b][BMW * wt + 32 * t + 16 * h];
                const v4u d8lo = *(const v4u *)d8p, d8hi = *(const v4u *)(d8p + 8);
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const uint32_t pair = r < 8 ? d8lo[r / 2] : d8hi[r / 2 - 4];
                    float a0 = acc[t][nt][r], a1 = acc[t][nt][r + 1];
                    fma_acc_f16<0>(a0, scaled_dot(Fc[r], swb, nswb), pair);
                    fma_acc_f16<1>(a1, scaled_dot(Fc[r + 1], swb, nswb), pair);
                    acc[t][nt][r] = a0;
                    acc[t][nt][r + 1] = a1;
                }
                Fc = Fn;
            }
        }
        min_term();
        if (more) {
            if constexpr (!kWeightsAhead && !kProgressive) load_w(kb_begin + it + 1, hdr, qw);
            store_x(buf ^ 1, dr);
        }
        __builtin_amdgcn_s_waitcnt(0);   /* this thread's loads to LDS have landed */
        __syncthreads();
        if constexpr (kWeightsAhead) {
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                hdr[nt] = hdrn[nt];
#pragma unroll
                for (int j2 = 0; j2 < 4; j2++) qw[nt][j2] = qwn[nt][j2];
            }
        }
        if constexpr (kProgressive) {
            /* pieces 1-3 of the next step sit in the sets of pieces 0-2 */
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                qw[nt][3] = qw[nt][2];
                qw[nt][2] = qw[nt][1];
                qw[nt][1] = qw[nt][0];
                qw[nt][0] = spare[nt];
            }
        }
    }
}

/* Store an output tile: lane holds weight row n0+64*wn+32*nt+l32 for tokens
 * m0+BMW*wt+32*t + 8*(r/4) + 4*h + r%4 (paired tile: r < 8, the sum of the
 * even and odd sub-block rows r and r + 8). */
template <int TT, int WGT, int WGN, int PR = 0>
__device__ __forceinline__ void mmq_store(float *__restrict__ out, int M, int N, int m0, int n0,
                                          const v16f (&acc)[TT][2], int accum) {
    constexpr int BMW = MmqShape<TT, WGT, WGN, PR>::BMW;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wt = wave % WGT, wn = wave / WGT;
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int n = n0 + 64 * wn + 32 * nt + l32;
        if (n >= N) continue;
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < (PR ? 8 : 16); r++) {
                const int m = m0 + BMW * wt + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                const float v = PR ? acc[t][nt][r] + acc[t][nt][r + 8] : acc[t][nt][r];
                if (m < M) {
                    float *dst = out + (size_t)m * N + n;
                    *dst = accum ? *dst + v : v;
                }
            }
    }
}

/* Grid over (tile, K split); splits > 1 write fp32 partials per split.
 * WPE: waves per SIMD the register budget is cut for. */
template <int TT, int WGT, int WGN, int WPE = 2, int PR = 0>
__global__ __launch_bounds__(256, WPE) void sera_q4k_mmq_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, float *__restrict__ y, float *__restrict__ partial,
        int M, int N, int K, int kb_per_split, int accum, int tiled) {
    static_assert(WGT * WGN == 4, "4 waves per workgroup");
    using S = MmqShape<TT, WGT, WGN, PR>;
    __shared__ __attribute__((aligned(16))) MmqSmem<S::BM, PR> sm;
    const int ntt = (M + S::BM - 1) / S::BM;
    const int nrt = (N + S::BN - 1) / S::BN;
    const int tile = mmq_tile_of(blockIdx.x, ntt * nrt);
    const int n0 = (tile / ntt) * S::BN;
    const int m0 = (tile % ntt) * S::BM;
    const int nkb_total = K / Q4K_QK;
    const int kb_begin = blockIdx.y * kb_per_split;
    const int kb_end = min(nkb_total, kb_begin + kb_per_split);
    v16f acc[TT][2];
    mmq_segment<TT, WGT, WGN, PR, TT == 1 && WPE <= 2>(sm, W, xq, xds, N, K, m0, n0, kb_begin, kb_end, acc, tiled);
    float *out = partial ? partial + (size_t)blockIdx.y * M * N : y;
    mmq_store<TT, WGT, WGN, PR>(out, M, N, m0, n0, acc, partial ? 0 : accum);
}

/* Stream-K schedule: P persistent workgroups split the ntiles x nkb
 * (tile, super-block) units evenly, so the last round of tiles does not
 * leave workgroup slots idle. Workgroup w owns units [w*U/P, (w+1)*U/P)
 * and walks them in order; a tile whose units are not all its own is a
 * split tile. Each contributor of a split tile writes its accumulators to
 * its own slot, then bumps the tile's counter; the contributor that brings
 * the counter to the contributor count sums all slots in contributor order
 * (deterministic), stores the tile and resets the counter to zero for the
 * next call. No workgroup ever waits on another. Logical ids are remapped
 * so each XCD runs a contiguous range of units (the tiles sharing weight
 * rows meet in one L2). */
__device__ __forceinline__ int64_t sk_u0(int w, int64_t U, int P) { return (int64_t)w * U / P; }
__device__ __forceinline__ int sk_owner(int64_t u, int64_t U, int P) { return (int)(((u + 1) * P - 1) / U); }

template <int TT, int WGT, int WGN, int WPE = 2, int PR = 0>
__global__ __launch_bounds__(256, WPE) void sera_q4k_mmq_streamk_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq,
        const uint32_t *__restrict__ xds, float *__restrict__ y, float *__restrict__ slots,
        int *__restrict__ counters, int M, int N, int K, int accum, int tiled) {
    static_assert(WGT * WGN == 4, "4 waves per workgroup");
    using S = MmqShape<TT, WGT, WGN, PR>;
    __shared__ __attribute__((aligned(16))) MmqSmem<S::BM, PR> sm;
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int P = gridDim.x;                       /* multiple of 8 */
    const int w = (blockIdx.x & 7) * (P >> 3) + (blockIdx.x >> 3);
    const int ntt = (M + S::BM - 1) / S::BM;
    const int nrt = (N + S::BN - 1) / S::BN;
    const int nkb = K / Q4K_QK;
    const int64_t U = (int64_t)ntt * nrt * nkb;
    const int64_t myu0 = sk_u0(w, U, P), myu1 = sk_u0(w + 1, U, P);

    for (int64_t u = myu0; u < myu1;) {
        const int t = (int)(u / nkb);
        const int kb0 = (int)(u - (int64_t)t * nkb);
        const int kb1 = (int)min<int64_t>(nkb, kb0 + (myu1 - u));
        const int m0 = (t % ntt) * S::BM, n0 = (t / ntt) * S::BN;
        v16f acc[TT][2];
        mmq_segment<TT, WGT, WGN, PR, TT == 1 && WPE <= 2>(sm, W, xq, xds, N, K, m0, n0, kb0, kb1, acc, tiled);
        if (kb0 == 0 && kb1 == nkb) {
            mmq_store<TT, WGT, WGN, PR>(y, M, N, m0, n0, acc, accum);
        } else {
            /* slot rule: 2c for a contributor c whose range starts inside the
             * tile, 2c + 1 for one that started before it (then the tile is
             * its last); each contributor has at most one of each */
            const int64_t a = (int64_t)t * nkb;
            const int c0 = sk_owner(a, U, P), c1 = sk_owner(a + nkb - 1, U, P);
            float *mine = slots + (size_t)(2 * w + (myu0 <= a ? 1 : 0)) * (S::NACC * 256);
            /* Slot traffic uses device-scope (write-through, cache-bypassing)
             * stores and loads, so the hand-off needs no cache-wide fence:
             * each thread's stores have reached the coherence point when its
             * wait returns, before the counter moves; the last contributor
             * reads the slots back from that point. */
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        __hip_atomic_store(&mine[(size_t)((tt * 2 + nt) * 16 + r) * 256 + tid], acc[tt][nt][r],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(&counters[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c1 - c0;
            __syncthreads();
            if (s_last) {
                if (tid == 0) __hip_atomic_store(&counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int c = c0; c <= c1; c++) {
                    const float *src = slots + (size_t)(2 * c + (sk_u0(c, U, P) <= a ? 1 : 0)) * (S::NACC * 256);
#pragma unroll
                    for (int tt = 0; tt < TT; tt++)
#pragma unroll
                        for (int nt = 0; nt < 2; nt++)
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const float v = __hip_atomic_load(&src[(size_t)((tt * 2 + nt) * 16 + r) * 256 + tid],
                                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                acc[tt][nt][r] = c == c0 ? v : acc[tt][nt][r] + v;
                            }
                }
                mmq_store<TT, WGT, WGN, PR>(y, M, N, m0, n0, acc, accum);
            }
        }
        u += kb1 - kb0;
    }
}

/* Whole tiles, then a split tail. The first dp_tiles workgroups each run
 * one whole output tile (the full rounds of resident workgroups, tiles in
 * the XCD-contiguous order of mmq_tile_of). The remaining R = ntiles -
 * dp_tiles tiles are cut along K into `pieces` ranges of near-equal length,
 * one workgroup per (tile, range), so the last round of tiles is spread
 * over every workgroup slot instead of leaving most of them idle. Pieces
 * are ordered range-major, tiles (token tiles fastest) within a range, so
 * the token tiles that share a range's weight bytes run together on one
 * XCD. The pieces of a tile hand off as in the stream-K kernel: each writes
 * its accumulators to its own slot with device-scope stores, waits for
 * them, and bumps the tile's counter; the piece that completes the count
 * sums the slots in piece order, stores the tile and resets the counter. No workgroup waits on another, and the result
 * does not depend on which piece finishes last. */
/* Buffer-resource word 3 for raw 32-bit accesses on gfx950 (the DATA_FORMAT
 * field set to 32 bits, as the MMVQ kernels' resources) and the sc1 cache
 * policy bit of the buffer builtins' aux operand. */
#define MMQ_SLOT_RSRC_FLAGS 0x00020000
#define MMQ_SC1 16

template <int TT, int WGT, int WGN, int WPE = 2, int PR = 0>
__global__ __launch_bounds__(256, WPE) void sera_q4k_mmq_tail_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const uint32_t *__restrict__ xds,
        float *__restrict__ y, float *__restrict__ slots, int *__restrict__ counters, int M, int N, int K,
        int dp_tiles, int pieces, int accum, int tiled) {
    static_assert(WGT * WGN == 4, "4 waves per workgroup");
    using S = MmqShape<TT, WGT, WGN, PR>;
    __shared__ __attribute__((aligned(16))) MmqSmem<S::BM, PR> sm;
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int ntt = (M + S::BM - 1) / S::BM;
    const int nrt = (N + S::BN - 1) / S::BN;
    const int ntiles = ntt * nrt;
    const int nkb = K / Q4K_QK;
    const int wg = blockIdx.x;
    int t, piece = 0, kb0 = 0, kb1 = nkb;
    if (wg < dp_tiles) {
        t = mmq_tile_of(wg, dp_tiles);
    } else {
        const int R = ntiles - dp_tiles;
        const int L = mmq_tile_of(wg - dp_tiles, R * pieces);
        piece = L / R;
        t = dp_tiles + (L - piece * R);
        kb0 = piece * nkb / pieces;
        kb1 = (piece + 1) * nkb / pieces;
    }
    const int m0 = (t % ntt) * S::BM, n0 = (t / ntt) * S::BN;
    v16f acc[TT][2];
    mmq_segment<TT, WGT, WGN, PR, TT == 1 && WPE <= 2>(sm, W, xq, xds, N, K, m0, n0, kb0, kb1, acc, tiled);
    if (wg < dp_tiles || pieces == 1) {
        mmq_store<TT, WGT, WGN, PR>(y, M, N, m0, n0, acc, accum);
        return;
    }
    const int r = t - dp_tiles;
    /* slot (r, p): S::NACC / 4 chunks of 16 bytes per thread, chunk j of
     * thread tid at byte (j * 256 + tid) * 16 of the slot, written and read
     * with 16-byte buffer accesses carrying the sc1 (agent coherence) cache
     * policy, the policy the agent-scope atomic accesses of the stream-K
     * hand-off use, so no stale line of another XCD's L2 is read */
    constexpr int kChunks = S::NACC / 4;
    constexpr int kSlotBytes = S::NACC * 256 * 4;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        slots + (size_t)r * pieces * (S::NACC * 256), (short)0, pieces * kSlotBytes, MMQ_SLOT_RSRC_FLAGS);
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int tt = j / 8, nt = (j / 4) & 1, q0 = 4 * (j & 3);
        const v4f v = {acc[tt][nt][q0], acc[tt][nt][q0 + 1], acc[tt][nt][q0 + 2], acc[tt][nt][q0 + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), rs, (j * 256 + tid) * 16,
                                               piece * kSlotBytes, MMQ_SC1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&counters[r], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == pieces - 1;
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(&counters[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    /* every piece's sums, this one's included, are read back from the
     * slots (this one's stores were acknowledged before the counter moved),
     * which keeps one set of accumulators live instead of two */
    for (int p = 0; p < pieces; p++) {
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int tt = j / 8, nt = (j / 4) & 1, q0 = 4 * (j & 3);
            const v4f v = __builtin_bit_cast(
                v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, (j * 256 + tid) * 16, p * kSlotBytes, MMQ_SC1));
#pragma unroll
            for (int e = 0; e < 4; e++) acc[tt][nt][q0 + e] = p == 0 ? v[e] : acc[tt][nt][q0 + e] + v[e];
        }
    }
    mmq_store<TT, WGT, WGN, PR>(y, M, N, m0, n0, acc, accum);
}

/* Sums the split-K partials in split order: y = ((p0 + p1) + p2) + ... */
__global__ __launch_bounds__(256) void sera_splitk_reduce_kernel(
        const float4 *__restrict__ partial, float4 *__restrict__ y, size_t n4, int splits, int accum) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float4 s = partial[i];
    for (int k = 1; k < splits; k++) {
        const float4 v = partial[(size_t)k * n4 + i];
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    if (accum) {
        const float4 o = y[i];
        s = make_float4(o.x + s.x, o.y + s.y, o.z + s.z, o.w + s.w);
    }
    y[i] = s;
}

/* y[i] (+)= sum over k of partial[k*n + i], k = 0..splits-1 in order, added
 * to y[i] when accum != 0; n % 4 == 0. */
extern "C" hipError_t sera_launch_splitk_reduce_acc(const float *partial, float *y, size_t n, int splits, int accum,
                                                    hipStream_t s) {
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(sera_splitk_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       (const float4 *)partial, (float4 *)y, n4, splits, accum);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_splitk_reduce(const float *partial, float *y, size_t n, int splits,
                                                hipStream_t s) {
    return sera_launch_splitk_reduce_acc(partial, y, n, splits, 0, s);
}

/* Token-tile width of the workgroup for M tokens: 16 (the paired tile, one
 * per wave), 32 (one token tile per wave, 4 waves along weight rows) or 64
 * (two per wave); all at 2 waves per SIMD, and all tiles span 256 weight
 * rows. The 32-token tile ran at 3 waves per SIMD until the magic-seeded
 * epilogue: its 16 seed registers made that budget spill (37 -> 52 us on
 * gate/up at 32 tokens), while at 2 waves with the next step's weights
 * issued ahead it measures 37 us. Measured on MI355X against 128 x
 * 128 tiles (both under stream-K): the 64 x 256 tile is the fastest at 512
 * tokens for both the 5120 -> 25600 and the 25600 -> 5120 shapes. */
extern "C" int sera_mmq_bm(int M) { return M <= 16 ? 16 : M <= 32 ? 32 : 64; }

/* Weight rows per tile: 256, or 128 for the 64-token tile when 256-row
 * tiles would leave at most 64 tiles (k/v at up to 1024 tokens, q and o up
 * to 128). The 128-row tile is 4 waves of 32 tokens x 64 rows (each weight
 * row unpacked by two waves, so it is slower on large grids: gate/up at
 * 512 tokens 242 against 207 us, o 100 against 78) and doubles the grid of
 * the narrow matrices (us, best schedule of each against the 256-row tile:
 * k/v at 256 / 512 / 1024 tokens 18.8 / 24.0 / 31.4 against 23.1 / 26.9 /
 * 32.4; q at 128 tokens 30.2 against 31.7; o at 256 tokens, 80 tiles, 55.7
 * against 50.6). */
static constexpr int kNarrowTileMax = 64;
static int mmq_bn(int M, int N) {
    const int bm = sera_mmq_bm(M);
    if (bm == 64 && ((M + 63) / 64) * ((N + 255) / 256) <= kNarrowTileMax) return 128;
    return 256;
}

/* Workgroups of the stream-K MMQ kernel one CU keeps resident: two for
 * either tile. The 32-token stream-K kernel is built for 2 waves per SIMD:
 * cut to 3 (168 VGPRs) it spills inside the K loop and measured 20-33%
 * slower. */
extern "C" int sera_mmq_wgs_per_cu(int M) { (void)M; return 2; }

/* Split-K factor: the split count in {1, 2, 4, 8, 16} (never fewer than 2
 * super-blocks per split, at most 2048 workgroups) of least modelled time.
 * The model is per CU: the busiest of the 256 CUs holds L = ceil(wgs / 256)
 * workgroups and runs them two at a time, a pair costing kPairUs and a lone
 * workgroup kLoneUs per super-block of a 64 x 256 tile (x0.6 for the 32-token
 * tile, x0.5 for the paired 16-token tile); a split adds the partial sums'
 * write and read, 8 bytes per output per split at 8 TB/s, and the reduce
 * launch. Fitted to MI355X timings of 43 Qwen3-32B shapes (q, k/v, o,
 * gate/up, down at 16-2048 tokens, every split count): its pick is within
 * 3.2% of the fastest split count on every one of them. */
static constexpr float kLoneUs = 3.2f, kPairUs = 5.75f;
static constexpr float kPartialBytesPerUs = 8.0e6f, kReduceUs = 1.0f;
static constexpr int kModelCUs = 256, kMaxSplitWgs = 2048;

extern "C" int sera_mmq_splits(int M, int N, int K) {
    const int bm = sera_mmq_bm(M);
    const int bn = mmq_bn(M, N);
    const int tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int nkb = K / Q4K_QK;
    const float tile_scale = bm == 16 ? 0.5f : bm == 32 ? 0.6f : 1.0f;
    int best = 1;
    float best_us = 0.0f;
    for (int s = 1; s <= 16; s *= 2) {
        if (s > 1 && (nkb / s < 2 || (int64_t)tiles * s > kMaxSplitWgs)) break;
        const int64_t L = ((int64_t)tiles * s + kModelCUs - 1) / kModelCUs;
        const int kb = (nkb + s - 1) / s;
        float us = (float)((L / 2) * kPairUs + (L % 2) * kLoneUs) * kb * tile_scale;
        if (s > 1) us += kReduceUs + (float)s * M * N * 8.0f / kPartialBytesPerUs;
        if (s == 1 || us < best_us) { best = s; best_us = us; }
    }
    return best;
}

/* Rows of the MMQ activation stage: M rounded up to the token tile. */
extern "C" int sera_mmq_padded_rows(int M) {
    const int bm = sera_mmq_bm(M);
    return (M + bm - 1) / bm * bm;
}

template <int TT, int WGT, int WGN, int WPE, int PR = 0>
static hipError_t launch_mmq_cfg(int tiled, const uint8_t *W, const int8_t *xq, const uint32_t *xds, float *y,
                                 float *partial, int M, int N, int K, int splits, int accum, hipStream_t s) {
    constexpr int BM = MmqShape<TT, WGT, WGN, PR>::BM, BN = MmqShape<TT, WGT, WGN, PR>::BN;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int nkb = K / Q4K_QK;
    const int per = (nkb + splits - 1) / splits;
    dim3 grid(tiles, splits);
    hipLaunchKernelGGL((sera_q4k_mmq_kernel<TT, WGT, WGN, WPE, PR>), grid, dim3(256), 0, s, W, xq, xds, y,
                       splits > 1 ? partial : nullptr, M, N, K, per, accum, tiled);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return sera_launch_splitk_reduce_acc(partial, y, (size_t)M * N, splits, accum, s);
}

/* partial: M*N*splits floats of scratch when splits > 1 (M*N % 4 == 0);
 * accum != 0 adds the product to y. */
extern "C" hipError_t sera_launch_q4k_mmq(uint32_t qtype, const void *W, const void *stage, float *y, float *partial,
                                          int M, int N, int K, int splits, hipStream_t s) {
    return sera_launch_q4k_mmq_acc(qtype, W, stage, y, partial, M, N, K, splits, 0, s);
}

extern "C" hipError_t sera_launch_q4k_mmq_acc(uint32_t qtype, const void *W, const void *stage, float *y,
                                              float *partial, int M, int N, int K, int splits, int accum,
                                              hipStream_t s) {
    const int tiled = qtype == SERA_QTYPE_Q4K_TILED;
    if ((!tiled && qtype != 12u) || (tiled && N % Q4K_TILE_ROWS)) return hipErrorInvalidValue;
    const int Mpad = sera_mmq_padded_rows(M);
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const uint32_t *xds = (const uint32_t *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    if (sera_mmq_bm(M) == 16)
        return launch_mmq_cfg<1, 1, 4, 2, 1>(tiled, w, xq, xds, y, partial, M, N, K, splits, accum, s);
    if (sera_mmq_bm(M) == 32)
        return launch_mmq_cfg<1, 1, 4, 2>(tiled, w, xq, xds, y, partial, M, N, K, splits, accum, s);
    if (mmq_bn(M, N) == 128)
        return launch_mmq_cfg<1, 2, 2, 2>(tiled, w, xq, xds, y, partial, M, N, K, splits, accum, s);
    return launch_mmq_cfg<2, 1, 4, 2>(tiled, w, xq, xds, y, partial, M, N, K, splits, accum, s);
}

/* ---- stream-K schedule ---------------------------------------------------- */

/* Output tiles of the MMQ grid for M tokens. */
extern "C" int sera_mmq_tiles(int M, int N) {
    const int bm = sera_mmq_bm(M);
    const int bn = mmq_bn(M, N);
    return ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

/* Floats of one stream-K or tail partial slot: the largest tile's
 * accumulators for M tokens (the paired 16-token tile keeps its 32 MFMA
 * rows); a 128-row tile uses half of its slot. */
extern "C" int sera_mmq_slot_floats(int M) {
    const int bm = sera_mmq_bm(M);
    return (bm < 32 ? 32 : bm) * 256;
}

template <int TT, int WGT, int WGN, int WPE, int PR = 0>
static hipError_t launch_mmq_streamk_cfg(int tiled, const uint8_t *W, const int8_t *xq, const uint32_t *xds,
                                         float *y, float *slots, int *counters, int M, int N, int K, int P, int accum,
                                         hipStream_t s) {
    hipLaunchKernelGGL((sera_q4k_mmq_streamk_kernel<TT, WGT, WGN, WPE, PR>), dim3(P), dim3(256), 0, s, W, xq, xds, y,
                       slots, counters, M, N, K, accum, tiled);
    return hipGetLastError();
}

/* Stream-K MMQ over P persistent workgroups (P a multiple of 8, at most the
 * workgroups the device keeps resident, and ntiles*K/256 >= P).
 * slots: 2*P*sera_mmq_slot_floats(M) floats; counters: sera_mmq_tiles(M,N)
 * ints, zero on entry and zero again on exit. */
extern "C" hipError_t sera_launch_q4k_mmq_streamk(uint32_t qtype, const void *W, const void *stage, float *y,
                                                  float *slots, int *counters, int M, int N, int K, int P,
                                                  hipStream_t s) {
    return sera_launch_q4k_mmq_streamk_acc(qtype, W, stage, y, slots, counters, M, N, K, P, 0, s);
}

extern "C" hipError_t sera_launch_q4k_mmq_streamk_acc(uint32_t qtype, const void *W, const void *stage, float *y,
                                                      float *slots, int *counters, int M, int N, int K, int P,
                                                      int accum, hipStream_t s) {
    const int tiled = qtype == SERA_QTYPE_Q4K_TILED;
    if ((!tiled && qtype != 12u) || (tiled && N % Q4K_TILE_ROWS)) return hipErrorInvalidValue;
    const int Mpad = sera_mmq_padded_rows(M);
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const uint32_t *xds = (const uint32_t *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    if (sera_mmq_bm(M) == 16)
        return launch_mmq_streamk_cfg<1, 1, 4, 2, 1>(tiled, w, xq, xds, y, slots, counters, M, N, K, P, accum, s);
    if (sera_mmq_bm(M) == 32)
        return launch_mmq_streamk_cfg<1, 1, 4, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, P, accum, s);
    if (mmq_bn(M, N) == 128)
        return launch_mmq_streamk_cfg<1, 2, 2, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, P, accum, s);
    return launch_mmq_streamk_cfg<2, 1, 4, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, P, accum, s);
}

/* ---- whole tiles + split tail ---------------------------------------------- */

/* Whole-tile workgroups and K pieces of the tail schedule for M tokens of an
 * N x K matrix on `cus` compute units (64-token tiles, M > 32). The device
 * keeps 2 workgroups per CU resident, so P = 2 * cus run per round. The
 * whole tiles are a multiple of P (all full rounds, or one round fewer);
 * the R tiles left are cut into c K ranges (c = 1: whole as well). Each
 * choice is priced by a rounds model of the greedy dispatch: rounds of P
 * workgroups at kTailPairUs per super-block, a last partial round at
 * kTailLoneUs when it fills no more than one workgroup per CU, and
 * kTailFixUs per piece of a split tile (the hand-off and the last piece's
 * reads). Fitted to a sweep of (whole tiles, c) on 14 Qwen3-32B shapes
 * (q, k/v, o, gate/up, down at 64-2048 tokens) on MI355X: its pick is
 * within 1.6% of the fastest measured choice on every shape where the
 * schedule is used (sera_q4k_mmq_schedule). The split tiles' slots must
 * fit max_slot_floats. */
static constexpr float kTailPairUs = 5.0f, kTailLoneUs = 3.2f, kTailFixUs = 1.5f;

static float tail_cost(int64_t dp_rounds, int64_t R, int c, int nkb, int P, int C) {
    const int64_t n = R * c;
    const int w = (nkb + c - 1) / c;
    const int64_t full = n / P, rem = n % P;
    float us = (float)dp_rounds * nkb * kTailPairUs + (float)full * w * kTailPairUs;
    if (rem) us += (float)w * (rem > C ? kTailPairUs : kTailLoneUs);
    if (c > 1) us += kTailFixUs * c;
    return us;
}

extern "C" void sera_mmq_tail_plan(int M, int N, int K, int cus, size_t max_slot_floats, int *dp_tiles,
                                   int *pieces) {
    const int T = sera_mmq_tiles(M, N);
    const int nkb = K / Q4K_QK;
    const int C = cus > 0 ? cus : kModelCUs;
    const int P = 2 * C;
    const int rounds = T / P;
    int best_dp = T, best_c = 1;
    float best = tail_cost(rounds, T - (int64_t)rounds * P, 1, nkb, P, C);
    for (int fold = 0; fold <= (rounds > 0 ? 1 : 0); fold++) {
        const int dp = (rounds - fold) * P;
        const int R = T - dp;
        if (R == 0) continue;
        for (int c = 2; c <= (nkb < 16 ? nkb : 16); c++) {
            if ((size_t)R * c * sera_mmq_slot_floats(M) > max_slot_floats) break;
            const float us = tail_cost(rounds - fold, R, c, nkb, P, C);
            if (us < best) { best = us; best_dp = dp; best_c = c; }
        }
    }
    *dp_tiles = best_dp;
    *pieces = best_c;
}

/* Floats of the tail schedule's slots and ints of its counters. */
extern "C" size_t sera_mmq_tail_slot_floats(int M, int N, int dp_tiles, int pieces) {
    const int R = sera_mmq_tiles(M, N) - dp_tiles;
    return pieces > 1 && R > 0 ? (size_t)R * pieces * sera_mmq_slot_floats(M) : 0;
}

template <int TT, int WGT, int WGN, int WPE, int PR = 0>
static hipError_t launch_mmq_tail_cfg(int tiled, const uint8_t *W, const int8_t *xq, const uint32_t *xds, float *y,
                                      float *slots, int *counters, int M, int N, int K, int dp_tiles, int pieces,
                                      int accum, hipStream_t s) {
    const int T = sera_mmq_tiles(M, N);
    const int grid = dp_tiles + (T - dp_tiles) * pieces;
    hipLaunchKernelGGL((sera_q4k_mmq_tail_kernel<TT, WGT, WGN, WPE, PR>), dim3(grid), dim3(256), 0, s, W, xq, xds, y,
                       slots, counters, M, N, K, dp_tiles, pieces, accum, tiled);
    return hipGetLastError();
}

/* Tail-scheduled MMQ: dp_tiles whole tiles (0..tiles), the rest in `pieces`
 * K ranges (1..K/256). slots: sera_mmq_tail_slot_floats() floats; counters:
 * tiles - dp_tiles ints, zero on entry and zero again on exit. */
extern "C" hipError_t sera_launch_q4k_mmq_tail_acc(uint32_t qtype, const void *W, const void *stage, float *y,
                                                   float *slots, int *counters, int M, int N, int K, int dp_tiles,
                                                   int pieces, int accum, hipStream_t s) {
    const int tiled = qtype == SERA_QTYPE_Q4K_TILED;
    if ((!tiled && qtype != 12u) || (tiled && N % Q4K_TILE_ROWS)) return hipErrorInvalidValue;
    const int T = sera_mmq_tiles(M, N);
    if (dp_tiles < 0 || dp_tiles > T || pieces < 1 || pieces > K / Q4K_QK) return hipErrorInvalidValue;
    const int Mpad = sera_mmq_padded_rows(M);
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const uint32_t *xds = (const uint32_t *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    if (sera_mmq_bm(M) == 16)
        return launch_mmq_tail_cfg<1, 1, 4, 2, 1>(tiled, w, xq, xds, y, slots, counters, M, N, K, dp_tiles, pieces,
                                                   accum, s);
    if (sera_mmq_bm(M) == 32)
        return launch_mmq_tail_cfg<1, 1, 4, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, dp_tiles, pieces,
                                                accum, s);
    if (mmq_bn(M, N) == 128)
        return launch_mmq_tail_cfg<1, 2, 2, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, dp_tiles, pieces,
                                                accum, s);
    return launch_mmq_tail_cfg<2, 1, 4, 2>(tiled, w, xq, xds, y, slots, counters, M, N, K, dp_tiles, pieces, accum,
                                            s);
}
