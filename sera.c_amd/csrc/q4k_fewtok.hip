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

#include <mutex>

typedef uint32_t ft_v4u __attribute__((ext_vector_type(4)));
typedef float ft_v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void ft_lds_void;
typedef __attribute__((address_space(1))) const void ft_global_cvoid;

#define SERA_FEWTOK_MAX_TOKENS 16
#define SERA_FEWTOK_RSRC_FLAGS 0x00020000   /* gfx9 buffer descriptor word 3: 32-bit dword format */
#define SERA_FEWTOK_LDS_CHUNK_TOKENS 320   /* chunk x staged tokens: 40 super-blocks of 8, 20 of 16 */
#define SERA_FEWTOK_XROW (Q4K_QK + 32)     /* LDS bytes per staged token and super-block: 16 columns + 2 pads */
#define SERA_FEWTOK_XSLOTS (SERA_FEWTOK_XROW / 16)
/* waves per workgroup of a persistent grid (one workgroup per CU: 2 waves
 * per SIMD); 12 waves for one token group, 3 per SIMD, measured 8% slower
 * on the LM head */
template <int TG> constexpr int fewtok_persist_waves() { return 8; }

/* Zero bytes read by the lanes whose MFMA operand is zero: they address
 * the zero area with the same immediate offsets as the real lanes (up to
 * one token group of rows and 160 bytes of columns, plus 16), from one of
 * two bases 16 bytes apart. */
static constexpr __host__ __device__ int fewtok_zero_bytes(int tok) { return (tok / 8 - 1) * 8 * SERA_FEWTOK_XROW + 192; }

/* Floats per row of the min-term factors [u][row][token]: the tokens plus
 * 4 per extra token group. A 4-byte LDS read is served in two passes of 32
 * lanes over 32 banks; its real lanes (n < 8 of K groups g) read rows 2 g
 * (+ 1) at n, so with 16 tokens the rows 0 and 2 of one pass would share
 * banks; 20-float rows put the pass's two 8-lane runs 8 banks apart. */
static constexpr __host__ __device__ int fewtok_mrow(int tok) { return tok + 4 * (tok / 8 - 1); }

/* LDS byte offset of the zero area: after the scale factors, at 0 mod 256.
 *
 * Bank conflicts of the A reads (64 banks of 4 bytes). gfx950 serves a
 * 16-byte LDS read in four passes of 16 lanes: within each half wave, the
 * lane quads (lane >> 2 & 7) of even bit count {0, 3, 5, 6} form one pass
 * and {1, 2, 4, 7} the other (measured with SQ_LDS_BANK_CONFLICT on lane
 * pairs). In a pass, two lanes reading different addresses in one bank
 * cost a cycle; lanes reading one address share it. The 288-byte token
 * rows shift a token's bank by 8 and a column by 4, so a pass's 8 real
 * lanes (tokens 0-3 on one column and 4-7 on another, the columns 1 apart
 * or, past the first column pair, 4 apart) read 8 disjoint 4-bank runs,
 * e.g. starts {0,8,16,24,36,44,52,60} for quads {0, 3, 5, 6}. Relative to
 * the zero area, every even-quad pass leaves banks 4-7 free and every
 * odd-quad pass banks 0-3 (super-block, token group and column offsets
 * move every lane alike: multiples of 256 bytes or common immediates), so
 * the zero lanes of an even-quad pass read at zero + 16 and the others at
 * zero + 0, one address per pass. (With 272-byte rows two reads per
 * instruction conflicted.) */
static inline __host__ __device__ int fewtok_zero_offset(int chunk, int tok) {
    const int end = chunk * (tok * SERA_FEWTOK_XROW + 8 * (tok + fewtok_mrow(tok)) * (int)sizeof(float));
    return (end + 255) & ~255;
}

/* LDS bytes of a workgroup for `chunk` super-blocks of `tok` staged tokens:
 * quants (padded rows), d8, the min-term activation factor, the zero area. */
static inline __host__ __device__ size_t fewtok_lds_bytes(int chunk, int tok) {
    return (size_t)fewtok_zero_offset(chunk, tok) + fewtok_zero_bytes(tok);
}

/* s_waitcnt operands (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
 * 6:4, lgkmcnt 11:8; a field at its maximum is not waited on) */
#define SERA_WAITCNT_LGKM0 0xC07F
#define SERA_WAITCNT_VM0 0x0F70
static constexpr int sera_waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

/* Staged weights (WS > 0 super-blocks per copy): each wave copies its 16
 * rows' next WS super-blocks into one of two LDS buffers with 16-byte loads
 * to LDS, all issued at once, while it computes from the other. On GGUF
 * bytes a copy reads 16 runs of WS * 144 bytes (one per row) instead of the
 * 16 x 64-byte pieces per instruction of the direct loads. Loads-only
 * kernels measured that order 14-16% faster with 2-4 super-blocks per copy
 * and 2-3 workgroups per CU (gate/up, 74 MB: 13.3-14.0 against 15.8 us);
 * in this kernel the staged activations leave LDS for one copy in flight
 * per wave, and the gain is 4% (the launcher). A buffer holds row n's WS
 * blocks at 16 n * RS bytes, unpadded. A 16-byte read is served in four
 * passes of 16 lanes (lane quads of even and odd bit count per half wave);
 * in each pass 8 rows read one piece and 8 others the next, and no row
 * placement gives both those reads and the 16 headers distinct banks:
 * unpadded rows (2 runs of 4 banks apart) cost 4 conflict cycles per
 * super-block, an odd slot count per row (conflict-free headers) 8. */
template <int WS> struct FewtokWs {
    static constexpr int RS = 9 * WS;                                  /* 16-byte slots per row */
    static constexpr int NI = (16 * RS + 63) / 64;                     /* copy instructions */
    static constexpr int BUF = NI * 1024;                              /* LDS bytes of one buffer */
};

/* Row of sub-block b in the min-term factors [u][row][token]: sub-blocks g
 * and 4 + g, which one lane reads together, sit in adjacent rows (one
 * token row apart, so the pair never shares a bank). */
__device__ __forceinline__ int fewtok_mslot(int b) { return (b & 3) * 2 + (b >> 2); }

struct FewtokW {
    ft_v4u hd;      /* d | dmin, 12 scale bytes */
    ft_v4u q[2];    /* nibble bytes at 16 + 64 j + 16 g */
};

/* TG token groups of 8 (M <= 8 TG), FORM 0: MMVQ formula on a row stage
 * (dsf: d8, d8*S as fp32); FORM 1: MMQ formula on an MMQ stage (ds: fp16
 * d8, fp16 sum of x), cuda/mmq/mmq.cuh:2269-2283,1440-1472:
 *   y = sum_b fp16(d*sc_b) * d8_b * I_b + fp16(-dmin*m_b) * s8_b */
template <int NW, int TG, int FORM, bool PERSIST, int WS = 0>
__global__ __launch_bounds__(NW * 64) void sera_q4k_fewtok_kernel(
        const uint8_t *__restrict__ W, const int8_t *__restrict__ xq, const void *__restrict__ xsc,
        float *__restrict__ y, float *__restrict__ slots, int *__restrict__ counters, int M, int N, int K,
        int chunk, int accum, int out_tiles, int tiled) {
    constexpr int TOK = 8 * TG;                          /* staged tokens */
    extern __shared__ __attribute__((aligned(16))) uint8_t ft_smem[];
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   /* wave-uniform: LDS copy targets need no waterfall */
    const int n = lane & 15;          /* B column (weight row), A row */
    const int g = lane >> 4;          /* 16-wide K group */
    const int hq = g & 1;
    const int nkb = K / Q4K_QK;
    const int kb0 = blockIdx.y * chunk;
    const int C = min(nkb - kb0, chunk);
    /* LDS: quants [u][t][288] | d8 [u][b][t] | min factor [u][mslot(b)][t] | zero */
    int8_t *xs = (int8_t *)ft_smem;
    float *d8s = (float *)(ft_smem + (size_t)chunk * TOK * SERA_FEWTOK_XROW);
    float *mns = d8s + (size_t)chunk * 8 * TOK;
    constexpr int MR = fewtok_mrow(TOK);                 /* floats per min-factor row */
    uint8_t *zero = ft_smem + fewtok_zero_offset(chunk, TOK);
    /* PERSIST: results of the workgroup's tiles, [token][row], out_tiles
     * tiles of 16 rows per token */
    float *outb = (float *)(ft_smem + fewtok_lds_bytes(chunk, TOK));
    const int ocap = 16 * out_tiles;

    /* 16-row tiles. One tile per wave: wave w of workgroup b takes tile
     * NW b + w (rows past N are clamped and never stored; split K's
     * hand-off counts the NW tiles of a workgroup). PERSIST (one K split,
     * an even chunk, a grid smaller than the tile groups): the workgroup
     * stages its chunk once and takes a balanced range [tb, te) of all
     * ceil(N / 16) tiles; wave w starts on tile tb + w and then takes the
     * next free one from an LDS counter. */
    __shared__ int s_next;
    int tb, te;
    if constexpr (!PERSIST) {
        tb = blockIdx.x * NW;
        te = tb + NW;
    } else {
        const long T = (N + 15) / 16;
        tb = (int)(blockIdx.x * T / gridDim.x);
        te = (int)((blockIdx.x + 1) * T / gridDim.x);
    }
    int tile = tb + wave;
    int row;
    bool row_ok;
    auto rows_of = [&](int t, int &r, bool &ok) {
        r = 16 * t + n;
        ok = r < N;
        if (!ok) r = N - 1;
    };
    rows_of(tile, row, row_ok);
    const int bstride = q4k_block_stride(tiled);   /* super-block to super-block of one row */
    const uint32_t rstride = (uint32_t)q4k_row_stride(tiled, nkb);
    /* Direct loads are buffer loads from a resource over tile t (its first
     * row and the chunk's first block, through the chunk's last block of its
     * last row): the lane's row offset is the vector offset and the
     * super-block step the scalar offset, so a load takes no vector address
     * arithmetic. Rows past N read row N - 1; a tile past the last row (a
     * wave with no tile, or the end of a workgroup's range) reads the last
     * tile's rows and is never stored. */
    auto tile_row0 = [&](int t) { return min(16 * t, 16 * ((N - 1) / 16)); };
    auto tile_rsrc = [&](int t) {
        const int r0 = tile_row0(t);
        const uint32_t bytes = (uint32_t)(min(N - r0, 16) - 1) * rstride + (uint32_t)C * (uint32_t)bstride;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W + q4k_block_offset(tiled, (size_t)r0, kb0, nkb)),
                                                 (short)0, (int)bytes, SERA_FEWTOK_RSRC_FLAGS);
    };
    auto tile_lane = [&](int t) { return (uint32_t)min(n, N - 1 - tile_row0(t)) * rstride; };
    __amdgpu_buffer_rsrc_t wr = tile_rsrc(tile), wnext;
    uint32_t wl = tile_lane(tile), wlnext;
    /* super-block u of the chunk (u < C; the loop never asks for more) */
    auto load_from = [&](__amdgpu_buffer_rsrc_t rs, uint32_t lo, int u, FewtokW &w) {
        const int so = u * bstride;
        const uint32_t lq = lo + 16 * g;
        w.hd = __builtin_amdgcn_raw_buffer_load_b128(rs, lo, so, 0);
        w.q[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, lq + 16, so, 0);
        w.q[1] = __builtin_amdgcn_raw_buffer_load_b128(rs, lq + 80, so, 0);
    };
    auto load = [&](int u, FewtokW &w) { load_from(wr, wl, u, w); };
    FewtokW wa, wb;
    /* WS: the wave's two weight buffers after the staged activations, and
     * the copy of sub-chunk sc (super-blocks WS sc .. WS sc + WS - 1 of the
     * chunk, clamped to the chunk: a partial last copy re-reads its last
     * super-block) into buffer bf. Slot q = 64 i + lane of the buffer is
     * piece q % RS of row q / RS (pieces past the row's 9 WS, the pad, and
     * slots past row 15 copy a valid piece and are never read). */
    using Ws = FewtokWs<WS ? WS : 1>;
    uint8_t *wbuf = ft_smem + fewtok_lds_bytes(chunk, TOK) + (size_t)wave * 2 * Ws::BUF;
    /* per copy instruction i: the lane's source in the chunk's first
     * sub-chunk and its super-block there */
    /* The tile's first row and block as a wave-uniform base, each lane's
     * slot as a 32-bit offset from it (rows of a 16-row tile lie in one tile
     * of the tiled layout). The slot's (row, piece) advance by (3, 10) or
     * (4, -8) per instruction (64 = 3 * 18 + 10): a few full-rate adds per
     * instruction ahead of the first copy, where a division and 64-bit
     * offsets per instruction measured slower. */
    /* Waves whose tile lies past the last row (N < 16 NW, or the last
     * workgroup of a grid) read the last tile's rows instead; they are
     * never stored. */
    const int wrow0 = min(16 * tile, 16 * ((N - 1) / 16));
    const uint8_t *wtile = W + q4k_block_offset(tiled, (size_t)wrow0, kb0, nkb);
    uint32_t wso[WS ? Ws::NI : 1];
    int wsu[WS ? Ws::NI : 1];
    if constexpr (WS > 0) {
        static_assert(Ws::RS == 18, "per-instruction slot step laid out for 18 slots per row");
        const int rmax = min(N - 1 - wrow0, 15);   /* 0..15 */
        const uint32_t rstride = (uint32_t)q4k_row_stride(tiled, nkb);
        int r = lane / 18, o = lane - 18 * r;
#pragma unroll
        for (int i = 0; i < Ws::NI; i++) {
            const int u = o >= 9 ? 1 : 0;
            wsu[i] = u;
            wso[i] = (uint32_t)min(r, rmax) * rstride + (uint32_t)(min(u, C - 1) * bstride + 16 * (o - 9 * u));
            o += 10;
            r += o >= 18 ? 4 : 3;
            o -= o >= 18 ? 18 : 0;
        }
    }
    auto ws_issue = [&](int sc, int bf) {
        const bool whole = WS * sc + WS <= C;
        const uint8_t *wsb = wtile + (size_t)(whole ? WS * sc : 0) * bstride;
#pragma unroll
        for (int i = 0; i < Ws::NI; i++) {
            /* a whole sub-chunk moves every lane alike; the last one clamps */
            const uint32_t du = whole ? 0u : (uint32_t)((min(WS * sc + wsu[i], C - 1) - min(wsu[i], C - 1)) * bstride);
            __builtin_amdgcn_global_load_lds((ft_global_cvoid *)(wsb + (wso[i] + du)),
                                             (ft_lds_void *)(wbuf + bf * Ws::BUF + 1024 * i), 16, 0, 0);
        }
    };
    /* super-block ul of the sub-chunk in buffer bf, in the layout load() gives */
    auto ws_read = [&](int bf, int ul, FewtokW &w) {
        const uint8_t *b = wbuf + bf * Ws::BUF + n * (16 * Ws::RS) + ul * Q4K_BLOCK_BYTES;
        w.hd = *(const ft_v4u *)b;
        w.q[0] = *(const ft_v4u *)(b + 16 + 16 * g);
        w.q[1] = *(const ft_v4u *)(b + 80 + 16 * g);
    };
    const int nsub = WS ? (C + WS - 1) / WS : 0;
    if constexpr (WS > 0) {
        ws_issue(0, 0);                /* in flight during the activation staging */
        if (nsub > 1) ws_issue(1, 1);
    } else {
        if (tile < te) load(0, wa);    /* in flight during the activation staging */
        if (PERSIST && (C & 3) == 0 && tile < te) load(1, wb);
    }
    if (PERSIST && tid == 0) s_next = 0;

    /* --- stage the chunk's activations --- */
    {
        /* quants: 16-byte slot s of token row (u, t) holds column s (slots
         * 16-17 are the row's pad, filled with copies of column 15 and never
         * read); one wave-instruction writes 64 consecutive slots (1 KB),
         * lanes past the chunk are masked off; tokens past M copy the last.
         * The 288-byte rows keep the A reads free of bank conflicts (at the
         * zero area's offset), and every operand of a lane sits at a
         * constant offset from one base. */
        constexpr int XS = SERA_FEWTOK_XSLOTS;
        const int slots = C * TOK * XS;
        /* slot q = (u, t, col) with q = (u TOK + t) XS + col, decoded once
         * and advanced by NW * 64 slots per pass with carries; the source
         * is a 32-bit offset from the chunk's first column */
        constexpr int STEP = NW * 64, SU = STEP / (TOK * XS), ST = STEP % (TOK * XS) / XS, SC = STEP % XS;
        const int8_t *xbase = xq + (size_t)kb0 * Q4K_QK;
        int q = wave * 64 + lane;
        int u = q / (TOK * XS), t = q % (TOK * XS) / XS, col = q % XS;
        for (int base = wave * 64; base < slots; base += STEP) {
            const uint32_t off = (uint32_t)(min(t, M - 1) * K + u * Q4K_QK + 16 * min(col, 15));
            if (q < slots)
                __builtin_amdgcn_global_load_lds((ft_global_cvoid *)(xbase + off),
                                                 (ft_lds_void *)(xs + (size_t)base * 16), 16, 0, 0);
            q += STEP;
            col += SC;
            const int cc = col >= XS ? 1 : 0;
            col -= cc * XS;
            t += ST + cc;
            const int tc = t >= TOK ? 1 : 0;
            t -= tc * TOK;
            u += SU + tc;
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
            /* 32-bit element offsets from the chunk's first scales */
            if (FORM == 0) {
                const int u = i / (TOK * 4), t = (i >> 2) % TOK, p = i & 3;
                f[r] = ((const ft_v4u *)xsc + (size_t)kb0 * 4)[(uint32_t)(min(t, M - 1) * (K / 64) + u * 4 + p)];
            } else {
                const int u = i / (TOK * 2), t = (i >> 1) % TOK, p = i & 1;
                f[r] = ((const ft_v4u *)xsc + (size_t)kb0 * 2)[(uint32_t)(min(t, M - 1) * (K / 128) + u * 2 + p)];
            }
        }
#pragma unroll
        for (int r = 0; r < SCR; r++) {
            const int i = tid + r * NW * 64;
            if (i < items) {
                if (FORM == 0) {
                    const int u = i / (TOK * 4), t = (i >> 2) % TOK, p = i & 3;
                    float *d8u = d8s + u * 8 * TOK, *mnu = mns + u * 8 * MR;
                    d8u[(2 * p) * TOK + t] = __uint_as_float(f[r].x);
                    d8u[(2 * p + 1) * TOK + t] = __uint_as_float(f[r].y);
                    mnu[fewtok_mslot(2 * p) * MR + t] = __uint_as_float(f[r].z);
                    mnu[fewtok_mslot(2 * p + 1) * MR + t] = __uint_as_float(f[r].w);
                } else {
                    const int u = i / (TOK * 2), t = (i >> 1) % TOK, p = i & 1;
                    float *d8u = d8s + u * 8 * TOK, *mnu = mns + u * 8 * MR;
                    const uint32_t ds[4] = {f[r].x, f[r].y, f[r].z, f[r].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        d8u[(4 * p + e) * TOK + t] = h2f_bits(ds[e] & 0xffffu);
                        mnu[fewtok_mslot(4 * p + e) * MR + t] = h2f_bits(ds[e] >> 16);
                    }
                }
            }
        }
        for (int i = tid; i < fewtok_zero_bytes(TOK) / 16; i += NW * 64) ((ft_v4u *)zero)[i] = (ft_v4u){0u, 0u, 0u, 0u};
    }
    __builtin_amdgcn_s_waitcnt(0);    /* this thread's loads to LDS have landed */
    __syncthreads();

    /* A operand: lane (row i = n, group g) is real when (i < 8) == (g < 2):
     * token 8 tg + (i & 7) on sub-block 4j + 2 (i >> 3) + h, 16 bytes at
     * k-half hq, i.e. column 2 (4j + 2 (i >> 3) + h) + hq of the token row.
     * Every (tg, j, h) is a constant offset from the lane's base for super-
     * block u, a_base + u * a_step; the other lanes have step 0 and a base
     * in the zero area (16 bytes up for the lane quads of even bit count,
     * see fewtok_zero_offset), so they read zeros at the same offsets. Staged
     * tokens past M hold copies of the last token; their results are never
     * stored. The min-term A (FORM 0 d8*S, FORM 1 the fp16 sum of x) works
     * the same way: lanes n < 8 read token 8 tg + n of sub-blocks g, 4 + g. */
    const bool a_real = (n < 8) == (g < 2);
    const int zoff = (int)(zero - (uint8_t *)ft_smem);
    const int a_base = a_real ? (n & 7) * SERA_FEWTOK_XROW + 16 * (4 * (n >> 3) + hq)
                              : zoff + 16 * (1 - (__builtin_popcount((lane >> 2) & 7) & 1));
    const int a_step = a_real ? TOK * SERA_FEWTOK_XROW : 0;
    /* min-term A: zero lanes read the zero area at a bank the real lanes of
     * their 32-lane pass leave free (8 with one token group; 16 for lanes
     * 0-31 and 0 for 32-63 with two) */
    const int m_zero = zoff + (TG == 1 ? 32 : lane < 32 ? 64 : 0);
    const int m_base = n < 8 ? (int)((uint8_t *)mns - (uint8_t *)ft_smem) + 4 * (2 * g * MR + n) : m_zero;
    const int m_step = n < 8 ? 4 * 8 * MR : 0;
    const int sg = g >> 1;            /* result sub-block: 4j + 2 sg + h */
    const int tq = 4 * hq;            /* result tokens 8 tg + tq .. + 3 */
    /* FORM 1 scale bytes as fp16 1024 + v: v_perm puts sub-block bytes
     * (2 sg, 2 sg + 1) under exponent byte 0x64 (selector bytes 0-3 pick
     * the scale word, 4 the 0x64 word) */
    const uint32_t sel_sc = (2u * sg) | (4u << 8) | ((2u * sg + 1u) << 16) | (4u << 24);
    ft_v4f acc[TG];
    const v4i magic = sera_magic_seed<4>();

    auto compute = [&](int u, const FewtokW &w) {
        const uint8_t *au = ft_smem + a_base + u * a_step;
        const uint8_t *mu = ft_smem + m_base + u * m_step;
        const float *d8u = d8s + u * 8 * TOK;
        /* the super-block's LDS operands first: they do not wait for the
         * weights, so their latency overlaps the wait for the header */
        v4i Ar[4][TG];
        ft_v4f D8r[4][TG];
        float am0[TG], am1[TG];
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            am0[tg] = *(const float *)(mu + 32 * tg);
            am1[tg] = *(const float *)(mu + 4 * MR + 32 * tg);
        }
#pragma unroll
        for (int jh = 0; jh < 4; jh++)
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                Ar[jh][tg] = *(const v4i *)(au + 8 * SERA_FEWTOK_XROW * tg + 32 * (jh & 1) + 128 * (jh >> 1));
                D8r[jh][tg] = *(const ft_v4f *)&d8u[(4 * (jh >> 1) + 2 * sg + (jh & 1)) * TOK + 8 * tg + tq];
            }
        /* (scale, min) bytes of sub-blocks 0-3 and 4-7 (src/q3_quant.c:44-55) */
        const ft_v4u hd = w.hd;
        const uint32_t sc03 = hd.y & 0x3F3F3F3Fu;
        const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
        const uint32_t sc47 = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        /* sub-block scale and min products: FORM 0 exact in fp32 (d*sc,
         * -dmin*m); FORM 1 one fp16 rounding each, as the reference's half2
         * store (d, dmin) * (1, -1) * (sc, m): the bytes become fp16 1024 + v,
         * an exact subtraction leaves v, one packed RNE multiply the product */
        float swv[4], bm0, bm1;
        if constexpr (FORM == 0) {
            const float d = h2f_bits(hd.x & 0xffffu), ndmin = -h2f_bits(hd.x >> 16);
            const uint32_t s03 = sc03 >> (16 * sg), s47 = sc47 >> (16 * sg);
            swv[0] = d * (float)(s03 & 0xffu);
            swv[1] = d * (float)((s03 >> 8) & 0xffu);
            swv[2] = d * (float)(s47 & 0xffu);
            swv[3] = d * (float)((s47 >> 8) & 0xffu);
            bm0 = ndmin * (float)((m03 >> (8 * g)) & 0xffu);
            bm1 = ndmin * (float)((m47 >> (8 * g)) & 0xffu);
        } else {
            typedef _Float16 ft_h2 __attribute__((ext_vector_type(2)));
            const ft_h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
            const uint32_t dd = (hd.x & 0xffffu) * 0x10001u, nm = (hd.x >> 16) * 0x10001u ^ 0x80008000u;
            const ft_h2 d2 = __builtin_bit_cast(ft_h2, dd), nm2 = __builtin_bit_cast(ft_h2, nm);
            const ft_h2 p03 = (__builtin_bit_cast(ft_h2, __builtin_amdgcn_perm(0x64646464u, sc03, sel_sc)) - bias) * d2;
            const ft_h2 p47 = (__builtin_bit_cast(ft_h2, __builtin_amdgcn_perm(0x64646464u, sc47, sel_sc)) - bias) * d2;
            const uint32_t mg = __builtin_amdgcn_perm(m47, m03, (uint32_t)g | ((4u + g) << 8));
            const ft_h2 pm = (__builtin_bit_cast(ft_h2, __builtin_amdgcn_perm(0x64646464u, mg, 0x04010400u)) - bias) * nm2;
            swv[0] = (float)p03.x;
            swv[1] = (float)p03.y;
            swv[2] = (float)p47.x;
            swv[3] = (float)p47.y;
            bm0 = (float)pm.x;
            bm1 = (float)pm.y;
        }
        /* min term: lane (n, g) gives A[n][g] and B[g][n] for sub-blocks g
         * and 4 + g */
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            acc[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(am0[tg], bm0, acc[tg], 0, 0, 0);
            acc[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(am1[tg], bm1, acc[tg], 0, 0, 0);
        }
#pragma unroll
        for (int jh = 0; jh < 4; jh++) {
            const int j = jh >> 1, h = jh & 1;
            const float swb = swv[jh];
            const float nswb = -SERA_MAGIC_F * swb;
            const ft_v4u q = w.q[j];
            v4i B;
            B.x = (int)((q.x >> (4 * h)) & 0x0F0F0F0Fu);
            B.y = (int)((q.y >> (4 * h)) & 0x0F0F0F0Fu);
            B.z = (int)((q.z >> (4 * h)) & 0x0F0F0F0Fu);
            B.w = (int)((q.w >> (4 * h)) & 0x0F0F0F0Fu);
#pragma unroll
            for (int tg = 0; tg < TG; tg++) {
                const v4i A = Ar[jh][tg];
                const ft_v4f D8 = D8r[jh][tg];
                /* magic-seeded: (I * scale) rounded once, then * d8 into acc */
                const v4i F = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, magic, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[tg][r] = fmaf(scaled_dot(F[r], swb, nswb), D8[r], acc[tg][r]);
            }
        }
    };
    /* one tile's results: split K hands partials to the last split; one
     * tile per wave stores directly; PERSIST keeps them in LDS, so its loop
     * issues no global stores and the load counting stays exact across
     * tiles. Returns false when this workgroup's split is not the last. */
    auto finish = [&]() -> bool {
        /* lanes g and g ^ 2 hold the two sub-block halves of the same outputs */
#pragma unroll
        for (int tg = 0; tg < TG; tg++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[tg][r] += __shfl_xor(acc[tg][r], 32, 64);
        const bool owner = g < 2 && row_ok;

        if (gridDim.y > 1) {
            /* split K: this split's partial of the tile goes to
             * slots[split][t][row] with device-scope stores, so the hand-off
             * needs no cache-wide fence */
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
                s_last = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) == S - 1;
            __syncthreads();
            if (!s_last) return false;
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
        if constexpr (!PERSIST) {
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
        } else if (g < 2) {
#pragma unroll
            for (int tg = 0; tg < TG; tg++)
#pragma unroll
                for (int r = 0; r < 4; r++) outb[(8 * tg + tq + r) * ocap + 16 * (tile - tb) + n] = acc[tg][r];
        }
        return true;
    };
    /* One super-block in flight, issued before the current one's compute
     * (the scheduling barriers keep each load group ahead of the compute it
     * overlaps). Measured against two in flight (the next two issued after
     * each compute): 4-6% faster at 4-8 tokens (gate/up 19.6 -> 18.5 us,
     * down 25.3 -> 23.9), equal at 16; deeper prefetch, in groups of 2-5
     * super-blocks or only before the staging, was slower at every size. */
    if constexpr (WS > 0) {
        static_assert(!PERSIST, "staged weights serve one tile per wave");
#pragma unroll
        for (int tg = 0; tg < TG; tg++) acc[tg] = (ft_v4f){0.f, 0.f, 0.f, 0.f};
        /* the barrier above waited for sub-chunks 0 and 1 */
        for (int sc = 0; sc < nsub; sc++) {
            const int bf = sc & 1;
            const int nu = min(WS, C - WS * sc);
#pragma unroll
            for (int ul = 0; ul < WS; ul++) {
                if (ul < nu) {
                    ws_read(bf, ul, wa);
                    compute(WS * sc + ul, wa);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (sc + 2 < nsub) {
                /* buffer bf is free once its LDS reads have returned; then
                 * sub-chunk sc + 1 (issued before this copy) is waited for */
                __builtin_amdgcn_s_waitcnt(SERA_WAITCNT_LGKM0);
                ws_issue(sc + 2, bf);
                __builtin_amdgcn_s_waitcnt(sera_waitcnt_vm(Ws::NI));
            } else {
                __builtin_amdgcn_s_waitcnt(SERA_WAITCNT_VM0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        finish();
    } else if constexpr (!PERSIST) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) acc[tg] = (ft_v4f){0.f, 0.f, 0.f, 0.f};
        int u0 = 0;
        for (; u0 + 1 < C; u0 += 2) {
            load(u0 + 1, wb);
            __builtin_amdgcn_sched_barrier(0);
            compute(u0, wa);
            __builtin_amdgcn_sched_barrier(0);
            load(min(u0 + 2, C - 1), wa);   /* past the chunk: re-read, unused */
            __builtin_amdgcn_sched_barrier(0);
            compute(u0 + 1, wb);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (u0 < C) compute(u0, wa);   /* odd chunk: the last super-block */
        finish();
    } else if ((C & 3) == 0) {
        /* two to four super-blocks in flight: the loop takes four per turn
         * in two register pairs, loading one pair while it computes the
         * other; the last turn's second pair of loads is the next tile's
         * first two super-blocks (past the range it re-reads this tile's
         * rows). Against one in flight (the loop below) on the 151936-row
         * LM head: 2-8 tokens 84-87 against 87-90 us, 16 tokens 97.5-98
         * against 99-102; tiled bytes at 16 tokens 94.8 against 98.7. The
         * same loop on one tile per wave (gate/up, down, o at 2-16 tokens)
         * was 2-6% slower than the loop below it. */
        FewtokW wc, wd;
        while (tile < te) {
#pragma unroll
            for (int tg = 0; tg < TG; tg++) acc[tg] = (ft_v4f){0.f, 0.f, 0.f, 0.f};
            int next = 0;
            if (lane == 0)
                next = tb + NW + __hip_atomic_fetch_add(&s_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            next = __builtin_amdgcn_readfirstlane(next);
            int nrow;
            bool nrow_ok;
            const int nt = next < te ? next : tile;
            rows_of(nt, nrow, nrow_ok);
            wnext = tile_rsrc(nt);
            wlnext = tile_lane(nt);
            for (int u0 = 0; u0 < C; u0 += 4) {
                load(u0 + 2, wc);
                load(u0 + 3, wd);
                __builtin_amdgcn_sched_barrier(0);
                compute(u0, wa);
                compute(u0 + 1, wb);
                __builtin_amdgcn_sched_barrier(0);
                int last = __builtin_amdgcn_readfirstlane(u0 + 4 == C ? 1 : 0);
                __asm__ volatile("" : "+s"(last));
                const uint32_t lo = last ? wlnext : wl;
                const __amdgpu_buffer_rsrc_t rs = last ? wnext : wr;
                load_from(rs, lo, last ? 0 : u0 + 4, wa);
                load_from(rs, lo, last ? 1 : u0 + 5, wb);
                __builtin_amdgcn_sched_barrier(0);
                compute(u0 + 2, wc);
                compute(u0 + 3, wd);
                __builtin_amdgcn_sched_barrier(0);
            }
            finish();
            tile = next;
            row = nrow;
            row_ok = nrow_ok;
            wr = wnext;
            wl = wlnext;
        }
        __syncthreads();
        const int r0 = 16 * tb, nr = min(16 * te, N) - r0;
        for (int i = tid; i < nr * M; i += NW * 64) {
            const int t = i / nr, r = i - t * nr;
            float *dst = y + (size_t)t * N + r0 + r;
            const float v = outb[t * ocap + r];
            *dst = accum ? *dst + v : v;
        }
    } else {
        while (tile < te) {
#pragma unroll
            for (int tg = 0; tg < TG; tg++) acc[tg] = (ft_v4f){0.f, 0.f, 0.f, 0.f};
            /* the wave's next tile; its first super-block is the last pair's
             * second load (past the range it re-reads this tile's rows) */
            int next = 0;
            if (lane == 0)
                next = tb + NW + __hip_atomic_fetch_add(&s_next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            next = __builtin_amdgcn_readfirstlane(next);
            int nrow;
            bool nrow_ok;
            const int nt = next < te ? next : tile;
            rows_of(nt, nrow, nrow_ok);
            wnext = tile_rsrc(nt);
            wlnext = tile_lane(nt);
            /* even chunk: the select on an opaque flag keeps one loop body and
             * its exact load counting (the compiler would peel the last pair) */
            for (int u0 = 0; u0 < C; u0 += 2) {
                load(u0 + 1, wb);
                __builtin_amdgcn_sched_barrier(0);
                compute(u0, wa);
                __builtin_amdgcn_sched_barrier(0);
                int last = __builtin_amdgcn_readfirstlane(u0 + 2 == C ? 1 : 0);
                __asm__ volatile("" : "+s"(last));
                load_from(last ? wnext : wr, last ? wlnext : wl, last ? 0 : u0 + 2, wa);
                __builtin_amdgcn_sched_barrier(0);
                compute(u0 + 1, wb);
                __builtin_amdgcn_sched_barrier(0);
            }
            finish();
            tile = next;
            row = nrow;
            row_ok = nrow_ok;
            wr = wnext;
            wl = wlnext;
        }
        /* the workgroup's rows [16 tb, 16 te) of every token, coalesced */
        __syncthreads();
        const int r0 = 16 * tb, nr = min(16 * te, N) - r0;
        for (int i = tid; i < nr * M; i += NW * 64) {
            const int t = i / nr, r = i - t * nr;
            float *dst = y + (size_t)t * N + r0 + r;
            const float v = outb[t * ocap + r];
            *dst = accum ? *dst + v : v;
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


/* Per-device facts the persistent grid is sized from: the CU count, the
 * LDS one workgroup may use, and the occupancy of each kernel instance per
 * LDS size (cached on the exact byte count; guarded by a mutex, since
 * several host threads may launch). */
struct FewtokDevice {
    int cus = 0;
    int max_lds = 0;
};
static std::mutex g_fewtok_mu;

static bool fewtok_device(int *dev_out, FewtokDevice *out) {
    static FewtokDevice devs[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return false;
    std::lock_guard<std::mutex> lock(g_fewtok_mu);
    FewtokDevice &d = devs[dev];
    if (d.cus == 0) {
        int cus = 0, lds = 0, optin = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0 ||
            hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds <= 0)
            return false;
        if (hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, dev) == hipSuccess && optin > lds)
            lds = optin;
        d.cus = cus;
        d.max_lds = lds;
    }
    *dev_out = dev;
    *out = d;
    return true;
}

/* Workgroups of one launch that the device holds at once (CUs times the
 * occupancy the kernel's registers and LDS allow), or 0 if unknown. */
template <int NW, int TG, int FORM>
static int fewtok_resident(size_t lds) {
    constexpr bool PERSIST = true;
    constexpr int kEntries = 8;
    static int cache[16][kEntries][2];   /* [device][entry] -> (lds bytes, workgroups per CU) */
    static int next[16];
    int dev = 0;
    FewtokDevice d;
    if (!fewtok_device(&dev, &d)) return 0;
    if (lds > (size_t)d.max_lds) return 0;
    {
        std::lock_guard<std::mutex> lock(g_fewtok_mu);
        for (int e = 0; e < kEntries; e++)
            if (cache[dev][e][0] == (int)lds && cache[dev][e][1] > 0) return d.cus * cache[dev][e][1];
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sera_q4k_fewtok_kernel<NW, TG, FORM, PERSIST>, NW * 64,
                                                      lds) != hipSuccess || per_cu <= 0)
        return 0;
    std::lock_guard<std::mutex> lock(g_fewtok_mu);
    const int e = next[dev]++ % kEntries;
    cache[dev][e][0] = (int)lds;
    cache[dev][e][1] = per_cu;
    return d.cus * per_cu;
}

/* Grid (workgroups along the rows), persistent-buffer tiles (0: one tile
 * per wave) and LDS bytes of a launch on the current device. */
template <int NW, int TG, int FORM>
static void fewtok_grid(int N, int K, int chunk, bool allow_persist, int *groups_out, int *out_tiles_out,
                        size_t *lds_out) {
    const int nkb = K / Q4K_QK;
    const int splits = (nkb + chunk - 1) / chunk;
    const size_t base = fewtok_lds_bytes(chunk, 8 * TG);
    const int tiles = (N + 15) / 16;
    int groups = (N + 16 * NW - 1) / (16 * NW), out_tiles = 0;
    size_t lds = base;
    if constexpr (NW == fewtok_persist_waves<TG>()) {
        int dev = 0;
        FewtokDevice d;
        if (allow_persist && splits == 1 && (nkb & 1) == 0 && fewtok_device(&dev, &d)) {
            /* more tile groups than resident workgroups: a persistent grid,
             * each workgroup staging the activations once for its range of
             * tiles and keeping the results in LDS until its last tile (the
             * buffer's size feeds back into the occupancy, hence the two
             * rounds) */
            auto out_bytes = [&](int g) { return (size_t)((tiles + g - 1) / g) * 16 * 8 * TG * sizeof(float); };
            const int natural = groups;
            for (int round = 0; round < 2; round++) {
                const int resident = fewtok_resident<NW, TG, FORM>(base + out_bytes(groups));
                if (resident > 0 && groups > resident) groups = resident;
            }
            /* the result buffer must fit the workgroup's LDS: with more
             * tiles per workgroup than that allows (a very tall matrix),
             * take more workgroups, each with a shorter range (they need
             * not all be resident: no workgroup waits on another) */
            while (groups < natural && base + out_bytes(groups) > (size_t)d.max_lds) {
                const size_t room = (size_t)d.max_lds > base ? (size_t)d.max_lds - base : 0;
                const int per = (int)(room / ((size_t)16 * 8 * TG * sizeof(float)));   /* tiles that fit */
                groups = per > 0 ? (tiles + per - 1) / per : natural;
                if (groups > natural) groups = natural;
            }
            if (groups < natural) {
                out_tiles = (tiles + groups - 1) / groups;
                lds = base + out_bytes(groups);
            } else {
                groups = natural;
            }
        }
    }
    *groups_out = groups;
    *out_tiles_out = out_tiles;
    *lds_out = lds;
}

template <int NW, int TG, int FORM, bool PERSIST, int WS = 0>
static hipError_t launch_fewtok(int tiled, const uint8_t *W, const int8_t *xq, const void *xsc, float *y,
                                float *slots, int *counters, int M, int N, int K, int chunk, int accum, int groups,
                                int out_tiles, size_t lds, hipStream_t s) {
    dim3 grid(groups, (K / Q4K_QK + chunk - 1) / chunk);
    hipLaunchKernelGGL((sera_q4k_fewtok_kernel<NW, TG, FORM, PERSIST, WS>), grid, dim3(NW * 64), lds, s, W, xq, xsc,
                       y, slots, counters, M, N, K, chunk, accum, out_tiles, tiled);
    return hipGetLastError();
}

/* One tile per wave. GGUF bytes in 8-wave workgroups (the matrices whose
 * rows or K reach 16384) take the staged-weight kernel with 2-super-block
 * copies when its buffers fit the device's LDS beside the staged
 * activations; everything else loads straight into registers. Measured
 * (us, staged against direct, GGUF bytes): gate/up 2-8 tokens 18.6-19.0
 * against 19.4-19.8, down 21.8-24.4 against 22.7-25.2, 16 tokens equal;
 * on the 4-wave shapes (q, o) 2-7 us slower, and on the tiled layout 1.6-2
 * us slower on every shape. Copies of 3 or 4 super-blocks leave no LDS for
 * two buffers of 8 waves at 20-block chunks; 10-block chunks (2 splits)
 * were slower with either kernel. */
static constexpr int kFewtokWs = 2;
template <int NW, int TG, int FORM>
static hipError_t launch_fewtok_tiles(int tiled, const uint8_t *W, const int8_t *xq, const void *xsc, float *y,
                                      float *slots, int *counters, int M, int N, int K, int chunk, int accum,
                                      hipStream_t s) {
    int groups, out_tiles;
    size_t lds;
    fewtok_grid<NW, TG, FORM>(N, K, chunk, false, &groups, &out_tiles, &lds);
    if constexpr (NW == 8) {
        const size_t lds_ws = lds + (size_t)NW * 2 * FewtokWs<kFewtokWs>::BUF;
        int dev = 0;
        FewtokDevice d;
        if (!tiled && fewtok_device(&dev, &d) && lds_ws <= (size_t)d.max_lds)
            return launch_fewtok<NW, TG, FORM, false, kFewtokWs>(tiled, W, xq, xsc, y, slots, counters, M, N, K, chunk,
                                                                 accum, groups, 0, lds_ws, s);
    }
    return launch_fewtok<NW, TG, FORM, false>(tiled, W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, groups, 0,
                                              lds, s);
}

template <int TG, int FORM>
static hipError_t launch_fewtok_nw(int nw, int tiled, const uint8_t *W, const int8_t *xq, const void *xsc, float *y,
                                   float *slots, int *counters, int M, int N, int K, int chunk, int accum,
                                   hipStream_t s) {
    constexpr int P = fewtok_persist_waves<TG>();
    int groups, out_tiles;
    size_t lds;
    fewtok_grid<P, TG, FORM>(N, K, chunk, true, &groups, &out_tiles, &lds);
    if (out_tiles > 0)
        return launch_fewtok<P, TG, FORM, true>(tiled, W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, groups,
                                                out_tiles, lds, s);
    if (nw == 8)
        return launch_fewtok_tiles<8, TG, FORM>(tiled, W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, s);
    return launch_fewtok_tiles<4, TG, FORM>(tiled, W, xq, xsc, y, slots, counters, M, N, K, chunk, accum, s);
}

/* y (+)= X . W^T for 1 <= M <= 16, W in the layout of qtype (12 or
 * SERA_QTYPE_Q4K_TILED). form 0: row stage, MMVQ formula (M <= 8); form 1:
 * MMQ stage, MMQ formula. chunk: super-blocks per workgroup
 * (1..sera_fewtok_max_chunk(M), 0 = planned); when it splits K, slots holds
 * splits*M*N floats and counters sera_fewtok_groups() ints, zero on entry
 * and zero again after the kernel. */
extern "C" hipError_t sera_launch_q4k_fewtok_acc(uint32_t qtype, int form, const void *W, const void *stage,
                                                 float *y, float *slots, int *counters, int M, int N, int K,
                                                 int chunk, int accum, hipStream_t s) {
    const int tiled = qtype == SERA_QTYPE_Q4K_TILED;
    if ((!tiled && qtype != 12u) || (tiled && N % Q4K_TILE_ROWS)) return hipErrorInvalidValue;
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    if (c > sera_fewtok_max_chunk(M)) return hipErrorInvalidValue;   /* the LDS staging is sized for this */
    const char *base = (const char *)stage;
    const uint8_t *w = (const uint8_t *)W;
    if (form == 0) {
        const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
        return launch_fewtok_nw<1, 0>(nw, tiled, w, (const int8_t *)(base + L.qs), base + L.dsf, y, slots, counters,
                                      M, N, K, c, accum, s);
    }
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K);
    if (M > 8)
        return launch_fewtok_nw<2, 1>(nw, tiled, w, (const int8_t *)(base + L.qs), base + L.ds, y, slots, counters,
                                      M, N, K, c, accum, s);
    return launch_fewtok_nw<1, 1>(nw, tiled, w, (const int8_t *)(base + L.qs), base + L.ds, y, slots, counters, M, N,
                                  K, c, accum, s);
}

/* Workgroups along the rows of the launch sera_launch_q4k_fewtok_acc makes
 * on the current device (fewer than the row groups when the grid is
 * persistent), or -1 for an invalid chunk. */
extern "C" int sera_fewtok_grid(int form, int M, int N, int K, int chunk) {
    int nw, c;
    sera_fewtok_plan(M, N, K, &nw, &c);
    if (chunk > 0) c = chunk;
    if (c > sera_fewtok_max_chunk(M)) return -1;
    int groups = 0, out_tiles = 0;
    size_t lds = 0;
    const bool tg2 = form == 1 && M > 8;
    if (tg2) fewtok_grid<fewtok_persist_waves<2>(), 2, 1>(N, K, c, true, &groups, &out_tiles, &lds);
    else if (form == 1) fewtok_grid<fewtok_persist_waves<1>(), 1, 1>(N, K, c, true, &groups, &out_tiles, &lds);
    else fewtok_grid<fewtok_persist_waves<1>(), 1, 0>(N, K, c, true, &groups, &out_tiles, &lds);
    if (out_tiles > 0) return groups;
    return (N + 16 * nw - 1) / (16 * nw);
}
