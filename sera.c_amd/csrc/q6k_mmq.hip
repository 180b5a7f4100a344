/*
 * q6k_mmq.hip - Q6_K x Q8_1 tiled GEMM on CDNA4 fp16 MFMA (prefill, M > 8).
 *
 * Arithmetic of the reference MMQ for Q6_K (tensor-core branch of
 * vec_dot_q6_K_q8_1_mma, cuda/mmq/mmq.cuh:2687-2786, tiles from
 * load_tiles_q6_K :2512-2596, D4 activations): per 32-wide sub-block b of a
 * super-block with its two 16-wide groups,
 *   J_b = sc_2b * I_2b + sc_2b+1 * I_2b+1       (exact integer, :2775)
 *   y   = sum_blk d * sum_b d8_b * J_b           (fp32 d8, d per block, :2784)
 * where I_g = sum (q - 32) * q8 over group g.
 *
 * gfx950 mapping. The int8 group scales change every 16 weights, so an int8
 * MFMA result would need two scale multiplies, a convert and an FMA per
 * element and sub-block on the VALU. Instead the scales go into the weight
 * operand, exactly: with sc = 16*sh + sl (sh in [-8, 7], sl in [0, 15]),
 * (q-32)*sl and 16*(q-32)*sh are integers of at most 13 significant bits,
 * exact in fp16, and the int8 activation quants are exact in fp16 too. Two
 * v_mfma_f32_32x32x16_f16 per 16 K (one per part) accumulate
 * sum q8 * (q-32) * sc, every product and partial sum an integer below 2^24,
 * so the fp32 result IS the integer J_b, bit for bit. The epilogue is then
 * one FMA per element and sub-block (J_b * d8_b), plus one per block (d).
 *   - weights are the A operand: lane = weight row (MFMA row), so the group
 *     scales are per-lane values. A lane of half h takes, for sub-block
 *     (j, q), weights l = 16h + [0, 16) of the quarter: one 16-wide group,
 *     one scale. Its runs (4 ql, 2 qh, the 16 scales and d of the block)
 *     come from the weight tile in LDS, funnel-shifted into place on GGUF
 *     bytes (rows are only 2-byte aligned). The raw quant bytes become fp16
 *     (1024 + q) by v_perm under exponent byte 0x64, and one packed fp16 FMA
 *     per pair gives (q-32)*s.
 *   - activations are the B operand: lane = token (MFMA column), so d8 is
 *     one LDS word per lane and sub-block; output element r of a lane is
 *     weight row 8(r/4) + 4h + r%4, whose d the wave passes through LDS
 *     once per K step.
 *   - activations (fp16 quants, fp32 d8) for the workgroup's tokens go
 *     global -> LDS directly (16-byte loads to LDS, 1 KB per wave
 *     instruction); 16-byte chunks are XOR-swizzled by token so a
 *     half-wave's 32 tokens reading one chunk hit distinct banks. The
 *     quantizer writes d8 transposed per K step so it lands in LDS as
 *     [sub-block][token].
 *   - tiles: 32 or 64 tokens x 128 weight rows per workgroup, 4 waves along
 *     the rows (one 32 x 32 MFMA tile per token tile), two workgroups per
 *     CU. 32 tokens double-buffer the activations per K step; 64 tokens
 *     (the operand build shared by twice the tokens) keep one buffer, in
 *     two K halves, each reloaded while the other is read.
 *   - schedules: split-K with a fixed-order reduce launch when tiles are
 *     few; or the tail schedule (whole tiles, then K pieces handed off
 *     through per-tile counters, summed in piece order by the last piece).
 */
#include "sera_launch.h"

typedef __attribute__((address_space(3))) void q6m_lds_void;
typedef __attribute__((address_space(1))) const void q6m_global_cvoid;
typedef _Float16 q6h2 __attribute__((ext_vector_type(2)));
typedef _Float16 q6v8h __attribute__((ext_vector_type(8)));
typedef uint32_t q6v4u __attribute__((ext_vector_type(4)));
typedef float q6v4f __attribute__((ext_vector_type(4)));

#define Q6K_BLOCK_BYTES 210
#define Q6M_RSRC_FLAGS 0x00020000   /* gfx9 buffer descriptor word 3: 32-bit dword format */
#define Q6M_BN 128
#define Q6M_WCH 15    /* 16-byte LDS chunks per weight row and K step: a 210-byte block at any
                         2-byte phase needs 14; the 15th spreads row starts over more banks */
/* GGUF bytes: row r of the tile sits at slot 15 r + (r + 16) / 32, one pad
 * slot after row 15 of each 32. A wave's rows r and r + 16 then start 4
 * banks apart instead of on the same bank, and consecutive rows, whose
 * 2-byte phases differ by 8 bytes when K / 256 = 4 mod 8 (K = 5120,
 * 25600), interleave, so a half-wave's dword reads of its 32 rows' runs
 * hit 32 distinct banks. */

template <int BM, int XB>
struct alignas(16) Q6MmqSmem {
    alignas(16) _Float16 xs[XB][BM][Q4K_QK];
    alignas(16) float d8[2][8][BM];
    alignas(16) float dw[4][32];   /* each wave's 32 row scales d of the K step */
    alignas(16) uint32_t wd[Q6M_BN];   /* split layout: the dword holding each row's d */
    alignas(16) uint8_t w[31 * 1024];   /* Q6M_BN rows of Q6M_WCH chunks, one pad chunk per 32 rows on GGUF bytes */
};

namespace {

/* Consecutive workgroup ids go to consecutive XCDs (8 on MI355X); give each
 * XCD a contiguous run of tiles, token tiles fastest, so workgroups on one
 * XCD share weight rows in its L2. */
__device__ __forceinline__ int q6m_tile_of(int wg, int ntiles) {
    const int nx = 8;
    const int full = (ntiles / nx) * nx;
    if (wg >= full) return wg;
    const int per = ntiles / nx;
    return (wg % nx) * per + wg / nx;
}

__device__ __forceinline__ q6h2 q6m_h2(uint32_t u) { return __builtin_bit_cast(q6h2, u); }

/* 16 bytes that start `sh` bits into the 5 dwords p[0..4] */
__device__ __forceinline__ q6v4u q6m_align16(const uint32_t *p, uint32_t sh) {
    q6v4u r;
    r.x = __builtin_amdgcn_alignbit(p[1], p[0], sh);
    r.y = __builtin_amdgcn_alignbit(p[2], p[1], sh);
    r.z = __builtin_amdgcn_alignbit(p[3], p[2], sh);
    r.w = __builtin_amdgcn_alignbit(p[4], p[3], sh);
    return r;
}

/* raw 6-bit quants of quarter Q (bits 2Q..2Q+1 of qh, low nibble of ql for
 * Q < 2, high nibble for Q >= 2), four per dword (src/q3_quant.c:88-95) */
template <int Q>
__device__ __forceinline__ uint32_t q6m_raw(uint32_t ql, uint32_t qh) {
    const uint32_t nib = (Q >= 2 ? (ql >> 4) : ql) & 0x0F0F0F0Fu;
    const uint32_t hi = Q == 0 ? (qh << 4) : Q == 1 ? (qh << 2) : Q == 2 ? qh : (qh >> 2);
    return nib | (hi & 0x30303030u);
}

__device__ __forceinline__ int q6m_sext8(uint32_t w, int sh) { return (int)(w << (24 - sh)) >> 24; }

/* Workgroup barriers that wait only for what they name: this wave's LDS reads
 * (and, for the second, all but its VM most recent vector memory loads), never the
 * vmcnt(0) a __syncthreads adds. The memory clobber keeps the compiler from
 * moving loads or LDS accesses across. */
__device__ __forceinline__ void q6m_barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int VM>
__device__ __forceinline__ void q6m_barrier_vm() {
    static_assert(VM >= 0 && VM < 16, "vmcnt immediate");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

}  // namespace

/* Buffer-resource word 3 for raw 32-bit accesses and the sc1 cache-policy
 * bit of the buffer builtins' aux operand (the tail hand-off's slots). */
#define Q6M_SLOT_RSRC_FLAGS 0x00020000
#define Q6M_SC1 16

/* Split-K (TAIL false): grid (tiles, K splits); splits > 1 write fp32
 * partials per split for a reduce launch.
 * Tail (TAIL true): the first dp_tiles workgroups each run a whole tile
 * (XCD-contiguous order); the remaining tiles are cut along K into `pieces`
 * near-equal ranges, one workgroup per (tile, range), ranges major and
 * token tiles fastest within one. Each piece stores its sums to its own
 * slot (`partial`) with sc1 stores, waits for them and bumps the tile's
 * counter; the piece that completes the count adds the slots in piece
 * order, stores the tile and resets the counter. No workgroup waits on
 * another, and the result does not depend on which piece ends last. */
template <int TT, int WPE, bool SPLIT, bool TAIL = false>
__global__ __launch_bounds__(256, WPE) void sera_q6k_mmq_kernel(
        const uint8_t *__restrict__ W, const uint16_t *__restrict__ Wd, uint64_t wbytes, const _Float16 *__restrict__ xh,
        const float *__restrict__ d8t, float *__restrict__ y, float *__restrict__ partial, int *__restrict__ counters,
        int M, int Mpad, int N, int K, int kb_per_split, int dp_tiles, int pieces, int accum) {
    constexpr int BM = 32 * TT;
    /* activation buffers: two for 32 tokens; one for 64 (the 64 KB of a
     * second would leave one workgroup per CU) */
    constexpr int XB = TT == 1 ? 2 : 1;
    /* weight-tile slots (16-byte chunks): GGUF bytes add one pad slot after
     * row 15 of every 32 (the row placement above) */
    constexpr int WSLOTS = Q6M_BN * Q6M_WCH + (SPLIT ? 0 : Q6M_BN / 32);
    constexpr int WINST = (WSLOTS + 63) / 64;   /* load-to-LDS instructions per weight tile */
    __shared__ __attribute__((aligned(16))) Q6MmqSmem<BM, XB> sm;
    static_assert(WINST * 1024 <= (int)sizeof(sm.w), "weight tile");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   /* uniform: scalar LDS addresses and branches */
    const int l32 = lane & 31, h = lane >> 5;
    const int ntt = Mpad / BM, nrt = (N + Q6M_BN - 1) / Q6M_BN;
    const int nb = K / Q4K_QK;
    int tile, kb0, kb1, piece = 0;
    if constexpr (TAIL) {
        const int wg = blockIdx.x;
        if (wg < dp_tiles) {
            tile = q6m_tile_of(wg, dp_tiles);
            kb0 = 0;
            kb1 = nb;
        } else {
            /* each range's tiles in the XCD-contiguous order of a whole
             * grid, as the splits of the split-K grid */
            const int R = ntt * nrt - dp_tiles;
            piece = (wg - dp_tiles) / R;
            tile = dp_tiles + q6m_tile_of(wg - dp_tiles - piece * R, R);
            kb0 = piece * nb / pieces;
            kb1 = (piece + 1) * nb / pieces;
        }
    } else {
        tile = q6m_tile_of(blockIdx.x, ntt * nrt);
        kb0 = blockIdx.y * kb_per_split;
        kb1 = min(nb, kb0 + kb_per_split);
    }
    const int n0 = (tile / ntt) * Q6M_BN, m0 = (tile % ntt) * BM;
    /* GGUF: 210-byte blocks at any 2-byte phase; split: 208-byte aligned
     * blocks (ql, qh, sc) and d from the separate array Wd */
    constexpr uint32_t BB = SPLIT ? Q6K_SPLIT_QBYTES : Q6K_BLOCK_BYTES;
    const uint32_t rb = (uint32_t)nb * BB;

    /* weights: resource from the tile's first row (16-byte aligned down) to
     * the end of the matrix rounded up to 16 bytes (a chunk that straddles the
     * end must not read as zero); rows >= N are clamped (never stored) */
    const uint64_t gbase = ((uint64_t)n0 * rb) & ~(uint64_t)15;
    const uint64_t rem = ((wbytes - gbase) + 15) & ~(uint64_t)15;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(W + gbase), (short)0, (int)(rem > 0x7fffffffu ? 0x7fffffffu : rem), Q6M_RSRC_FLAGS);

    /* weight tile of K step kb -> LDS: row r's block from its 16-byte-aligned
     * start, chunks 0..13 at w[r*240 + 16c]; 1 KB per wave-instruction */
    /* split layout: 16-byte aligned blocks, so a lane's offset is its row's
     * chunk plus kb * 208 (the scalar offset); the two chunks past the block
     * load the row's first chunk again (same line, never read) */
    /* tile loads per wave: a literal, since an array bound that depends on
     * SPLIT here made the host pass drop the kernel stubs */
    constexpr int WI = 8;
    static_assert((WINST + 3) / 4 == WI, "tile loads per wave");
    /* loop-invariant lane offsets of the tile loads. GGUF: the slot's row
     * start plus 16 c, or 2^31 for a slot that holds nothing (beyond any
     * resource range, so it loads zeros); a K step adds kb * 210 and rounds
     * down to 16 bytes, (g & ~15) + 16 c = (g + 16 c) & ~15 */
    uint32_t wvo[WI];
#pragma unroll
    for (int i = 0; i < WI; i++) {
        const int inst = wave + 4 * i;
        if constexpr (SPLIT) {
            const int f = inst * 64 + lane;
            const int r = f / Q6M_WCH, c = f - r * Q6M_WCH;
            const uint32_t g = (uint32_t)((uint64_t)min(n0 + r, N - 1) * rb - gbase);
            wvo[i] = g + (c < 13 ? 16u * (uint32_t)c : 0u);
        } else {
            /* slot f: 32-row group f / 481, pad slot 240 of each */
            const int f = inst * 64 + lane;
            const int grp = f / (32 * Q6M_WCH + 1), q = f - grp * (32 * Q6M_WCH + 1);
            const int qq = q < 16 * Q6M_WCH ? q : q - 1;
            const int rr = qq / Q6M_WCH, c = qq - rr * Q6M_WCH;
            const int r = 32 * grp + rr;
            const bool live = inst < WINST && f < WSLOTS && q != 16 * Q6M_WCH && c < 14;
            wvo[i] = live ? (uint32_t)((uint64_t)min(n0 + min(r, Q6M_BN - 1), N - 1) * rb - gbase) + 16u * (uint32_t)c
                          : 0x80000000u;
        }
    }
    auto issue_w = [&](int kb) {
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const int inst = wave + 4 * i;
            if (inst < WINST) {
                if constexpr (SPLIT) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (q6m_lds_void *)&sm.w[inst * 1024], 16, wvo[i],
                                                             kb * (int)BB, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (q6m_lds_void *)&sm.w[inst * 1024], 16,
                                                             (wvo[i] + (uint32_t)kb * BB) & ~15u, 0, 0, 0);
                }
            }
        }
        if constexpr (SPLIT) {
            /* d of the 128 rows (2 bytes each in Wd [N][K/256]): the aligned
             * dword holding it, which never leaves the page of its valid half */
            if (wave >= 2) {
                const int row = min(n0 + 64 * (wave - 2) + lane, N - 1);
                const size_t idx = (size_t)row * nb + kb;
                __builtin_amdgcn_global_load_lds((q6m_global_cvoid *)(Wd + (idx & ~(size_t)1)),
                                                 (q6m_lds_void *)&sm.wd[64 * (wave - 2)], 4, 0, 0);
            }
        }
    };
    /* activations of K step kb: BM tokens x 256 fp16 and 8 x BM fp32 d8.
     * Two buffers: token rows of 512 bytes, chunk c of token t in column
     * c ^ (t & 31). One buffer: two K halves of BM rows of 256 bytes (chunk c
     * in half c >> 4, column (c & 15) ^ (t & 15)), loaded half by half. */
    /* Buffer loads to LDS from resources over the tile's token rows: the
     * lane's part of each address is a loop-invariant vector offset, the
     * token row and K step a scalar offset, so the K loop spends no vector
     * instructions on addresses (global loads from 64-bit lane pointers
     * took one 64-bit add each). */
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16 *>(xh + (size_t)m0 * K), (short)0, (int)(2u * (uint32_t)BM * (uint32_t)K), Q6M_RSRC_FLAGS);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(d8t + m0), (short)0, (int)(4u * (uint32_t)(8 * nb) * (uint32_t)Mpad), Q6M_RSRC_FLAGS);
    /* activation loads per wave and K step (or K half); a literal array
     * bound, as with the tile loads below */
    constexpr int XI = 4;
    static_assert((XB == 1 ? BM / 16 : BM / 8) == XI, "activation loads per wave");
    uint32_t xoff[XI];
#pragma unroll
    for (int i = 0; i < XI; i++) {
        const int inst = wave + 4 * i;
        if constexpr (XB == 1) {
            const int tl = lane >> 4, tok = 4 * inst + tl;
            xoff[i] = (uint32_t)(2 * (tl * K + 8 * ((lane & 15) ^ (tok & 15))));
        } else {
            const int tl = lane >> 5, tok = 2 * inst + tl;
            xoff[i] = (uint32_t)(2 * (tl * K + 8 * ((lane & 31) ^ (tok & 31))));
        }
    }
    auto issue_xh = [&](int kb, int half) {
#pragma unroll
        for (int i = 0; i < BM / 16; i++) {
            const int inst = wave + 4 * i;          /* 1 KB = four tokens' half rows */
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (q6m_lds_void *)&sm.xs[0][0][(half * BM + 4 * inst) * 128], 16,
                                                     xoff[i], 2 * (4 * inst * K + kb * Q4K_QK + 128 * half), 0, 0);
        }
    };
    auto issue_xs = [&](int kb, int buf) {
#pragma unroll
        for (int i = 0; i < BM / 8; i++) {
            const int inst = wave + 4 * i;          /* 1 KB = two tokens */
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (q6m_lds_void *)&sm.xs[buf][2 * inst][0], 16, xoff[i],
                                                     2 * (2 * inst * K + kb * Q4K_QK), 0, 0);
        }
    };
    /* by the last waves, which issue one weight-tile load fewer; the lane's
     * four floats (b, t..t+3) of [8][BM] sit at f = (wave - W0) * 256 +
     * 4 lane = b BM + t, and at b Mpad + t in the stage's K step */
    constexpr int W0 = 4 - BM / 32;
    const int d8f = (wave - W0) * 256 + lane * 4;
    const uint32_t d8off = (uint32_t)(4 * ((d8f / BM) * Mpad + d8f % BM));
    auto issue_d8 = [&](int kb, int buf) {
        if (wave >= W0) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (q6m_lds_void *)&sm.d8[buf][0][(wave - W0) * 256], 16, d8off,
                                                     4 * kb * 8 * Mpad, 0, 0);
        }
    };

    /* this lane's weight row (B column) and its phase in the LDS window */
    const int wr = 32 * wave + l32;
    const uint32_t rowg = (uint32_t)((uint64_t)min(n0 + wr, N - 1) * rb - gbase);
    /* split layout: which half of its wd dword is this row's d (parity of
     * row * nb + kb) */
    const int dpar = SPLIT ? (min(n0 + wr, N - 1) & 1) * (nb & 1) : 0;

    v16f acc[TT], tmp[TT];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            acc[t][r] = 0.0f;
            tmp[t][r] = 0.0f;
        }

    if (kb0 < kb1) {
        issue_w(kb0);
        issue_d8(kb0, 0);
        if constexpr (XB == 2) {
            issue_xs(kb0, 0);
        } else {
            issue_xh(kb0, 0);
            issue_xh(kb0, 1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int kb = kb0; kb < kb1; kb++) {
        const int buf = (kb - kb0) & 1;
        const int kn = min(kb + 1, kb1 - 1);
        /* the lane's runs of this block from LDS: ql[64j + 32p + 16h + 0..15],
         * qh[32j + 16h + 0..15], bytes 192..207 (scales) and d */
        const uint32_t base = SPLIT ? (uint32_t)wr * (Q6M_WCH * 16)
                                    : (uint32_t)(wr * Q6M_WCH + ((wr + 16) >> 5)) * 16u +
                                          ((rowg + (uint32_t)kb * BB) & 15u);
        const uint32_t sh = (base & 2u) * 8u;
        q6v4u QL[4], QH[2], SC;
        uint32_t dword = 0;
        if constexpr (SPLIT) {
#pragma unroll
            for (int i = 0; i < 4; i++) QL[i] = *(const q6v4u *)&sm.w[base + 32u * i + 16u * h];
#pragma unroll
            for (int i = 0; i < 2; i++) QH[i] = *(const q6v4u *)&sm.w[base + 128u + 32u * i + 16u * h];
            SC = *(const q6v4u *)&sm.w[base + 192u];
        } else {
            /* every run starts a multiple of 16 bytes after the block, so
             * (base + X) & ~3 = (base & ~3) + X: one address register, the
             * runs at immediate offsets */
            const uint32_t *w4 = (const uint32_t *)&sm.w[(base & ~3u) + 16u * h];
            constexpr uint32_t X[6] = {0u, 32u, 64u, 96u, 128u, 160u};
#pragma unroll
            for (int i = 0; i < 6; i++) {
                const uint32_t *p = w4 + X[i] / 4;
                const uint32_t v[5] = {p[0], p[1], p[2], p[3], p[4]};
                if (i < 4) QL[i] = q6m_align16(v, sh);
                else QH[i - 4] = q6m_align16(v, sh);
            }
            const uint32_t *p = (const uint32_t *)&sm.w[(base & ~3u) + 192u];
            const uint32_t v[5] = {p[0], p[1], p[2], p[3], p[4]};
            SC = q6m_align16(v, sh);
            dword = v[4];
        }
        if constexpr (SPLIT) dword = sm.wd[wr] >> (16 * ((dpar + kb) & 1));
        const float d = h2f_bits((SPLIT ? dword : dword >> sh) & 0xffffu);
        sm.dw[wave][l32] = d;   /* read back by this wave only, for the rows its outputs hold */
        /* every wave has its runs: the weight buffer is free (one activation
         * buffer: the second K half's loads may still be in flight) */
        if constexpr (XB == 2) {
            __syncthreads();
            if (kb + 1 < kb1) {
                issue_w(kb + 1);
                issue_d8(kb + 1, buf ^ 1);   /* buffer last read one step ago, freed by the barrier */
                issue_xs(kb + 1, buf ^ 1);
            }
        } else {
            /* Unconditional: the last step loads its own K step again into
             * buffers it has finished reading. The wait counts below then
             * hold on every step, and the step body has no branch (a branch
             * lets the compiler sink the scaling FMAs past it and spill the
             * MFMA results they wait for). */
            q6m_barrier_lds();
            issue_w(kn);
            issue_d8(kn, buf ^ 1);
        }

        /* The lane's group scales sc = 16*sh + sl of sub-blocks b = 2m, 2m+1
         * (scale bytes 2b + h, all in dword m), as fp16 pairs: sl/16, -66*sl,
         * sh and -1056*sh. A byte v < 64 becomes the fp16 1024 + v under
         * exponent byte 0x64; sh + 8 = (high nibble) ^ 8 for sh = sc >> 4. */
        q6h2 SL16[4], CL[4], SH[4], CH[4];
        {
            const uint32_t sel = h ? 0x04030401u : 0x04020400u;
            const q6h2 b1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            const q6h2 b1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
            const q6h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
            const q6h2 k66 = {(_Float16)-66.0f, (_Float16)-66.0f};
            const q6h2 k1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const uint32_t lo = SC[m] & 0x0F0F0F0Fu;
                const uint32_t hi = ((SC[m] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
                const q6h2 sl = q6m_h2(__builtin_amdgcn_perm(0x64646464u, lo, sel)) - b1024;
                const q6h2 shv = q6m_h2(__builtin_amdgcn_perm(0x64646464u, hi, sel)) - b1032;
                SL16[m] = sl * k16;      /* exact: sl <= 15 */
                CL[m] = sl * k66;
                SH[m] = shv;
                CH[m] = shv * k1056;
            }
        }

        /* sub-block (j, q): 2 x 2 MFMAs per token tile (K halves u, scale
         * parts). The activations are 16*q8, so the parts are
         * (q-32)*sh and (q-32)*sl/16, both exact in fp16: fma(1024+q, s, c)
         * with c = -1056*sh or -66*sl. */
        auto mfma_sb = [&](int j, int q, v16f (&C)[TT]) {
            const int b = 4 * j + q, m = b >> 1, odd = b & 1;
            const _Float16 sl16 = odd ? SL16[m].y : SL16[m].x, cl = odd ? CL[m].y : CL[m].x;
            const _Float16 shh = odd ? SH[m].y : SH[m].x, ch = odd ? CH[m].y : CH[m].x;
            const q6h2 s_hi = {shh, shh}, s_lo = {sl16, sl16}, c_hi = {ch, ch}, c_lo = {cl, cl};
#pragma unroll
            for (int u = 0; u < 2; u++) {
                uint32_t v[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t ql = QL[2 * j + (q & 1)][2 * u + e], qh = QH[j][2 * u + e];
                    v[e] = q == 0 ? q6m_raw<0>(ql, qh) : q == 1 ? q6m_raw<1>(ql, qh)
                         : q == 2 ? q6m_raw<2>(ql, qh) : q6m_raw<3>(ql, qh);
                }
                q6v8h Blo, Bhi;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    /* fp16 (1024 + q) pairs from bytes 2(k&1), 2(k&1)+1 of v[k>>1] */
                    const q6h2 t = q6m_h2(__builtin_amdgcn_perm(0x64646464u, v[k >> 1],
                                                                (k & 1) ? 0x04030402u : 0x04010400u));
                    const q6h2 lo = __builtin_elementwise_fma(t, s_lo, c_lo);   /* (q-32)*sl/16 */
                    const q6h2 hi = __builtin_elementwise_fma(t, s_hi, c_hi);   /* (q-32)*sh */
                    Blo[2 * k] = lo.x;
                    Blo[2 * k + 1] = lo.y;
                    Bhi[2 * k] = hi.x;
                    Bhi[2 * k + 1] = hi.y;
                }
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const int tok = 32 * t + l32;
                    const int chunk = (16 * j + 4 * q + 2 * h + u) ^ (tok & 31);
                    const q6v8h X = *(const q6v8h *)&sm.xs[buf][tok][8 * chunk];
                    const v16f zero = {};
                    C[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Blo, X, u == 0 ? zero : C[t], 0, 0, 0);
                    C[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Bhi, X, C[t], 0, 0, 0);
                }
            }
        };
        /* the same for one token tile, the operand build split out */
        auto build_b = [&](int j, int q, q6v8h (&Blo)[2], q6v8h (&Bhi)[2]) {
            const int b = 4 * j + q, m = b >> 1, odd = b & 1;
            const _Float16 sl16 = odd ? SL16[m].y : SL16[m].x, cl = odd ? CL[m].y : CL[m].x;
            const _Float16 shh = odd ? SH[m].y : SH[m].x, ch = odd ? CH[m].y : CH[m].x;
            const q6h2 s_hi = {shh, shh}, s_lo = {sl16, sl16}, c_hi = {ch, ch}, c_lo = {cl, cl};
#pragma unroll
            for (int u = 0; u < 2; u++) {
                uint32_t v[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t ql = QL[2 * j + (q & 1)][2 * u + e], qh = QH[j][2 * u + e];
                    v[e] = q == 0 ? q6m_raw<0>(ql, qh) : q == 1 ? q6m_raw<1>(ql, qh)
                         : q == 2 ? q6m_raw<2>(ql, qh) : q6m_raw<3>(ql, qh);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const q6h2 t = q6m_h2(__builtin_amdgcn_perm(0x64646464u, v[k >> 1],
                                                                (k & 1) ? 0x04030402u : 0x04010400u));
                    const q6h2 lo = __builtin_elementwise_fma(t, s_lo, c_lo);
                    const q6h2 hi = __builtin_elementwise_fma(t, s_hi, c_hi);
                    Blo[u][2 * k] = lo.x;
                    Blo[u][2 * k + 1] = lo.y;
                    Bhi[u][2 * k] = hi.x;
                    Bhi[u][2 * k + 1] = hi.y;
                }
            }
        };
        auto mfma_t = [&](int j, int q, int t, const q6v8h (&Blo)[2], const q6v8h (&Bhi)[2], v16f &C) {
            const int tok = 32 * t + l32;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int col = (4 * q + 2 * h + u) ^ (tok & 15);
                const q6v8h X = *(const q6v8h *)&sm.xs[0][0][(j * BM + tok) * 128 + 8 * col];
                const v16f zero = {};
                C = __builtin_amdgcn_mfma_f32_32x32x16_f16(Blo[u], X, u == 0 ? zero : C, 0, 0, 0);
                C = __builtin_amdgcn_mfma_f32_32x32x16_f16(Bhi[u], X, C, 0, 0, 0);
            }
        };
        auto epi_t = [&](int j, int q, int t, const v16f &C) {
            const float f = sm.d8[buf][4 * j + q][32 * t + l32];
#pragma unroll
            for (int r = 0; r < 16; r++) tmp[t][r] = fmaf(C[r], f, tmp[t][r]);
        };
        /* C is the exact integer J_b; scale by the tokens' d8 */
        auto epi_sb = [&](int j, int q, const v16f (&C)[TT]) {
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const float f = sm.d8[buf][4 * j + q][32 * t + l32];
#pragma unroll
                for (int r = 0; r < 16; r++) tmp[t][r] = fmaf(C[t][r], f, tmp[t][r]);
            }
        };
        if constexpr (XB == 2) {
            /* software pipeline: the MFMAs of sub-block b+1 run while the VALU
             * scales sub-block b */
            v16f Ca[TT], Cb[TT];
            mfma_sb(0, 0, Ca);
            mfma_sb(0, 1, Cb);
            epi_sb(0, 0, Ca);
            mfma_sb(0, 2, Ca);
            epi_sb(0, 1, Cb);
            mfma_sb(0, 3, Cb);
            epi_sb(0, 2, Ca);
            mfma_sb(1, 0, Ca);
            epi_sb(0, 3, Cb);
            mfma_sb(1, 1, Cb);
            epi_sb(1, 0, Ca);
            mfma_sb(1, 2, Ca);
            epi_sb(1, 1, Cb);
            mfma_sb(1, 3, Cb);
            epi_sb(1, 2, Ca);
            epi_sb(1, 3, Cb);
        } else {
            /* 64 tokens: both token tiles' MFMAs use one operand build; the
             * MFMAs of one token tile run while the VALU scales the other's
             * previous result (one accumulator per token tile) */
            v16f C0, C1;
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const int j = b >> 2, q = b & 3;
                if (b == 4) {
                    /* the first K half is read by every wave; the second has
                     * landed: every wave issued at least 8 loads after it
                     * (waves 0-1: 8 of the weight tile; 2-3: 7, d8 and, on the
                     * split layout, d) */
                    q6m_barrier_vm<8>();
                    issue_xh(kn, 0);
                }
                q6v8h Blo[2], Bhi[2];
                build_b(j, q, Blo, Bhi);
                mfma_t(j, q, 0, Blo, Bhi, C0);
                if (b > 0) epi_t((b - 1) >> 2, (b - 1) & 3, 1, C1);
                mfma_t(j, q, 1, Blo, Bhi, C1);
                epi_t(j, q, 0, C0);
            }
            epi_t(1, 3, 1, C1);
        }
        /* output element r of a lane is weight row 8(r/4) + 4h + r%4 of the
         * wave's 32: that row's d from the lane that decoded it */
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const q6v4f d4 = *(const q6v4f *)&sm.dw[wave][8 * g + 4 * h];
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    acc[t][4 * g + e] = fmaf(tmp[t][4 * g + e], d4[e], acc[t][4 * g + e]);
                    tmp[t][4 * g + e] = 0.0f;
                }
        }
        if constexpr (XB == 2) {
            __builtin_amdgcn_s_waitcnt(0);   /* this thread's loads to LDS have landed */
            __syncthreads();
        } else {
            q6m_barrier_vm<0>();   /* loads landed; the second K half is read by every wave */
            issue_xh(kn, 1);
        }
    }
    if constexpr (XB == 1) __builtin_amdgcn_s_waitcnt(0);   /* no load to LDS outlives the workgroup */

    /* lane holds token m0 + 32t + l32 for weight rows
     * n0 + 32*wave + 8(r/4) + 4h + r%4: four consecutive outputs per g */
    auto store = [&](float *out, bool add) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const int m = m0 + 32 * t + l32;
            if (m >= M) continue;
            float *row = out + (size_t)m * N;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int col = n0 + 32 * wave + 8 * g + 4 * h;
                if ((N & 3) == 0 && col < N) {   /* 16-byte aligned, all four in range */
                    q6v4f v = {acc[t][4 * g], acc[t][4 * g + 1], acc[t][4 * g + 2], acc[t][4 * g + 3]};
                    if (add) v += *(const q6v4f *)(row + col);
                    *(q6v4f *)(row + col) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (col + e < N) row[col + e] = add ? row[col + e] + acc[t][4 * g + e] : acc[t][4 * g + e];
                }
            }
        }
    };
    if constexpr (!TAIL) {
        if (partial) store(partial + (size_t)blockIdx.y * M * N, false);
        else store(y, accum != 0);
        return;
    } else {
        if ((int)blockIdx.x < dp_tiles || pieces == 1) {
            store(y, accum != 0);
            return;
        }
        /* slot (r, p): TT * 16 floats per thread as 16-byte chunks, chunk j
         * of thread tid at byte (j * 256 + tid) * 16 of the slot; sc1 stores
         * and loads, as the counter's agent-scope atomics, so no stale line
         * of another XCD's L2 is read */
        __shared__ int s_last;
        const int r = tile - dp_tiles;
        constexpr int kChunks = TT * 4;
        constexpr int kSlotBytes = TT * 16 * 256 * 4;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            partial + (size_t)r * pieces * (TT * 16 * 256), (short)0, pieces * kSlotBytes, Q6M_SLOT_RSRC_FLAGS);
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const q6v4f v = {acc[j / 4][4 * (j & 3)], acc[j / 4][4 * (j & 3) + 1], acc[j / 4][4 * (j & 3) + 2],
                             acc[j / 4][4 * (j & 3) + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(q6v4u, v), rs, (j * 256 + tid) * 16,
                                                   piece * kSlotBytes, Q6M_SC1);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(&counters[r], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == pieces - 1;
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) __hip_atomic_store(&counters[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        /* every piece's sums, this one's included, from the slots in piece
         * order (this one's stores were acknowledged before the counter moved) */
        for (int p = 0; p < pieces; p++) {
#pragma unroll
            for (int j = 0; j < kChunks; j++) {
                const q6v4f v = __builtin_bit_cast(
                    q6v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, (j * 256 + tid) * 16, p * kSlotBytes, Q6M_SC1));
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc[j / 4][4 * (j & 3) + e] = p == 0 ? v[e] : acc[j / 4][4 * (j & 3) + e] + v[e];
            }
        }
        store(y, accum != 0);
    }
}

/* Token tile: 64 (the weight operand build, the VALU bound, shared by twice
 * the tokens) when the padded rows divide by 64 and the 64-token grid holds
 * at least 1024 (tile, super-block) pairs; below that the 32-token tile's
 * twice as many workgroups are faster (attn_v 1024 x 5120 at 64-256 tokens). */
extern "C" int sera_q6k_mmq_tile_tokens(int M, int N, int K) {
    const int mp = sera_q6k_mmq_padded_rows(M);
    if (mp % 64) return 32;
    const long pairs = (long)(mp / 64) * ((N + Q6M_BN - 1) / Q6M_BN) * (K / Q4K_QK);
    return pairs >= 1024 ? 64 : 32;
}

/* K splits: double while the grid holds fewer than 1024 (tile, split)
 * workgroups (two resident per CU, two rounds on 256 CUs) and each split
 * keeps at least 2 super-blocks. */
extern "C" int sera_q6k_mmq_splits(int M, int N, int K) {
    const int bm = sera_q6k_mmq_tile_tokens(M, N, K);
    const int tiles = ((M + bm - 1) / bm) * ((N + Q6M_BN - 1) / Q6M_BN);
    const int nkb = K / Q4K_QK;
    int s = 1;
    while (tiles * s < 1024 && nkb / (s * 2) >= 2 && s < 16) s *= 2;
    return s;
}

template <int TT, int WPE, bool SPLIT>
static hipError_t launch_q6k_mmq(const uint8_t *W, const uint16_t *Wd, uint64_t wbytes, const _Float16 *xh,
                                 const float *d8t, float *y, float *partial, int M, int Mpad, int N, int K, int splits,
                                 int accum, hipStream_t s) {
    constexpr int BM = 32 * TT;
    const int tiles = (Mpad / BM) * ((N + Q6M_BN - 1) / Q6M_BN);
    const int nkb = K / Q4K_QK;
    const int per = (nkb + splits - 1) / splits;
    splits = (nkb + per - 1) / per;
    hipLaunchKernelGGL((sera_q6k_mmq_kernel<TT, WPE, SPLIT, false>), dim3(tiles, splits), dim3(256), 0, s, W, Wd,
                       wbytes, xh, d8t, y, splits > 1 ? partial : nullptr, nullptr, M, Mpad, N, K, per, 0, 1, accum);
    if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
    if (splits == 1) return hipSuccess;
    return sera_launch_splitk_reduce_acc(partial, y, (size_t)M * N, splits, accum, s);
}

/* stage: the Q6_K MMQ stage for Mpad = sera_q6k_mmq_padded_rows(M) rows;
 * partial: splits*M*N floats when splits > 1 (M*N % 4 == 0); accum != 0
 * adds the product to y. qtype 14: W is GGUF bytes; SERA_QTYPE_Q6K_SPLIT:
 * W is the split layout. */
extern "C" hipError_t sera_launch_q6k_mmq_acc(uint32_t qtype, const void *W, const void *stage, float *y,
                                              float *partial, int M, int N, int K, int splits, int accum,
                                              hipStream_t s) {
    const int Mpad = sera_q6k_mmq_padded_rows(M);
    const sera_stage_layout L = sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const _Float16 *xh = (const _Float16 *)(base + L.qs);
    const float *d8t = (const float *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    const uint64_t nblk = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    if (splits < 1) splits = 1;
    const bool wide = sera_q6k_mmq_tile_tokens(M, N, K) == 64;
    if (qtype == SERA_QTYPE_Q6K_SPLIT) {
        const uint16_t *wd = (const uint16_t *)(w + nblk * Q6K_SPLIT_QBYTES);
        return wide ? launch_q6k_mmq<2, 2, true>(w, wd, nblk * Q6K_SPLIT_QBYTES, xh, d8t, y, partial, M, Mpad, N, K,
                                                 splits, accum, s)
                    : launch_q6k_mmq<1, 2, true>(w, wd, nblk * Q6K_SPLIT_QBYTES, xh, d8t, y, partial, M, Mpad, N, K,
                                                 splits, accum, s);
    }
    return wide ? launch_q6k_mmq<2, 2, false>(w, nullptr, nblk * Q6K_BLOCK_BYTES, xh, d8t, y, partial, M, Mpad, N, K,
                                              splits, accum, s)
                : launch_q6k_mmq<1, 2, false>(w, nullptr, nblk * Q6K_BLOCK_BYTES, xh, d8t, y, partial, M, Mpad, N, K,
                                              splits, accum, s);
}

extern "C" hipError_t sera_launch_q6k_mmq(uint32_t qtype, const void *W, const void *stage, float *y, float *partial,
                                          int M, int N, int K, int splits, hipStream_t s) {
    return sera_launch_q6k_mmq_acc(qtype, W, stage, y, partial, M, N, K, splits, 0, s);
}

/* Output tiles of the Q6_K tile kernel for this shape (tokens x 128 rows). */
extern "C" int sera_q6k_mmq_tiles(int M, int N, int K) {
    const int bm = sera_q6k_mmq_tile_tokens(M, N, K);
    return (sera_q6k_mmq_padded_rows(M) / bm) * ((N + Q6M_BN - 1) / Q6M_BN);
}

/* Slot floats the tail schedule needs: one tile of sums per (split tile,
 * piece). */
extern "C" size_t sera_q6k_mmq_tail_slot_floats(int M, int N, int K, int dp_tiles, int pieces) {
    const int T = sera_q6k_mmq_tiles(M, N, K);
    if (pieces <= 1 || dp_tiles >= T) return 0;
    return (size_t)(T - dp_tiles) * (size_t)pieces * (size_t)sera_q6k_mmq_tile_tokens(M, N, K) * Q6M_BN;
}

template <int TT, bool SPLIT>
static hipError_t launch_q6k_tail(const uint8_t *W, const uint16_t *Wd, uint64_t wbytes, const _Float16 *xh,
                                  const float *d8t, float *y, float *slots, int *counters, int M, int Mpad, int N,
                                  int K, int dp, int pieces, int accum, hipStream_t s) {
    const int T = (Mpad / (32 * TT)) * ((N + Q6M_BN - 1) / Q6M_BN);
    if (pieces <= 1) {
        dp = T;
        pieces = 1;
    }
    const int grid = dp + (T - dp) * pieces;
    hipLaunchKernelGGL((sera_q6k_mmq_kernel<TT, 2, SPLIT, true>), dim3(grid), dim3(256), 0, s, W, Wd, wbytes, xh,
                       d8t, y, slots, counters, M, Mpad, N, K, 0, dp, pieces, accum);
    return hipGetLastError() == hipSuccess ? hipSuccess : hipErrorLaunchFailure;
}

/* The tail schedule: dp_tiles whole tiles, the other tiles in `pieces` K
 * ranges (0 <= dp_tiles <= tiles, 1 <= pieces <= K/256); slots:
 * sera_q6k_mmq_tail_slot_floats floats; counters: one int per split tile,
 * zero, left zero. */
extern "C" hipError_t sera_launch_q6k_mmq_tail_acc(uint32_t qtype, const void *W, const void *stage, float *y,
                                                   float *slots, int *counters, int M, int N, int K, int dp_tiles,
                                                   int pieces, int accum, hipStream_t s) {
    const int Mpad = sera_q6k_mmq_padded_rows(M);
    const sera_stage_layout L = sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K);
    const char *base = (const char *)stage;
    const _Float16 *xh = (const _Float16 *)(base + L.qs);
    const float *d8t = (const float *)(base + L.ds);
    const uint8_t *w = (const uint8_t *)W;
    const uint64_t nblk = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    const bool wide = sera_q6k_mmq_tile_tokens(M, N, K) == 64;
    if (qtype == SERA_QTYPE_Q6K_SPLIT) {
        const uint16_t *wd = (const uint16_t *)(w + nblk * Q6K_SPLIT_QBYTES);
        return wide ? launch_q6k_tail<2, true>(w, wd, nblk * Q6K_SPLIT_QBYTES, xh, d8t, y, slots, counters, M, Mpad,
                                               N, K, dp_tiles, pieces, accum, s)
                    : launch_q6k_tail<1, true>(w, wd, nblk * Q6K_SPLIT_QBYTES, xh, d8t, y, slots, counters, M, Mpad,
                                               N, K, dp_tiles, pieces, accum, s);
    }
    return wide ? launch_q6k_tail<2, false>(w, nullptr, nblk * Q6K_BLOCK_BYTES, xh, d8t, y, slots, counters, M, Mpad,
                                            N, K, dp_tiles, pieces, accum, s)
                : launch_q6k_tail<1, false>(w, nullptr, nblk * Q6K_BLOCK_BYTES, xh, d8t, y, slots, counters, M, Mpad,
                                            N, K, dp_tiles, pieces, accum, s);
}
