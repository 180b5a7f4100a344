/*
 * q4k_mmvq.hip - Q4_K x Q8_1 matrix-vector kernel for M <= 8 (decode).
 *
 * Arithmetic of the reference MMVQ (cuda/mmq/vecdotq.cuh:505-527,864-908):
 *   y[c][n] = sum_blk ( d * sum_b sc_b * d8_b * I_b  -  dmin * sum_b m_b * d8_b * S_b )
 * with I_b = sum of q4*q8 over sub-block b (exact int32, v_dot4_i32_i8) and
 * S_b = sum of q8 over b (precomputed by the row quantizer into dsf).
 *
 * gfx950 mapping (wave64, HBM-bound, activation-stationary):
 *   - a Q4_K super-block is a 16-byte header (d, dmin, 12 scale bytes) and
 *     128 qs bytes in four 32-byte pairs; pair j holds sub-block 2j (low
 *     nibbles) and 2j+1 (high nibbles). Four lanes (a quad) take one block,
 *     lane q loading pair q with two 16-byte loads; a wave-wide load of 64
 *     lanes covers 8 consecutive blocks of 2 rows (lanes 32-63 take the
 *     second row).
 *   - the header is fetched as one dword per lane (lane q loads dword q) and
 *     broadcast to the quad with DPP quad_perm: 4 bytes per lane through
 *     the texture path instead of 16.
 *   - each lane loads the Q8_1 slice matching its pair (64 int8 + one float4
 *     of scales) once per block group and reuses it for all weight rows the
 *     lane walks (R/2), so activation traffic per weight byte drops by R/2.
 *     The two half-waves (rows of either parity) need the same slice: each
 *     loads one 32-byte half of the quants and one v_permlane32_swap per
 *     dword hands every lane both halves, halving the activation loads.
 *   - buffer loads with loop-invariant 32-bit lane offsets; the block-group
 *     and row steps live in the scalar offset, so the loop has no address
 *     arithmetic on the vector ALU.
 *   - the NW waves of a workgroup split the row's block groups (K). Partial
 *     sums are reduce-scattered across rows and lanes with xor butterflies in
 *     DPP / lane-swap form (no LDS permutes) and summed across waves through
 *     LDS in a fixed order, so results repeat bit for bit.
 *   - every kernel argument is read in one scalar-load round at entry
 *     (otherwise the compiler sinks some into the branches that use them
 *     and each workgroup waits on a second round before its first load).
 *   Measured on gate/up at one token (interleaved runs, 8 weight copies):
 *   the half-wave activation loads, the DPP butterflies and the single
 *   argument round together took the kernel from 13.85 to 13.26 us.
 */
#include "sera_launch.h"
#include "sera_dpp.h"

typedef unsigned v4u __attribute__((ext_vector_type(4)));
#define SERA_RSRC_FLAGS 0x00020000   /* gfx9 buffer descriptor word 3: 32-bit dword format */

/* DPP quad_perm broadcast of one lane of each quad to the whole quad. */
template <int CTRL>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, SERA_RSRC_FLAGS);
}

/* One halving step of the row reduce-scatter: lanes with bit O set keep
 * the upper half of v[0..2h) and receive the partner's copy of it. */
template <int O>
__device__ __forceinline__ void rs_halve(float *v, int h, int lane) {
    const bool up = (lane & O) != 0;
#pragma unroll
    for (int i = 0; i < h; i++) {
        const float send = up ? v[i] : v[i + h];
        const float keep = up ? v[i + h] : v[i];
        v[i] = keep + xor_partner<O>(send);
    }
}

template <int NCOLS, int HR>
struct MmvqRegs {
    v4i xa0[NCOLS], xa1[NCOLS], xb0[NCOLS], xb1[NCOLS];
    v4u f[NCOLS];
    uint32_t hw[HR];
    v4u qa[HR], qc[HR];
};

/* Up to SERA_MMVQ_GROUP weight matrices of one K that read the same
 * activations (q/k/v, gate/up): workgroups [tile_end[g-1], tile_end[g])
 * take matrix g. accum != 0 adds to y instead of overwriting it. */
#define SERA_MMVQ_GROUP 4
struct MmvqGroup {
    const uint8_t *W[SERA_MMVQ_GROUP];
    float *y[SERA_MMVQ_GROUP];
    int N[SERA_MMVQ_GROUP];
    int tile_end[SERA_MMVQ_GROUP];
    int count;
    int accum;
    int tiled;      /* weights in the 16-row tiled layout (every matrix) */
};

template <int NCOLS, int R, int NW, bool GROUPED, bool TILED>
__global__ __launch_bounds__(NW * 64) void sera_q4k_mmvq_kernel(
        MmvqGroup grp, const int8_t *__restrict__ xq, const float4 *__restrict__ dsf, int K) {
    {
        const void *a0 = grp.W[0], *a1 = grp.y[0], *a2 = xq, *a3 = dsf;
        const int a4 = grp.N[0], a5 = K, a6 = grp.accum;
        __asm__ volatile("" : : "s"(a0), "s"(a1), "s"(a2), "s"(a3), "s"(a4), "s"(a5), "s"(a6));
    }
    /* one matrix: its pointers come straight from the kernel arguments, so
     * the first loads issue without the dependent scalar loads of the
     * matrix selection (measured 2-4% on one-token launches) */
    int gi = 0;
    if constexpr (GROUPED) {
#pragma unroll
        for (int i = 1; i < SERA_MMVQ_GROUP; i++)
            if (i < grp.count && (int)blockIdx.x >= grp.tile_end[i - 1]) gi = i;
    }
    const uint8_t *__restrict__ W = grp.W[gi];
    float *__restrict__ y = grp.y[gi];
    const int N = grp.N[gi];
    const int tile = (int)blockIdx.x - (gi ? grp.tile_end[gi - 1] : 0);
    constexpr int HR = R / 2;              /* rows per lane */
    __shared__ float s_part[NW][R][NCOLS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane & 3;                /* sub-block pair */
    const int g = (lane >> 2) & 7;         /* block within the group of 8 */
    const int rs = lane >> 5;              /* row parity */
    /* The last tile is shifted back to end at row N (it recomputes rows of
     * its neighbour and stores only its own): the range check of a raw
     * buffer load covers the vector offset but not the scalar row step, so
     * no row past N may be addressed. The launcher keeps R <= N, or R = 2
     * where row 1 sits in the vector offset. */
    const int tile0 = tile * R;
    const int row0 = tile0 + R > N && N >= R ? N - R : tile0;
    const int nb = K / Q4K_QK;
    const int ngroups = (nb + 7) >> 3;
    /* row and block strides of the layout; a tile of R <= 16 rows never
     * crosses a 16-row tile of the tiled layout (N % 16 == 0 there) */
    const int rowbytes = q4k_row_stride(TILED, nb);
    constexpr int bstride = TILED ? Q4K_TILE_ROWS * Q4K_BLOCK_BYTES : Q4K_BLOCK_BYTES;
    const int nrows = min(R, N - row0);
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(W + q4k_block_offset(TILED, row0, 0, nb),
                  (uint32_t)(TILED ? (nb - 1) * bstride + nrows * Q4K_BLOCK_BYTES : nrows * rowbytes));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xq, (uint32_t)(NCOLS * K));
    const __amdgpu_buffer_rsrc_t rf = make_rsrc(dsf, (uint32_t)(NCOLS * (K / 64) * 16));
    const int vo_w = rs * rowbytes + g * bstride;
    const int vo_hdr = vo_w + 4 * q;
    const int vo_qs = vo_w + 16 + 32 * q;
    const int vo_xh = g * Q4K_QK + 64 * q + 32 * rs;
    const int vo_f = (g * 4 + q) * 16;
    const int sh = 16 * (q & 1);
    const bool hi_pair = q >= 2;

    auto load = [&](int bg, MmvqRegs<NCOLS, HR> &t) {
#pragma unroll
        for (int c = 0; c < NCOLS; c++) {
            /* lanes of row parity rs load quant half rs of the slice */
            const int so = c * K + bg * 2048;
            t.xa0[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo_xh, so, 0));
            t.xa1[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo_xh + 16, so, 0));
            t.f[c] = __builtin_amdgcn_raw_buffer_load_b128(rf, vo_f, c * (K / 4) + bg * 512, 0);
        }
#pragma unroll
        for (int r = 0; r < HR; r++) {
            const int so = 2 * r * rowbytes + bg * 8 * bstride;
            t.hw[r] = __builtin_amdgcn_raw_buffer_load_b32(rw, vo_hdr, so, 0);
            t.qa[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_qs, so, 0);
            t.qc[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_qs + 16, so, 0);
        }
    };

    float acc[HR][NCOLS];
#pragma unroll
    for (int r = 0; r < HR; r++)
#pragma unroll
        for (int c = 0; c < NCOLS; c++) acc[r][c] = 0.0f;

    /* the whole slice per lane, for the K loop at one token (where the
     * half-wave loads and their swaps measured 2% slower on down) */
    auto load_full = [&](int bg, MmvqRegs<NCOLS, HR> &t) {
#pragma unroll
        for (int c = 0; c < NCOLS; c++) {
            const int so = c * K + bg * 2048;
            const int vo = vo_xh - 32 * rs;
            t.xa0[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo, so, 0));
            t.xa1[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo + 16, so, 0));
            t.xb0[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo + 32, so, 0));
            t.xb1[c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, vo + 48, so, 0));
            t.f[c] = __builtin_amdgcn_raw_buffer_load_b128(rf, vo_f, c * (K / 4) + bg * 512, 0);
        }
#pragma unroll
        for (int r = 0; r < HR; r++) {
            const int so = 2 * r * rowbytes + bg * 8 * bstride;
            t.hw[r] = __builtin_amdgcn_raw_buffer_load_b32(rw, vo_hdr, so, 0);
            t.qa[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_qs, so, 0);
            t.qc[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_qs + 16, so, 0);
        }
    };

    /* after load(): the quant halves of the two half-waves, swapped, so
     * every lane holds low half xa (sub-block 2q) and high half xb (2q+1) */
    auto swap_halves = [&](MmvqRegs<NCOLS, HR> &t) {
#pragma unroll
        for (int c = 0; c < NCOLS; c++) {
            const v4i h0 = t.xa0[c], h1 = t.xa1[c];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const auto p0 = __builtin_amdgcn_permlane32_swap(h0[e], h0[e], false, false);
                const auto p1 = __builtin_amdgcn_permlane32_swap(h1[e], h1[e], false, false);
                t.xa0[c][e] = (int)p0[0];
                t.xb0[c][e] = (int)p0[1];
                t.xa1[c][e] = (int)p1[0];
                t.xb1[c][e] = (int)p1[1];
            }
        }
    };

    auto compute = [&](const MmvqRegs<NCOLS, HR> &t) {
#pragma unroll
        for (int r = 0; r < HR; r++) {
            const uint32_t h0 = quad_bcast<0x00>(t.hw[r]);
            const uint32_t s1 = quad_bcast<0x55>(t.hw[r]) >> sh;
            const uint32_t s2 = quad_bcast<0xAA>(t.hw[r]) >> sh;
            const uint32_t s3 = quad_bcast<0xFF>(t.hw[r]) >> sh;
            /* 6-bit (scale, min) of sub-blocks 2q, 2q+1 as byte pairs
             * (src/q3_quant.c:44-55 evaluated for both at once) */
            const uint32_t scp = hi_pair ? ((s3 & 0x0F0Fu) | ((s1 >> 2) & 0x3030u)) : (s1 & 0x3F3Fu);
            const uint32_t mp = hi_pair ? (((s3 >> 4) & 0x0F0Fu) | ((s2 >> 2) & 0x3030u)) : (s2 & 0x3F3Fu);
            const int scA = (int)(scp & 0xFFu), scB = (int)(scp >> 8);
            const float mA = (float)(mp & 0xFFu), mB = (float)(mp >> 8);
            const float d = h2f_bits(h0 & 0xffffu);
            const float dmin = h2f_bits(h0 >> 16);
            const uint32_t w[8] = {t.qa[r].x, t.qa[r].y, t.qa[r].z, t.qa[r].w,
                                   t.qc[r].x, t.qc[r].y, t.qc[r].z, t.qc[r].w};
            int lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                lo[i] = (int)(w[i] & 0x0F0F0F0Fu);
                hi[i] = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
            }
#pragma unroll
            for (int c = 0; c < NCOLS; c++) {
                int ia = __builtin_amdgcn_sdot4(lo[0], t.xa0[c].x, 0, false);
                ia = __builtin_amdgcn_sdot4(lo[1], t.xa0[c].y, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[2], t.xa0[c].z, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[3], t.xa0[c].w, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[4], t.xa1[c].x, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[5], t.xa1[c].y, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[6], t.xa1[c].z, ia, false);
                ia = __builtin_amdgcn_sdot4(lo[7], t.xa1[c].w, ia, false);
                int ib = __builtin_amdgcn_sdot4(hi[0], t.xb0[c].x, 0, false);
                ib = __builtin_amdgcn_sdot4(hi[1], t.xb0[c].y, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[2], t.xb0[c].z, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[3], t.xb0[c].w, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[4], t.xb1[c].x, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[5], t.xb1[c].y, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[6], t.xb1[c].z, ib, false);
                ib = __builtin_amdgcn_sdot4(hi[7], t.xb1[c].w, ib, false);
                const float d8A = __uint_as_float(t.f[c].x), d8B = __uint_as_float(t.f[c].y);
                const float dSA = __uint_as_float(t.f[c].z), dSB = __uint_as_float(t.f[c].w);
                /* |I| <= 32*15*127 and sc <= 63: the product fits a 24-bit multiply */
                const float sumd = d8A * (float)__mul24(ia, scA) + d8B * (float)__mul24(ib, scB);
                const float summ = dSA * mA + dSB * mB;
                acc[r][c] = fmaf(d, sumd, fmaf(-dmin, summ, acc[r][c]));
            }
        }
    };

    /* groups of this wave: wave, wave+NW, ...; all lanes of a quad share blk.
     * One group in flight per wave keeps registers low; occupancy (several
     * waves per SIMD) hides the HBM latency. With at most one group per
     * wave (K <= 8 * 256 * NW) the work is straight-line code. */
    if (ngroups <= NW) {
        if (wave < ngroups && wave * 8 + g < nb) {
            MmvqRegs<NCOLS, HR> cur;
            load(wave, cur);
            swap_halves(cur);
            compute(cur);
        }
    } else {
        for (int bg = wave; bg < ngroups; bg += NW) {
            if (bg * 8 + g < nb) {
                MmvqRegs<NCOLS, HR> cur;
                if constexpr (NCOLS == 1) {
                    load_full(bg, cur);
                } else {
                    load(bg, cur);
                    swap_halves(cur);
                }
                compute(cur);
            }
        }
    }

    /* reduce-scatter: after log2(HR) halvings each lane holds one row's
     * partial; the remaining xor steps finish the 32-lane sum. */
#pragma unroll
    for (int c = 0; c < NCOLS; c++) {
        float v[HR];
#pragma unroll
        for (int r = 0; r < HR; r++) v[r] = acc[r][c];
        int ri = 0;
        if constexpr (HR >= 8) { rs_halve<16>(v, 4, lane); ri = ri * 2 + ((lane >> 4) & 1); }
        if constexpr (HR >= 4) {
            constexpr int o = HR >= 8 ? 8 : 16;
            rs_halve<o>(v, 2, lane);
            ri = ri * 2 + ((lane & o) ? 1 : 0);
        }
        if constexpr (HR >= 2) {
            constexpr int o = HR >= 8 ? 4 : (HR >= 4 ? 8 : 16);
            rs_halve<o>(v, 1, lane);
            ri = ri * 2 + ((lane & o) ? 1 : 0);
        }
        constexpr int ofirst = HR >= 8 ? 2 : (HR >= 4 ? 4 : (HR >= 2 ? 8 : 16));
        float s = v[0];
        if constexpr (ofirst >= 16) s += xor_partner<16>(s);
        if constexpr (ofirst >= 8) s += xor_partner<8>(s);
        if constexpr (ofirst >= 4) s += xor_partner<4>(s);
        if constexpr (ofirst >= 2) s += xor_partner<2>(s);
        s += xor_partner<1>(s);
        if ((lane & (2 * ofirst - 1)) == 0) s_part[wave][2 * ri + rs][c] = s;
    }
    __syncthreads();
    if (threadIdx.x < R * NCOLS) {
        const int r = threadIdx.x / NCOLS, c = threadIdx.x % NCOLS;
        float v = s_part[0][r][c];
#pragma unroll
        for (int w = 1; w < NW; w++) v += s_part[w][r][c];
        if (row0 + r >= tile0 && row0 + r < N) {
            float *dst = y + (size_t)c * N + row0 + r;
            *dst = grp.accum ? *dst + v : v;
        }
    }
}

template <int NCOLS, int R, int NW>
static hipError_t launch_mmvq(MmvqGroup grp, const int8_t *xq, const float4 *dsf, int K, hipStream_t s) {
    int tiles = 0;
    for (int i = 0; i < grp.count; i++) {
        tiles += (grp.N[i] + R - 1) / R;
        grp.tile_end[i] = tiles;
    }
    /* the layout is a template argument: runtime strides cost the GGUF
     * instance 4 VGPRs, one wave per SIMD of occupancy */
    if (grp.count == 1 && grp.tiled)
        hipLaunchKernelGGL((sera_q4k_mmvq_kernel<NCOLS, R, NW, false, true>), dim3(tiles), dim3(NW * 64), 0, s, grp,
                           xq, dsf, K);
    else if (grp.count == 1)
        hipLaunchKernelGGL((sera_q4k_mmvq_kernel<NCOLS, R, NW, false, false>), dim3(tiles), dim3(NW * 64), 0, s, grp,
                           xq, dsf, K);
    else if (grp.tiled)
        hipLaunchKernelGGL((sera_q4k_mmvq_kernel<NCOLS, R, NW, true, true>), dim3(tiles), dim3(NW * 64), 0, s, grp,
                           xq, dsf, K);
    else
        hipLaunchKernelGGL((sera_q4k_mmvq_kernel<NCOLS, R, NW, true, false>), dim3(tiles), dim3(NW * 64), 0, s, grp,
                           xq, dsf, K);
    return hipGetLastError();
}

/* Rows per workgroup (even, 2..16), from interleaved sweeps on MI355X over
 * the Qwen3-32B shapes (weights streamed from HBM, kernel us):
 *   one token: 4;
 *   2-4 tokens: 8 where more rows per loaded activation slice pay for a
 *     smaller grid - a long K (down, 25600: 19.4 / 20.7 / 23.0 at 2 / 3 /
 *     4 tokens against 19.5 / 21.9 / 24.3 with 4) or a very tall matrix
 *     (LM head at 2: 75.1 against 81.9), or 3-4 tokens on 8192 rows and
 *     more (q: 7.5 / 8.4 against 7.8 / 9.1) - and 4 elsewhere (gate/up 16.0
 *     against 16.2, o 5.7 / 6.6 / 8.2 against 6.6 / 7.8 / 8.7, k/v 2.8 /
 *     3.1 / 3.5 against 3.4 / 4.0 / 4.5);
 *   5 tokens: 4 (k/v 3.8 against 4.1 with 2);
 *   6-8 tokens: 2 (the R/2 x M partial sums of 4 rows cost occupancy:
 *     k/v at 8 tokens 5.3 against 18.7). */
extern "C" int sera_mmvq_rows_per_wave(int N, int K, int M) {
    if (M <= 1) return 4;
    if (M <= 4) return (K >= 16384 || N >= 65536 || (M >= 3 && N >= 8192)) ? 8 : 4;
    if (M == 5) return 4;
    return 2;
}

/* Waves per workgroup: one per group of 8 blocks, at most 4. One token
 * (measured on MI355X, weights streamed from HBM): with 3 groups (K = 5120)
 * a fourth, idle wave is 1-2% faster, since a 4-wave workgroup puts one
 * wave on each SIMD of the CU; from 8 groups (K = 25600: 13) 8 waves are
 * 3-4% faster than 4, with more of the row's groups in flight at once.
 * Neither helps at 2-3 tokens, whose waves hold more registers. */
template <int NCOLS, int R>
static hipError_t dispatch_nw(int K, const MmvqGroup &grp, const int8_t *xq, const float4 *dsf, hipStream_t s) {
    const int ngroups = (K / Q4K_QK + 7) / 8;
    int nw = ngroups >= 4 ? 4 : ngroups;
    if (NCOLS == 1 && ngroups == 3) nw = 4;
    if (NCOLS == 1 && ngroups >= 8) nw = 8;
    switch (nw) {
        case 1: return launch_mmvq<NCOLS, R, 1>(grp, xq, dsf, K, s);
        case 2: return launch_mmvq<NCOLS, R, 2>(grp, xq, dsf, K, s);
        case 3: return launch_mmvq<NCOLS, R, 3>(grp, xq, dsf, K, s);
        case 8: if constexpr (NCOLS == 1) return launch_mmvq<NCOLS, R, 8>(grp, xq, dsf, K, s);
                [[fallthrough]];
        default: return launch_mmvq<NCOLS, R, 4>(grp, xq, dsf, K, s);
    }
}

template <int NCOLS>
static hipError_t dispatch_r(int r, const MmvqGroup &grp, const int8_t *xq, const float4 *dsf, int K,
                             hipStream_t s) {
    /* register budget: R/2 x M partial sums plus two sets of loads */
    if (NCOLS > 2 && r > 8) r = 8;
    if (NCOLS > 4 && r > 4) r = 4;
    switch (r) {
        case 16: if constexpr (NCOLS <= 2) return dispatch_nw<NCOLS, 16>(K, grp, xq, dsf, s);
                 [[fallthrough]];
        case 8: if constexpr (NCOLS <= 4) return dispatch_nw<NCOLS, 8>(K, grp, xq, dsf, s);
                [[fallthrough]];
        case 4: return dispatch_nw<NCOLS, 4>(K, grp, xq, dsf, s);
        default: return dispatch_nw<NCOLS, 2>(K, grp, xq, dsf, s);
    }
}

/* count weight matrices (W[i], N[i] rows, output y[i]) of one K on one row
 * stage; rows = 0 picks the rows per workgroup from the smallest N. */
extern "C" hipError_t sera_launch_q4k_mmvq_group(uint32_t qtype, int count, const void *const *W, float *const *y,
                                                 const int *N, const void *stage, int M, int K, int rows, int accum,
                                                 hipStream_t s) {
    if (count < 1 || count > SERA_MMVQ_GROUP) return hipErrorInvalidValue;
    const int tiled = qtype == SERA_QTYPE_Q4K_TILED;
    if (!tiled && qtype != 12u) return hipErrorInvalidValue;
    for (int i = 0; i < count; i++)
        if (tiled && N[i] % Q4K_TILE_ROWS) return hipErrorInvalidValue;
    const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
    const char *base = (const char *)stage;
    const int8_t *xq = (const int8_t *)(base + L.qs);
    const float4 *dsf = (const float4 *)(base + L.dsf);
    MmvqGroup grp = {};
    int nmin = N[0];
    for (int i = 0; i < count; i++) {
        grp.W[i] = (const uint8_t *)W[i];
        grp.y[i] = y[i];
        grp.N[i] = N[i];
        if (N[i] < nmin) nmin = N[i];
    }
    grp.count = count;
    grp.accum = accum;
    grp.tiled = tiled;
    if (rows <= 0) rows = sera_mmvq_rows_per_wave(nmin, K, M);
    while (rows > 2 && rows > nmin) rows >>= 1;   /* the shifted last tile needs R <= N */
    if (tiled && rows > Q4K_TILE_ROWS) rows = Q4K_TILE_ROWS;
    switch (M) {
        case 1: return dispatch_r<1>(rows, grp, xq, dsf, K, s);
        case 2: return dispatch_r<2>(rows, grp, xq, dsf, K, s);
        case 3: return dispatch_r<3>(rows, grp, xq, dsf, K, s);
        case 4: return dispatch_r<4>(rows, grp, xq, dsf, K, s);
        case 5: return dispatch_r<5>(rows, grp, xq, dsf, K, s);
        case 6: return dispatch_r<6>(rows, grp, xq, dsf, K, s);
        case 7: return dispatch_r<7>(rows, grp, xq, dsf, K, s);
        case 8: return dispatch_r<8>(rows, grp, xq, dsf, K, s);
        default: return hipErrorInvalidValue;
    }
}

extern "C" hipError_t sera_launch_q4k_mmvq(uint32_t qtype, const void *W, const void *stage, float *y,
                                           int M, int N, int K, int rows, hipStream_t s) {
    return sera_launch_q4k_mmvq_group(qtype, 1, &W, &y, &N, stage, M, K, rows, 0, s);
}
