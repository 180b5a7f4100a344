/*
 * q4k_select.hip - gathered-row consumers of a quantized weight matrix:
 * the selected-row LM head (candidate logits) and the embedding row gather.
 *
 * Reference: candidate_logits_kernel / candidate_logits_batched_kernel
 * (src/q3_forward.cu:329-370, 566-607) compute, per (branch, candidate),
 *   logit = sum_k w[id][k] * hidden[branch][k]
 * in fp32 with w the dequantized weight (no Q8_1 on this path), and
 * embedding_kernel (:291-322) writes hidden[t][k] = w[id_t][k]. Both take
 * Q4_K or Q6_K rows.
 *
 * Dequant follows src/q3_quant.c:57-103 in fp32 with the same expression
 * order and no contraction: Q4_K (d*sc)*q - dmin*m, Q6_K (d*sc)*(q-32). The
 * Q6_K byte mapping is the GGUF one of q3_quant.c (and of the MMVQ/MMQ
 * kernels), not the one of the reference's device twin q6_value_dev
 * (:86-110), which leaves out the 128-weight half offset of ql/qh, takes
 * qh[l] instead of qh[l mod 32] and group 2*(l/16) + (l%32 >= 16) instead
 * of 2*(l/32) + (l%32)/16, so it agrees with q3_quant.c only on some
 * weights of each block.
 *
 * Q6_K rows come as GGUF bytes (qtype 14) or in the split device layout
 * (SERA_QTYPE_Q6K_SPLIT: 208-byte aligned ql/qh/sc blocks and a separate
 * fp16 d array); Q4_K rows as GGUF bytes (12) or in the 16-row tiled layout
 * (SERA_QTYPE_Q4K_TILED: the same blocks, ordered by 16-row tile, then
 * super-block, then row). Each layout gives the same values as its GGUF
 * bytes.
 *
 * gfx950 mapping: lane l of a wave takes weights 4l..4l+3 of each 256-weight
 * block (one sub-block, one group scale), reads its bytes as aligned dwords
 * through a buffer resource (GGUF Q6_K blocks are 2-byte aligned: funnel
 * shifts put the bytes in place) and its activations as one float4. A
 * candidate logit is one workgroup: four waves over quarters of the row,
 * each reduced with xor shuffles, then the four sums in wave order. An
 * embedding row is one wave per block.
 */
#include "sera_launch.h"

/* No floating-point contraction in this file: the values here must follow
 * the reference's separately rounded multiplies and adds (hipcc fuses a * b
 * + c into one FMA by default, and the _rn intrinsics are plain operators
 * that do not prevent it). Explicit fmaf calls are unaffected. */
#pragma clang fp contract(off)

#define SEL_RSRC_FLAGS 0x00020000   /* gfx9 buffer descriptor word 3: 32-bit dword format */

namespace {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sel_rsrc(const void *p, uint64_t bytes) {
    const uint64_t b = (bytes + 15) & ~(uint64_t)15;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(b > 0x7fffffffu ? 0x7fffffffu : b), SEL_RSRC_FLAGS);
}

/* 4 bytes at any byte offset */
__device__ __forceinline__ uint32_t sel_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t a = off & ~3u;
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(r, a, 0, 0);
    if ((off & 3u) == 0) return lo;
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(r, a + 4, 0, 0);
    return __builtin_amdgcn_alignbit(hi, lo, (off & 3u) * 8u);
}

/* Block bytes of a row in each layout: Q4_K 144, Q6_K GGUF 210, Q6_K split
 * 208 (ql, qh, sc; d in the separate array). */
template <int QT>
__host__ __device__ constexpr uint32_t sel_block_bytes() {
    return QT == 12 || QT == (int)SERA_QTYPE_Q4K_TILED ? Q4K_BLOCK_BYTES
           : QT == 14                                   ? Q6K_GGUF_BYTES
                                                        : Q6K_SPLIT_QBYTES;
}

/* From one block of a row to the next: the block size, or a 16-row tile of
 * blocks in the tiled Q4_K layout. */
template <int QT>
__host__ __device__ constexpr uint32_t sel_block_step() {
    return QT == (int)SERA_QTYPE_Q4K_TILED ? Q4K_TILE_ROWS * Q4K_BLOCK_BYTES : sel_block_bytes<QT>();
}

/* Byte offset of row id's first block. */
template <int QT>
__device__ __forceinline__ uint64_t sel_row_offset(uint32_t id, int nb) {
    return QT == (int)SERA_QTYPE_Q4K_TILED ? (uint64_t)q4k_block_offset(1, id, 0, (size_t)nb)
                                           : (uint64_t)id * nb * sel_block_bytes<QT>();
}

/* Weights e0..e0+3 (e0 % 4 == 0) of block `blk` of the row starting at byte
 * `row` (relative to the resource); dsplit = the block's fp16 d bits for the
 * split layout. */
template <int QT>
__device__ __forceinline__ void sel_dequant4(__amdgpu_buffer_rsrc_t r, uint32_t row, int blk, int e0, uint32_t dsplit,
                                             float w[4]) {
    if (QT == 12 || QT == (int)SERA_QTYPE_Q4K_TILED) {
        const uint32_t b = row + (uint32_t)blk * sel_block_step<QT>();
        const uint32_t h0 = __builtin_amdgcn_raw_buffer_load_b32(r, b, 0, 0);
        const uint32_t s0 = __builtin_amdgcn_raw_buffer_load_b32(r, b + 4, 0, 0);
        const uint32_t s1 = __builtin_amdgcn_raw_buffer_load_b32(r, b + 8, 0, 0);
        const uint32_t s2 = __builtin_amdgcn_raw_buffer_load_b32(r, b + 12, 0, 0);
        const int j = e0 >> 5, l = e0 & 31;
        const uint32_t qw = __builtin_amdgcn_raw_buffer_load_b32(r, b + 16 + 32 * (j >> 1) + l, 0, 0);
        uint32_t sc, m;
        q4k_scale_min(j, s0, s1, s2, &sc, &m);
        const float d = h2f_bits(h0 & 0xffffu), dmin = h2f_bits(h0 >> 16);
        const float d1 = __fmul_rn(d, (float)sc);
        const float m1 = __fmul_rn(dmin, (float)m);
        const uint32_t nib = (j & 1) ? (qw >> 4) : qw;
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = __fsub_rn(__fmul_rn(d1, (float)((nib >> (8 * i)) & 15u)), m1);
    } else {
        const uint32_t b = row + (uint32_t)blk * sel_block_bytes<QT>();
        const int jh = e0 >> 7, k = (e0 & 127) >> 5, l = e0 & 31;
        uint32_t ql, qh, sd, dd;
        if (QT == 14) {
            ql = sel_load4(r, b + 64 * jh + 32 * (k & 1) + l);
            qh = sel_load4(r, b + 128 + 32 * jh + l);
            sd = sel_load4(r, b + 192 + 8 * jh + 2 * k + (l >> 4));   /* byte 0 = the group scale */
            dd = sel_load4(r, b + 208);                                  /* low half = d */
        } else {   /* split: b is 16-byte aligned, l % 4 == 0 */
            ql = __builtin_amdgcn_raw_buffer_load_b32(r, b + 64 * jh + 32 * (k & 1) + l, 0, 0);
            qh = __builtin_amdgcn_raw_buffer_load_b32(r, b + 128 + 32 * jh + l, 0, 0);
            const uint32_t so = b + 192 + 8 * jh + 2 * k + (l >> 4);
            sd = __builtin_amdgcn_raw_buffer_load_b32(r, so & ~3u, 0, 0) >> (8 * (so & 3u));
            dd = dsplit;
        }
        const int sc = (int)(sd << 24) >> 24;
        const float dsc = __fmul_rn(h2f_bits(dd & 0xffffu), (float)sc);
        const uint32_t nib = (k >= 2) ? (ql >> 4) : ql;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = (int)(((nib >> (8 * i)) & 15u) | (((qh >> (8 * i + 2 * k)) & 3u) << 4)) - 32;
            w[i] = __fmul_rn(dsc, (float)q);
        }
    }
}

}  // namespace

/* One workgroup per (branch, candidate): its four waves take a quarter of
 * the row's blocks each (blocks [w nb/4, (w+1) nb/4)), and the four wave
 * sums are added in wave order. Invalid ids (>= N) give NaN. Wd: the split
 * layout's d array (unused otherwise). Four waves per row measured 1.1-1.5x
 * faster than one on the 16 x 128-candidate LM head (more rows in flight). */
template <int QT>
__global__ __launch_bounds__(256) void sera_candidate_logits_kernel(
        const uint8_t *__restrict__ W, const uint16_t *__restrict__ Wd, uint64_t wbytes, int N, int K,
        const float *__restrict__ hidden, const uint32_t *__restrict__ ids, int per_branch, int total,
        float *__restrict__ logits) {
    __shared__ float s_part[4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int index = blockIdx.x;
    const uint32_t id = ids[index];
    const bool valid = id < (uint32_t)N;
    float acc = 0.0f;
    if (valid) {
        const int nb = K / Q4K_QK;
        const uint64_t start = sel_row_offset<QT>(id, nb);
        const uint64_t base = start & ~(uint64_t)15;
        const __amdgpu_buffer_rsrc_t r = sel_rsrc(W + base, wbytes - base);
        const uint32_t row = (uint32_t)(start - base);
        const float *x = hidden + (size_t)(index / per_branch) * K;
        const uint16_t *drow = QT == SERA_QTYPE_Q6K_SPLIT ? Wd + (size_t)id * nb : nullptr;
        const int b1 = (wave + 1) * nb / 4;
        for (int blk = wave * nb / 4; blk < b1; blk++) {
            float w[4];
            sel_dequant4<QT>(r, row, blk, 4 * lane, QT == SERA_QTYPE_Q6K_SPLIT ? drow[blk] : 0u, w);
            const float4 xv = *(const float4 *)(x + blk * Q4K_QK + 4 * lane);
            acc = fmaf(w[0], xv.x, acc);
            acc = fmaf(w[1], xv.y, acc);
            acc = fmaf(w[2], xv.z, acc);
            acc = fmaf(w[3], xv.w, acc);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
    }
    if (lane == 0) s_part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
        logits[index] = valid ? ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3] : __builtin_nanf("");
}

/* One wave per (token, block): hidden[t][blk*256 + 4l + i] = w[id_t][...].
 * Tokens with ids >= N are left untouched, as in the reference. */
template <int QT>
__global__ __launch_bounds__(256) void sera_embedding_kernel(
        const uint8_t *__restrict__ W, const uint16_t *__restrict__ Wd, uint64_t wbytes, int N, int K,
        const uint32_t *__restrict__ ids, int tokens, float *__restrict__ hidden) {
    const int lane = threadIdx.x & 63;
    const int nb = K / Q4K_QK;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (int64_t)tokens * nb) return;
    const int t = (int)(unit / nb), blk = (int)(unit - (int64_t)t * nb);
    const uint32_t id = ids[t];
    if (id >= (uint32_t)N) return;
    const uint64_t start = sel_row_offset<QT>(id, nb);
    const uint64_t base = start & ~(uint64_t)15;
    const __amdgpu_buffer_rsrc_t r = sel_rsrc(W + base, wbytes - base);
    float w[4];
    sel_dequant4<QT>(r, (uint32_t)(start - base), blk, 4 * lane,
                     QT == SERA_QTYPE_Q6K_SPLIT ? Wd[(size_t)id * nb + blk] : 0u, w);
    *(float4 *)(hidden + (size_t)t * K + (size_t)blk * Q4K_QK + 4 * lane) = make_float4(w[0], w[1], w[2], w[3]);
}

namespace {
/* bytes the kernels address through the resource, and the d array */
uint64_t sel_qbytes(int qtype, int N, int K) {
    const uint64_t nblk = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    return nblk * (qtype == 12 || qtype == (int)SERA_QTYPE_Q4K_TILED ? Q4K_BLOCK_BYTES
                   : qtype == 14                                        ? Q6K_GGUF_BYTES
                                                                        : Q6K_SPLIT_QBYTES);
}
}  // namespace

/* qtype 12 (Q4_K), SERA_QTYPE_Q4K_TILED, 14 (Q6_K GGUF bytes) or
 * SERA_QTYPE_Q6K_SPLIT. */
extern "C" hipError_t sera_launch_candidate_logits(int qtype, const void *W, int N, int K, const float *hidden,
                                                   const uint32_t *ids, int branches, int per_branch,
                                                   float *logits, hipStream_t s) {
    const int total = branches * per_branch;
    const uint64_t qb = sel_qbytes(qtype, N, K);
    const uint8_t *w = (const uint8_t *)W;
    const uint16_t *wd = (const uint16_t *)(w + qb);
    const dim3 grid(total);
    if (qtype == 12)
        hipLaunchKernelGGL(sera_candidate_logits_kernel<12>, grid, dim3(256), 0, s, w, wd, qb, N, K, hidden, ids,
                           per_branch, total, logits);
    else if (qtype == (int)SERA_QTYPE_Q4K_TILED)
        hipLaunchKernelGGL(sera_candidate_logits_kernel<(int)SERA_QTYPE_Q4K_TILED>, grid, dim3(256), 0, s, w, wd, qb,
                           N, K, hidden, ids, per_branch, total, logits);
    else if (qtype == 14)
        hipLaunchKernelGGL(sera_candidate_logits_kernel<14>, grid, dim3(256), 0, s, w, wd, qb, N, K, hidden, ids,
                           per_branch, total, logits);
    else
        hipLaunchKernelGGL(sera_candidate_logits_kernel<(int)SERA_QTYPE_Q6K_SPLIT>, grid, dim3(256), 0, s, w, wd, qb,
                           N, K, hidden, ids, per_branch, total, logits);
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_embedding(int qtype, const void *W, int N, int K, const uint32_t *ids, int tokens,
                                            float *hidden, hipStream_t s) {
    const uint64_t qb = sel_qbytes(qtype, N, K);
    const uint8_t *w = (const uint8_t *)W;
    const uint16_t *wd = (const uint16_t *)(w + qb);
    const int64_t units = (int64_t)tokens * (K / Q4K_QK);
    const dim3 grid((unsigned)((units + 3) / 4));
    if (qtype == 12)
        hipLaunchKernelGGL(sera_embedding_kernel<12>, grid, dim3(256), 0, s, w, wd, qb, N, K, ids, tokens, hidden);
    else if (qtype == (int)SERA_QTYPE_Q4K_TILED)
        hipLaunchKernelGGL(sera_embedding_kernel<(int)SERA_QTYPE_Q4K_TILED>, grid, dim3(256), 0, s, w, wd, qb, N, K,
                           ids, tokens, hidden);
    else if (qtype == 14)
        hipLaunchKernelGGL(sera_embedding_kernel<14>, grid, dim3(256), 0, s, w, wd, qb, N, K, ids, tokens, hidden);
    else
        hipLaunchKernelGGL(sera_embedding_kernel<(int)SERA_QTYPE_Q6K_SPLIT>, grid, dim3(256), 0, s, w, wd, qb, N, K,
                           ids, tokens, hidden);
    return hipGetLastError();
}
