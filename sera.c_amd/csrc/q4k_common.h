/*
 * q4k_common.h - shared definitions for the gfx950 Q4_K linear kernels.
 *
 * GGUF Q4_K super-block (256 weights, 144 bytes), as in the reference's
 * src/q3_quant.h:28-33 and cuda/mmq/ggml-common.h:313-328:
 *   bytes 0-1   d     fp16  scale of the 6-bit sub-block scales
 *   bytes 2-3   dmin  fp16  scale of the 6-bit sub-block mins
 *   bytes 4-15  12 bytes of packed 6-bit (scale, min) for 8 sub-blocks
 *   bytes 16-143 qs[128]: sub-block j uses qs[(j/2)*32 + l], low nibble for
 *                even j, high nibble for odd j
 * Weight of sub-block j, element l: d*sc_j*q - dmin*m_j.
 *
 * Q8_1 activation stages (this library's device layout; the values are the
 * reference's block_q8_1 {half2 ds; int8 qs[32]} values, stored split):
 *   row stage (MMVQ):  qs  int8   [M][K]
 *                      ds  half2  [M][K/32]   (fp16 d, fp16 sum of x)
 *                      dsf float4 [M][K/64]   (d_2p, d_2p+1, d_2p*S_2p, d_2p+1*S_2p+1)
 *                                               S = sum of the 32 int8 quants
 *   mmq stage (MMQ):   qs  int8   [Mpad][K]
 *                      ds  half2  [Mpad][K/32]
 *   Q6_K mmq stage:    qs  fp16   [Mpad][K]          (16 x the int8 quants, exact)
 *                      ds  float  [K/256][8][Mpad]   (fp32 D4 scale d, per
 *                                  256-wide K step, sub-block, token)
 */
#ifndef SERA_Q4K_COMMON_H
#define SERA_Q4K_COMMON_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define Q4K_QK 256
#define Q4K_BLOCK_BYTES 144
#define Q8_QK 32

/* Q4_K weight layouts: qtype 12 keeps the GGUF bytes, row after row;
 * SERA_QTYPE_Q4K_TILED is this library's 16-row tiled device layout, the
 * same blocks reordered so that super-block b of 16 consecutive rows is one
 * 2304-byte run: block (row r, super-block b) at
 * ((r / 16) * (K / 256) + b) * 2304 + (r % 16) * 144. N must be a multiple
 * of 16. */
#ifndef SERA_QTYPE_Q4K_TILED
#define SERA_QTYPE_Q4K_TILED 268u
#endif
#define Q4K_TILE_ROWS 16

/* Byte offset of block (r, b) of an N x K matrix with nkb = K / 256. */
__host__ __device__ static inline size_t q4k_block_offset(int tiled, size_t r, size_t b, size_t nkb) {
    return tiled ? (((r >> 4) * nkb + b) * Q4K_TILE_ROWS + (r & 15)) * Q4K_BLOCK_BYTES
                 : (r * nkb + b) * Q4K_BLOCK_BYTES;
}
/* Bytes from block (r, b) to block (r, b + 1), and from row r to row r + 1
 * of the same tile (tiled) or of the matrix (GGUF). */
__host__ __device__ static inline int q4k_block_stride(int tiled) {
    return tiled ? Q4K_TILE_ROWS * Q4K_BLOCK_BYTES : Q4K_BLOCK_BYTES;
}
__host__ __device__ static inline int q4k_row_stride(int tiled, int nkb) {
    return tiled ? Q4K_BLOCK_BYTES : nkb * Q4K_BLOCK_BYTES;
}

/* Byte offsets of the sub-arrays of a stage, 256-byte aligned. */
static inline size_t sera_align256(size_t v) { return (v + 255u) & ~(size_t)255u; }

typedef struct {
    size_t qs;      /* int8  [rows][K]      */
    size_t ds;      /* half2 [rows][K/32]   */
    size_t dsf;     /* float4 [rows][K/64]  (row stage only, else 0) */
    size_t total;
} sera_stage_layout;

static inline sera_stage_layout sera_row_stage_layout(size_t rows, size_t K) {
    sera_stage_layout L;
    L.qs = 0;
    L.ds = sera_align256(rows * K);
    L.dsf = sera_align256(L.ds + rows * (K / 32) * 4);
    L.total = sera_align256(L.dsf + rows * (K / 64) * 16);
    return L;
}

static inline sera_stage_layout sera_mmq_stage_layout(size_t rows_padded, size_t K) {
    sera_stage_layout L;
    L.qs = 0;
    L.ds = sera_align256(rows_padded * K);
    L.dsf = 0;
    L.total = sera_align256(L.ds + rows_padded * (K / 32) * 4);
    return L;
}

/* What a quantizer reads as its activation row (the producer fused into
 * the Q8_1 quantize): kind 0 x itself; 1 RMSNorm, (x * inv_rms) * gamma
 * with inv_rms = 1 / sqrt(mean(x^2) + eps); 2 SiLU-mul,
 * (x / (1 + exp(-x))) * x2. */
typedef struct {
    int kind;
    const float *x2;
    const float *gamma;
    float eps;
} sera_producer;

/* Q6_K MMQ stage: Mpad is a multiple of the 32-token tile. */
static inline sera_stage_layout sera_q6k_mmq_stage_layout(size_t rows_padded, size_t K) {
    sera_stage_layout L;
    L.qs = 0;
    L.ds = sera_align256(rows_padded * K * 2);
    L.dsf = 0;
    L.total = sera_align256(L.ds + rows_padded * (K / 32) * 4);
    return L;
}

static inline int sera_q6k_mmq_padded_rows(int M) { return (M + 31) / 32 * 32; }

/* Q6_K device layouts of a weight matrix of nblk = N * K/256 blocks:
 *   GGUF  (qtype 14):  block b at 210*b: ql[128], qh[64], sc[16], fp16 d;
 *                      rows and blocks are only 2-byte aligned.
 *   split (qtype SERA_QTYPE_Q6K_SPLIT): block b's ql, qh, sc (208 bytes,
 *                      16-byte aligned) at 208*b; its fp16 d at
 *                      208*nblk + 2*b. The same byte count as GGUF. */
#define Q6K_GGUF_BYTES 210
#define Q6K_SPLIT_QBYTES 208
#ifndef SERA_QTYPE_Q6K_SPLIT
#define SERA_QTYPE_Q6K_SPLIT 270u
#endif

#ifdef __HIPCC__
typedef _Float16 f16;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f_bits(uint32_t bits16) {
    union { uint16_t u; f16 h; } c;
    c.u = (uint16_t)bits16;
    return (float)c.h;
}

__device__ __forceinline__ uint32_t f2h_bits(float f) {
    union { uint16_t u; f16 h; } c;
    c.h = (f16)f;             /* v_cvt_f16_f32: round to nearest even */
    return c.u;
}

/* Magic-seeded int8 MFMA epilogue. An int32 accumulator seeded with
 * 0x4B400000 returns 0x4B400000 + I, which read as a float is exactly
 * 1.5 * 2^23 + I for |I| < 2^22 (every per-32 dot: |I| <= 32 * 15 * 127).
 * Then fma(F, sw, -1.5 * 2^23 * sw) is I * sw rounded once, with no
 * integer-to-float convert; -1.5 * 2^23 * sw is exact whenever sw has at
 * most 22 significant bits (fp16 products and d * sc with sc < 64). The
 * caller then accumulates fma(t, d8, acc): two roundings per term, where a
 * single fma(sw * d8, I, acc) rounds once (relative difference at most
 * 2^-24 of the term; none when I * sw fits 24 bits). The
 * seed comes from an opaque register so that the compiler keeps one copy
 * live for every MFMA instead of rematerializing the moves per use. */
#define SERA_MAGIC_BITS 0x4B400000
#define SERA_MAGIC_F 12582912.0f
template <int NR>
__device__ __forceinline__ int __attribute__((ext_vector_type(NR))) sera_magic_seed() {
    int m = SERA_MAGIC_BITS;
    __asm__ volatile("" : "+v"(m));
    int __attribute__((ext_vector_type(NR))) v;
#pragma unroll
    for (int r = 0; r < NR; r++) v[r] = m;
    return v;
}
__device__ __forceinline__ float scaled_dot(int F, float sw, float nsw) { return fmaf(__int_as_float(F), sw, nsw); }

/* 6-bit (scale, min) of sub-block j from the 12 scale bytes held as three
 * little-endian dwords s0 = bytes 0-3, s1 = bytes 4-7, s2 = bytes 8-11
 * (src/q3_quant.c:44-55). */
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t *sc, uint32_t *m) {
    if (j < 4) {
        *sc = (s0 >> (8 * j)) & 63u;
        *m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xffu;        /* scales[j+4] */
        *sc = (b8 & 0xfu) | (((s0 >> (8 * jj)) >> 6 & 3u) << 4);  /* scales[j-4] >> 6 */
        *m = (b8 >> 4) | (((s1 >> (8 * jj)) >> 6 & 3u) << 4);     /* scales[j] >> 6 */
    }
}
#endif

#endif
