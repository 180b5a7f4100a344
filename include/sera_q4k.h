/*
 * sera_q4k.h - C ABI of the MI355X (gfx950) Q4_K linear kernels.
 *
 * This is the layer the q3_q4_linear boundary (q3_q4_linear.h) calls; it
 * plays the role of the reference's internal host glue cuda/q3_mmq.h:35-94
 * and of the test-oracle device decode src/q3_cuda_primitives.h. Plain C
 * types only: device pointers are void* / float*, a stream is a hipStream_t
 * passed as void* (NULL = the null stream). Every function enqueues on the
 * given stream and returns without synchronizing; none allocates device
 * memory.
 *
 * Return codes (as in cuda/q3_mmq.h): 0 success, -1 invalid arguments or
 * state, -2 activation-quantization launch failed, -3 matmul launch failed.
 * sera_q4k_last_error() gives the message of the last failure on the
 * calling thread.
 *
 * Layouts:
 *   W  GGUF Q4_K, N rows of K/256 blocks of 144 bytes (K % 256 == 0)
 *   X  fp32 [M][K] row-major, 16-byte aligned
 *   Y  fp32 [M][N] row-major: Y[token*N + feature]
 *   stages: see sera_q8_1_row_stage_offsets / sera_q8_1_mmq_stage_offsets
 */
#ifndef SERA_Q4K_H
#define SERA_Q4K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SERA_Q4K_MMVQ_MAX_BATCH 8    /* cuda/q3_mmq.h:77 Q3_MMVQ_MAX_BATCH */
#define SERA_Q4K_FEWTOK_MAX_BATCH 16 /* largest batch of the few-token MFMA kernel */

/* ---- set-up (cuda/q3_mmq.h:35-38, 84-94) ------------------------------ */

/* Select `device` and create the library's timing events. Returns 0. */
int sera_q4k_init(int device);

/* Persistent scratch bytes for calls with up to max_tokens rows, up to
 * max_features output features and contraction length up to max_k
 * (q3_mmq_arena_bytes, cuda/q3_mmq.cu:213-243). Holds the Q8_1 stage and
 * the split-K partial sums. */
size_t sera_q4k_arena_bytes(size_t max_tokens, int64_t max_features, int64_t max_k);

/* Attach caller-owned device scratch (q3_mmq_set_arena, cuda/q3_mmq.h:84).
 * The first 256 KB hold the stream-K tile counters, which this call clears
 * (a synchronous memset) and every call leaves zero again. */
int sera_q4k_set_arena(void *device_ptr, size_t bytes);

/* ---- whole linear: quantize + kernel (cuda/q3_mmq.h:52-63) ------------ */

/* Y[M][N] = X[M][K] . W^T through the MMQ tile path (any M >= 1).
 * Replaces q3_mmq_q4_K_dense (cuda/q3_mmq.cu:258-379); note M = tokens,
 * N = features here (the donor ABI had them swapped). timed != 0 records
 * the quantize/kernel event pairs (each costs GPU time per call). */
int sera_q4k_dense(const void *W, const float *X, float *Y, int M, int N, int K,
                   void *stream, int timed);

/* Same contract through the MMVQ path (MMVQ arithmetic), 1 <= M <= 8:
 * the dot4 MMVQ kernel or the few-token MFMA kernel (form 0), as
 * sera_q4k_vec_uses_fewtok (sera_q4k_vec_uses_fewtok_qt for the _qt call
 * below) chooses. Replaces q3_mmq_q4_K_dense_vec
 * (cuda/q3_mmq.cu:408-506). */
int sera_q4k_dense_vec(const void *W, const float *X, float *Y, int M, int N, int K,
                       void *stream, int timed);

/* Q4_K weights in the 16-row tiled device layout (no reference
 * counterpart; the reference keeps GGUF bytes on the device,
 * cuda/q3_model_loader_cuda.cu:290-342): block b of row r at byte
 * ((r/16)*(K/256) + b)*2304 + (r%16)*144, i.e. 16-row tiles one after the
 * other, each tile super-block by super-block, each super-block's 16 rows
 * back to back. Same 144-byte blocks and byte count as GGUF; N % 16 == 0.
 * A 16-row group of one super-block is one contiguous 2304-byte run, which
 * the few-token and MMQ kernels read with full-line loads. Values and
 * results are those of the GGUF bytes. sera_weight_upload /
 * sera_weight_to_device_layout produce it; a q3_q4_linear geometry and the
 * group, gathered-row and upload calls may carry this qtype. */
#define SERA_QTYPE_Q4K_TILED 268u

/* sera_q4k_dense / sera_q4k_dense_vec on the weight layout of qtype: 12
 * (GGUF bytes, what the two calls above take) or SERA_QTYPE_Q4K_TILED. */
int sera_q4k_dense_qt(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                      void *stream, int timed);
int sera_q4k_dense_vec_qt(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                          void *stream, int timed);

/* The MMVQ path of sera_q4k_dense_vec, allocating nothing and needing no
 * attached workspace. No counterpart in the reference: it is for callers
 * that cannot allocate device memory or attach a workspace (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 * Its scratch (row-group counters, the Q8_1 row stage, the few-token
 * kernel's split slots) is a static device array of
 * SERA_Q4K_STATIC_SCRATCH_BYTES that every GPU the library runs on holds
 * until the process ends; sera_q4k_init sets it up for its device, and
 * otherwise the first call on a device does (enqueueing a small clearing
 * kernel on `stream`). Shapes needing more scratch than that
 * (sera_q4k_dense_vec_static_bytes) are rejected with -1 and a message.
 * Same arithmetic, kernels and results as sera_q4k_dense_vec; enqueue only,
 * no timings. All calls on one GPU share its scratch: calls that overlap on
 * one GPU (concurrent streams or threads) race. */
#define SERA_Q4K_STATIC_SCRATCH_BYTES ((size_t)8 << 20)
int sera_q4k_dense_vec_static(const void *W, const float *X, float *Y, int M, int N, int K, void *stream);
size_t sera_q4k_dense_vec_static_bytes(int M, int N, int K);   /* 0 for a bad shape */

/* Kernel launches (quantize + matmul + split-K reduce if any) one dense or
 * dense_vec call makes for this shape; 0 for an invalid shape. */
int sera_q4k_kernel_launches(int M, int N, int K);

/* 1 if the MMVQ path (1 <= M <= 8) runs the few-token MFMA kernel for an
 * N x K matrix (tall matrices from 3 tokens, 4096-16383 rows from 6, or
 * from 5 when K >= 16384, never below 4096 rows), 0 if it runs the dot4
 * MMVQ kernel. No counterpart in the reference (cuda/mmq/mmvq.cu has one
 * kernel); a dispatch query. */
int sera_q4k_vec_uses_fewtok(int M, int N, int K);

/* The same query for the weight layout of qtype: 12 as above; on
 * SERA_QTYPE_Q4K_TILED the few-token kernel takes over earlier (matrices of
 * 16384+ rows from 2 tokens; 4096-16383 rows from 3 when K >= 16384, else
 * from 5 at 8192+ rows and from 6 below), as it gains more from the tiled
 * bytes than dot4 does. 0 for any other qtype. */
int sera_q4k_vec_uses_fewtok_qt(uint32_t qtype, int M, int N, int K);

/* 1 if a Q6_K call on the MMVQ path (1 <= M <= 8) runs the tile kernel on a
 * row-formula stage for an N x K matrix of GGUF bytes (from 4 tokens at
 * 16384 or more rows; at 4096-16383 rows from 6, or 5 when K >= 16384;
 * never below 4096), 0 if it runs the Q6_K MMVQ kernel. No counterpart in
 * the reference; a dispatch query. */
int sera_q6k_vec_uses_tile(int M, int N, int K);
/* The same per weight layout: qtype 14 as above; SERA_QTYPE_Q6K_SPLIT from
 * 4 tokens at 16384+ rows and at 4096-16383 from 7, or 6 when K >= 16384
 * (its MMVQ kernel is faster than the GGUF one); 0 for any other qtype. */
int sera_q6k_vec_uses_tile_qt(uint32_t qtype, int M, int N, int K);

/* Event timings of the last timed dense call, valid after the caller
 * synchronized its stream (q3_mmq_read_timings, cuda/q3_mmq.h:48-50). */
void sera_q4k_read_timings(double *quant_ms, double *kernel_ms, double *total_ms);

/* ---- building blocks -------------------------------------------------- */

/* Row-layout Q8_1 stage (MMVQ activations): qs int8 [M][K], ds half2
 * [M][K/32] = (fp16 d, fp16 sum), dsf float4 [M][K/64] =
 * (d_2p, d_2p+1, d_2p*S_2p, d_2p+1*S_2p+1) with S the int sum of 32 quants.
 * Quantizer of cuda/mmq/quantize.cu:4-48 (quantize_row_q8_1_cuda, :369-383). */
size_t sera_q8_1_row_stage_bytes(int M, int K);
void sera_q8_1_row_stage_offsets(int M, int K, size_t *qs, size_t *ds, size_t *dsf);
int sera_q8_1_quantize_row(const float *X, int M, int K, void *stage, void *stream);

/* MMQ-layout Q8_1 stage: qs int8 [Mpad][K], ds half2 [Mpad][K/32], rows
 * M..Mpad-1 zero; Mpad is M rounded up to the MMQ token tile (16 up to 16
 * tokens, 32 up to 32, else 64). Quantizer of cuda/mmq/quantize.cu:271-367
 * (quantize_mmq_q8_1<DS4>, launcher :385-413). */
int sera_q8_1_mmq_padded_rows(int M);
size_t sera_q8_1_mmq_stage_bytes(int M, int K);
void sera_q8_1_mmq_stage_offsets(int M, int K, size_t *qs, size_t *ds);
int sera_q8_1_quantize_mmq(const float *X, int M, int K, void *stage, void *stream);

/* MMVQ kernel on a row stage (mul_mat_vec_q<Q4_K>, cuda/mmq/mmvq.cu:393-587).
 * rows_per_tile = weight rows per workgroup in {2,4,8,16}, or 0 for the
 * built-in choice (sera_q4k_mmvq_rows_per_tile). */
int sera_q4k_mmvq(const void *W, const void *row_stage, float *Y, int M, int N, int K,
                  int rows_per_tile, void *stream);
int sera_q4k_mmvq_rows_per_tile(int M, int N, int K);

/* MMQ kernel on an MMQ stage (mul_mat_q<Q4_K> + stream-K fixup,
 * cuda/mmq/mmq.cuh:3641-4352). `splits` > 1 splits K; then `partial` must
 * hold splits*M*N floats (M*N % 4 == 0). splits = 0 picks the built-in
 * choice (sera_q4k_mmq_splits). */
int sera_q4k_mmq(const void *W, const void *mmq_stage, float *Y, float *partial, int M, int N,
                 int K, int splits, void *stream);
int sera_q4k_mmq_splits(int M, int N, int K);

/* MMQ kernel under a stream-K schedule (the role of mul_mat_q's stream-K
 * decomposition and mul_mat_q_stream_k_fixup, cuda/mmq/mmq.cuh:3641-4352):
 * `wgs` persistent workgroups (a multiple of 8; 0 = the device's resident
 * count) split the (tile, 256-wide K step) units evenly; split tiles are
 * summed in a fixed order by their last contributor, found with a per-tile
 * counter, so results repeat bit for bit and no workgroup waits on another.
 * slots: 2*wgs*sera_q4k_mmq_slot_floats(M) floats; counters:
 * sera_q4k_mmq_tiles(M, N) ints that must be zero and are zero again after
 * the kernel. Needs tiles*K/256 >= wgs. */
int sera_q4k_mmq_streamk(const void *W, const void *mmq_stage, float *Y, float *slots, int *counters,
                         int M, int N, int K, int wgs, void *stream);
int sera_q4k_mmq_streamk_wgs(int M);   /* resident workgroups for M tokens (after init) */
/* Schedule of the MMQ tile kernels for this shape (after init): 2 = whole
 * tiles + split tail (the 64-token tile, M > 32; below), 1 = stream-K
 * (16- and 32-token tiles, M <= 32, from one full round of resident
 * workgroups of tiles), 0 = plain tiles / split-K with the split count of
 * sera_q4k_mmq_splits (a per-CU cost model fitted to MI355X timings); -1
 * for a bad shape. sera_q4k_dense runs it where sera_q4k_mmq_uses_fewtok
 * is 0. */
int sera_q4k_mmq_schedule(int M, int N, int K);

/* MMQ kernel under the tail schedule (the role of mul_mat_q's stream-K
 * decomposition, cuda/mmq/mmq.cuh:3641-4352, for the last round of tiles
 * only): the first dp_tiles workgroups each run one whole output tile; each
 * of the remaining sera_q4k_mmq_tiles(M, N) - dp_tiles tiles is cut into
 * `pieces` near-equal K ranges, one workgroup per (tile, range), whose
 * partial sums are added in range order by the range that finishes last
 * (per-tile counters), so results repeat bit for bit and no workgroup waits
 * on another. slots: sera_q4k_mmq_tail_slot_floats() floats; counters:
 * tiles - dp_tiles ints, zero on entry and zero again after the kernel
 * (both may be NULL when pieces == 1 or dp_tiles == tiles). accum != 0 adds
 * the product to Y. sera_q4k_mmq_tail_plan gives the schedule's own choice
 * (after init; slots limited to max_slot_floats, or with 0 to what the
 * attached arena holds after the stage: the plan sera_q4k_dense runs for
 * M > 32). */
int sera_q4k_mmq_tail_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *slots, int *counters,
                         int M, int N, int K, int dp_tiles, int pieces, int accum, void *stream);
int sera_q4k_mmq_tail_plan(int M, int N, int K, size_t max_slot_floats, int *dp_tiles, int *pieces);
size_t sera_q4k_mmq_tail_slot_floats(int M, int N, int dp_tiles, int pieces);
/* 1 if sera_q4k_dense (the boundary's MMQ path) runs the few-token MFMA
 * kernel with the MMQ formula for this shape instead of the MMQ tiles: 1-8
 * tokens always, 9-16 tokens on matrices with N or K of 16384 or more (gate,
 * up, down, the LM head); 0 otherwise. No counterpart in the reference
 * (mul_mat_q has one kernel family); a dispatch query. */
int sera_q4k_mmq_uses_fewtok(int M, int N, int K);
/* MMQ output tiles for M tokens of N rows: 16, 32 or 64 tokens by 256 rows,
 * or 64 by 128 where 256-row tiles would number at most 64. */
int sera_q4k_mmq_tiles(int M, int N);
/* Floats of one stream-K or tail slot for M tokens (the largest tile's). */
int sera_q4k_mmq_slot_floats(int M);

/* Few-token kernel (1 <= M <= 16): Y (+)= X . W^T with two sub-blocks per
 * v_mfma_i32_16x16x64_i8. form 0 takes a row stage and computes the MMVQ
 * formula (as sera_q4k_mmvq, vec_dot_q4_K_q8_1, cuda/mmq/vecdotq.cuh:505-527),
 * M <= 8: it plays the role of mul_mat_vec_q<Q4_K, ncols> (cuda/mmq/mmvq.cu:
 * 393-587) for 4-8 tokens. form 1 takes an MMQ stage and computes the MMQ
 * formula (as sera_q4k_mmq, cuda/mmq/mmq.cuh:2269-2283,1440-1472).
 * chunk: super-blocks of K per workgroup, 1..40 for M <= 8 and 1..20 above,
 * 0 = the built-in choice. When the chunk splits K (sera_q4k_fewtok_splits >
 * 1), slots holds splits*M*N floats and counters sera_q4k_fewtok_groups(M,
 * N, K) ints that must be zero and are zero again after the kernel; the
 * last split of each row group sums the partials in split order, so results
 * repeat bit for bit. W and the stage 16-byte aligned; accum != 0 adds the
 * product to Y. */
int sera_q4k_fewtok(int form, const void *W, const void *stage, float *Y, float *slots, int *counters, int M, int N,
                    int K, int chunk, int accum, void *stream);

/* The four kernel calls above on the weight layout of qtype: 12 (GGUF
 * bytes, what the calls above take) or SERA_QTYPE_Q4K_TILED (N % 16 == 0).
 * Same arguments, kernels and results otherwise. */
int sera_q4k_mmvq_qt(uint32_t qtype, const void *W, const void *row_stage, float *Y, int M, int N, int K,
                     int rows_per_tile, void *stream);
int sera_q4k_mmq_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *partial, int M, int N,
                    int K, int splits, void *stream);
int sera_q4k_mmq_streamk_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *slots,
                            int *counters, int M, int N, int K, int wgs, void *stream);
int sera_q4k_fewtok_qt(uint32_t qtype, int form, const void *W, const void *stage, float *Y, float *slots,
                       int *counters, int M, int N, int K, int chunk, int accum, void *stream);
int sera_q4k_fewtok_splits(int M, int N, int K, int chunk);
int sera_q4k_fewtok_groups(int M, int N, int K);
/* Workgroups along the rows of that launch on the current device: the row
 * groups, or fewer when the grid is persistent (one K split, an even number
 * of super-blocks, more row groups than the device holds at once: each
 * workgroup stages the activations once for a balanced range of 16-row
 * tiles); -1 for a chunk past the limit, 0 for an invalid shape. No
 * counterpart in the reference (a query of this build's launch shape). */
int sera_q4k_fewtok_grid(int form, int M, int N, int K, int chunk);

/* Device Q4_K dequant, w = (d*sc)*q - (dmin*m) per weight; replaces
 * q3_cuda_dequantize_row (src/q3_cuda_primitives.h, cuda/q3_cuda_primitives.cu:13-95). */
int sera_q4k_dequantize(const void *W, size_t nblocks, float *out, void *stream);
/* The N x K matrix in the layout of qtype (12 or SERA_QTYPE_Q4K_TILED)
 * dequantized to row-major fp32 out[N][K], same values as above. */
int sera_q4k_dequantize_qt(uint32_t qtype, const void *W, int N, int K, float *out, void *stream);

/* Exact per-32 int32 dots I[m][n][b] = sum q4*q8 for the first M rows of a
 * stage's qs array (int8 [rows][K]). Test hook for the integer core shared
 * by both kernels (cuda/mmq/vecdotq.cuh:505-555). */
int sera_q4k_subblock_dots(const void *W, const void *stage_qs, int32_t *I, int M, int N, int K,
                           void *stream);

/* fp32 [rows][K] -> GGUF Q4_K bytes, bit-exact with the repo's quantizer
 * quantize_q4_k_matrix (tools/qwen3_q4.py:410-481). */
int sera_q4k_quantize(const float *X, int64_t rows, int64_t K, void *out, void *stream);

const char *sera_q4k_last_error(void);

/* ---- Q6_K weights (GGUF type 14): N rows of K/256 blocks of 210 bytes ---
 * Block: ql[128] low nibbles, qh[64] high 2 bits, sc[16] int8 scales of
 * 16-wide groups, fp16 d (cuda/mmq/ggml-common.h:348-357, src/q3_quant.c:78-103).
 * Rows are 2-byte aligned only; W itself must be 16-byte aligned and
 * readable up to the next 16-byte boundary past its last byte (any hipMalloc
 * allocation is).
 *
 * Every Q6_K entry point takes the qtype of its weight bytes: 14 for the
 * GGUF bytes, or SERA_QTYPE_Q6K_SPLIT for the split device layout that
 * sera_weight_upload / sera_weight_to_device_layout produce (no reference
 * counterpart; the reference keeps GGUF bytes on the device,
 * cuda/q3_model_loader_cuda.cu:290-342): the N*K/256 blocks in row order,
 * block b's ql, qh, sc (208 bytes) at 208*b, then all d as fp16 at
 * 208*N*K/256 + 2*b. Same byte count as GGUF; each block's 208 bytes are
 * 16-byte aligned, which the kernels load directly. Values and results are
 * those of the GGUF bytes. A q3_q4_linear geometry may carry this qtype. */
#define SERA_QTYPE_Q6K_SPLIT 270u

/* Y = X . W^T through the MMVQ path (MMVQ arithmetic), 1 <= M <= 8: the
 * reference quantizes Q6_K decode activations with the same
 * quantize_row_q8_1_cuda call as Q4_K. The dot4 MMVQ kernel on the row
 * stage, or, where sera_q6k_vec_uses_tile_qt says so (tall matrices from 4
 * tokens, 4096-16383 rows from 5-6 on GGUF bytes and from 6-7 on the split
 * layout), the fp16-MFMA tile kernel on a row-formula Q6_K stage. Replaces q3_mmq_q6_K_dense_vec (cuda/q3_mmq.cu:515-519 over
 * q3_mmq_dense_vec_impl, :408-506). */
int sera_q6k_dense_vec(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                       void *stream, int timed);

/* Same contract through the MMQ path, any M >= 1 (the ABI uses it for
 * M > 8). Replaces q3_mmq_q6_K_dense (cuda/q3_mmq.cu:388-393 over
 * q3_mmq_dense_impl, :258-379). Activations go through the D4 MMQ quantizer
 * (fp32 scale per 32 values, cuda/mmq/quantize.cu:271-367,
 * mmq.cuh:64-103). */
int sera_q6k_dense(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                   void *stream, int timed);

/* Kernel launches one sera_q6k_dense / sera_q6k_dense_vec call makes, on
 * GGUF bytes and (the _qt form) on either Q6_K layout. */
int sera_q6k_kernel_launches(int M, int N, int K);
int sera_q6k_kernel_launches_qt(uint32_t qtype, int M, int N, int K);

/* MMVQ kernel on a row stage (mul_mat_vec_q<Q6_K>, cuda/mmq/mmvq.cu:907-911,
 * with vec_dot_q6_K_q8_1, cuda/mmq/vecdotq.cuh:624-643,956-980):
 * y = sum_blk d * sum_g d8[g/2] * (I_g * sc_g), I_g the exact int dot of a
 * 16-wide group. GGUF bytes: rows = rows per wave in {1, 2, 4} (4 only for
 * M <= 4); split layout: rows per workgroup in {2, 4}; 0 = the built-in
 * choice (sera_q6k_mmvq_rows_per_wave for GGUF bytes). */
int sera_q6k_mmvq(uint32_t qtype, const void *W, const void *row_stage, float *Y, int M, int N, int K,
                  int rows, void *stream);
int sera_q6k_mmvq_rows_per_wave(int M, int N);

/* Q6_K MMQ activation stage (D4 quantizer of cuda/mmq/quantize.cu:271-367
 * with the layout mmq_get_q8_1_ds_layout selects for Q6_K,
 * cuda/mmq/mmq.cuh:64-103): 16 * quant as fp16 [Mpad][K] (exact integers),
 * fp32 d = 1/d_inv as [K/256][8][Mpad]; rows M..Mpad-1 zero, Mpad a
 * multiple of 32. sera_q8_1_quantize_row_q6k fills the same layout with the
 * row quantizer's values (cuda/mmq/quantize.cu:4-48, d8 = fp32(fp16 d)):
 * the MMVQ arithmetic on the tile kernel, which sera_q6k_dense_vec uses
 * where sera_q6k_vec_uses_tile_qt says so. */
int sera_q8_1_q6k_mmq_padded_rows(int M);
size_t sera_q8_1_q6k_mmq_stage_bytes(int M, int K);
void sera_q8_1_q6k_mmq_stage_offsets(int M, int K, size_t *qs, size_t *d);
int sera_q8_1_quantize_mmq_d4(const float *X, int M, int K, void *stage, void *stream);
int sera_q8_1_quantize_row_q6k(const float *X, int M, int K, void *stage, void *stream);

/* MMQ kernel on a Q6_K MMQ stage (mul_mat_q<Q6_K>, cuda/mmq/mmq.cuh:3570-3575
 * with load_tiles_q6_K :2512-2596 and vec_dot_q6_K_q8_1_mma :2634-2786):
 * y = sum_blk d * sum_b d8_b * (sc_2b*I_2b + sc_2b+1*I_2b+1). splits > 1
 * splits K (partial: splits*M*N floats, M*N % 4 == 0); 0 = built-in choice
 * (sera_q6k_mmq_splits_for). */
int sera_q6k_mmq(uint32_t qtype, const void *W, const void *q6k_mmq_stage, float *Y, float *partial, int M, int N,
                 int K, int splits, void *stream);
int sera_q6k_mmq_splits_for(int M, int N, int K);
/* The Q6_K tile kernel under the tail schedule (the role of mul_mat_q's
 * stream-K decomposition, cuda/mmq/mmq.cuh:3641-4352, as for Q4_K): the
 * first dp_tiles workgroups run one whole output tile each; each of the
 * other sera_q6k_mmq_tiles() - dp_tiles tiles is cut into `pieces` K
 * ranges, one workgroup per (tile, range), whose sums the range that ends
 * last adds in range order (per-tile counters): results repeat bit for bit
 * and no workgroup waits on another. slots: sera_q6k_mmq_tail_slot_floats()
 * floats; counters: tiles - dp_tiles ints, zero on entry and after (both
 * may be NULL when pieces == 1 or dp_tiles == tiles). accum != 0 adds the
 * product to Y. sera_q6k_mmq_tail_plan returns 1 and the (dp_tiles,
 * pieces) the dense paths run when they take this schedule (after init;
 * slots limited to max_slot_floats, 0 = no limit), else 0 (split-K). */
int sera_q6k_mmq_tail(uint32_t qtype, const void *W, const void *q6k_mmq_stage, float *Y, float *slots, int *counters,
                      int M, int N, int K, int dp_tiles, int pieces, int accum, void *stream);
int sera_q6k_mmq_tail_plan(int M, int N, int K, size_t max_slot_floats, int *dp_tiles, int *pieces);
size_t sera_q6k_mmq_tail_slot_floats(int M, int N, int K, int dp_tiles, int pieces);
/* Output tiles of the Q6_K tile kernel (token tile x 128 rows). */
int sera_q6k_mmq_tiles(int M, int N, int K);
/* Token tile of the Q6_K MMQ kernel for this shape: 32, or 64 when the
 * padded rows divide by 64 and the 64-token grid has at least 1024
 * (tile, super-block) pairs. The two give bit-identical results. */
int sera_q6k_mmq_tile_tokens(int M, int N, int K);

/* ---- weight upload into the device layout -------------------------------
 * Replaces the verbatim tensor copy of the reference's resident loader
 * (q3_loader_load, cuda/q3_model_loader_cuda.cu:171-373; pinned staging +
 * H2D + D2D at :290-342) for the weights of this path. qtype names the
 * device layout: 12 and 14 keep the GGUF bytes (a plain copy),
 * SERA_QTYPE_Q4K_TILED repacks GGUF Q4_K bytes into the tiled layout and
 * SERA_QTYPE_Q6K_SPLIT GGUF Q6_K bytes into the split layout, on the
 * device. The source is always the tensor's GGUF bytes (N rows of K/256
 * blocks). */

/* Bytes of the weight matrix in any of these layouts (= the GGUF size);
 * 0 for a bad qtype or shape. */
size_t sera_weight_bytes(uint32_t qtype, int N, int K);

/* GGUF bytes already on the device -> dst in the layout of qtype (enqueue
 * only). Split: gguf 2-byte aligned, dst 16-byte aligned, no overlap.
 * Tiled: both 16-byte aligned, no overlap, N % 16 == 0. */
int sera_weight_to_device_layout(uint32_t qtype, int N, int K, const void *gguf, void *dst, void *stream);

/* Host GGUF bytes -> dst in the layout of qtype, on `stream` (enqueue
 * only; host_gguf must stay valid until the stream reaches the copies, as
 * for hipMemcpyAsync; pinned memory makes the copies asynchronous). The
 * split layout streams the bytes through the caller's device staging
 * buffer (>= 210 bytes, 16-byte aligned; whole blocks per pass) and repacks
 * each pass into dst; the tiled layout likewise, whole 16-row groups per
 * pass (staging >= 16 * K/256 * 144 bytes); GGUF layouts copy straight to
 * dst (staging unused). */
int sera_weight_upload(uint32_t qtype, int N, int K, const void *host_gguf, void *dst, void *staging,
                       size_t staging_bytes, void *stream);

/* ---- fused linear group (the path's edges) -----------------------------
 * No single reference counterpart: one call replaces the sequence the
 * reference's forward pass makes around its q3_cuda_q4k_linear calls
 * (src/q3_forward.cu:1204-1351):
 *   outputs[i] = op(X) . W_i^T          for i < count (1..4)
 *   outputs[i] += op(X) . W_i^T         with SERA_LIN_ACCUMULATE, the
 *       residual add (q3_cuda_residual_add, :167-171,688-700) fused into
 *       the product's store: bit-identical to product-then-add;
 *   op(X) = X, or with SERA_LIN_RMSNORM (x * inv_rms) * gamma,
 *       inv_rms = 1/sqrt(mean(x^2) + eps) (q3_cuda_rms_norm, :117-146,
 *       659-672; sum order and IEEE sqrt/div as documented in
 *       q8_quantize.hip), or with SERA_LIN_SILU_MUL (x / (1 + exp(-x))) * X2
 *       (q3_cuda_silu_mul, :154-161,674-686), computed inside the Q8_1
 *       quantize (no materialized op(X)).
 * All weights share K and qtype (geometries are q3_q4_linear_geometry*);
 * the activations are quantized once for the group (q/k/v and gate/up read
 * the same normed input). At decode (Q4_K, M <= 8) the matrices the dot4
 * MMVQ kernel takes (sera_q4k_vec_uses_fewtok == 0) share one grouped
 * launch and the others run the few-token kernel one by one; a Q6_K group
 * shares one stage, so its largest matrix picks the kernel
 * (sera_q6k_vec_uses_tile_qt). Arithmetic per product as q3_cuda_q4k_linear (MMVQ
 * formula for M <= 8, MMQ above). gamma and X2 must be 16-byte aligned.
 * Uses the arena of sera_q4k_set_arena / q3_cuda_q4k_linear_set_workspace;
 * enqueue only. */
#define SERA_LINEAR_GROUP_MAX 4
#define SERA_LIN_ACCUMULATE 1u
#define SERA_LIN_RMSNORM 2u
#define SERA_LIN_SILU_MUL 4u
int sera_linear_group(int count, const void *const *geometries, const void *const *weights, float *const *outputs,
                      const float *X, const float *X2, const float *gamma, float eps, size_t M, unsigned flags,
                      void *stream);

/* One sera_linear_group call, for sera_q4k_bench_group_stream. */
typedef struct {
    int count;
    const void *geometries[SERA_LINEAR_GROUP_MAX];
    const void *weights[SERA_LINEAR_GROUP_MAX];
    float *outputs[SERA_LINEAR_GROUP_MAX];
    const float *X;
    const float *X2;
    const float *gamma;
    float eps;
    size_t M;
    unsigned flags;
} sera_linear_group_call;

/* ---- gathered rows of a Q4_K (12, SERA_QTYPE_Q4K_TILED) / Q6_K (14,
 * SERA_QTYPE_Q6K_SPLIT) matrix ---
 * fp32 dequant with the expression order of src/q3_quant.c:57-103 (Q4_K
 * (d*sc)*q - dmin*m, Q6_K (d*sc)*(q-32)) and the GGUF Q6_K byte mapping of
 * q3_quant.c. The reference's device twin q6_value_dev
 * (src/q3_forward.cu:86-110) indexes ql/qh and the group scale differently
 * from its own q3_quant.c for most weights of a block; these functions
 * follow q3_quant.c. hidden must be 16-byte aligned; W as for the linear
 * calls. */

/* Selected-row LM head: logits[b*C + c] = sum_k w[ids[b*C + c]][k] *
 * hidden[b][k] for b < branches, c < C = per_branch; fp32 weights times
 * fp32 hidden (no Q8_1). Replaces candidate_logits_kernel and
 * candidate_logits_batched_kernel (src/q3_forward.cu:329-370,566-607); the
 * reference's host wrappers q3_candidate_logits / _batched (:1826-1900)
 * copy host ids to the device first, here ids are device memory. ids >= N
 * give NaN logits. */
int sera_candidate_logits(int qtype, const void *W, int N, int K, const float *hidden, int branches,
                          const uint32_t *ids, int per_branch, float *logits, void *stream);

/* Embedding row gather: hidden[t][k] = w[ids[t]][k]; ids >= N leave the
 * row untouched. Replaces q3_cuda_embedding / embedding_kernel
 * (src/q3_forward.cu:291-322,757-774). */
int sera_embedding(int qtype, const void *W, int N, int K, const uint32_t *ids, int tokens, float *hidden,
                   void *stream);

/* ---- bench loops (the role of src/q3_bench_q4_linear.cu:181-226) ------- */

/* `warmup` untimed and `iters` timed q3_cuda_q4k_linear calls on weight
 * copies weights[i % nweights]; *elapsed_ms spans the timed calls.
 * `geometry` is a q3_q4_linear_geometry* (include/q3_q4_linear.h). */
int sera_q4k_bench_linear(const void *geometry, const void *const *weights, int nweights,
                          const float *X, size_t M, float *Y, void *stream, int warmup,
                          int iters, double *elapsed_ms);

/* Kernel-only loop on a prepared stage (path 0 = MMVQ with param =
 * rows_per_wave, 1 = MMQ with param = splits, 2/3 = few-token kernel form
 * 0/1 with param = splits, 4 = stream-K MMQ with param = workgroups and
 * `partial` holding the slots followed by the zeroed tile counters, 5 =
 * Q6_K MMVQ with param = rows per wave, 6 = Q6_K MMQ with param = splits on
 * a Q6_K MMQ stage, 7 / 8 = selected-row LM head on Q6_K / Q4_K rows with
 * stage = fp32 hidden [M][K], partial = the M*param candidate ids, param =
 * candidates per branch): `iters` launches back to back between one event pair
 * on `stream`; *avg_kernel_ms = pair time / iters, *elapsed_ms = pair time.
 * partial_floats is the size of `partial`; a path whose scratch does not fit
 * returns -2 without launching. */
int sera_q4k_bench_kernel(int path, const void *const *weights, int nweights, const void *stage,
                          float *Y, float *partial, size_t partial_floats, int M, int N, int K, int param,
                          void *stream, int warmup, int iters, double *avg_kernel_ms, double *elapsed_ms);

/* `reps` timed passes (after `warmup`) over a sequence of
 * q3_cuda_q4k_linear calls: geometries[i] (q3_q4_linear_geometry*),
 * weights[i], xs[i] with Ms[i] rows, ys[i]. *ms_per_rep: one pass.
 * use_graph != 0: the pass is captured once into a HIP graph and replayed
 * (stream must not be the null stream). */
int sera_q4k_bench_stream(const void *const *geometries, const void *const *weights,
                          const float *const *xs, const size_t *Ms, float *const *ys, int ncalls,
                          void *stream, int warmup, int reps, int use_graph, double *ms_per_rep);

/* sera_q4k_bench_stream for a sequence of sera_linear_group calls (the
 * fused decode stream). */
int sera_q4k_bench_group_stream(const sera_linear_group_call *calls, int ncalls, void *stream, int warmup, int reps,
                                int use_graph, double *ms_per_rep);

#ifdef __cplusplus
}
#endif

#endif
