/*
 * sera_launch.h - internal declarations shared between the kernel sources
 * and the host runtime (not installed, not part of the C ABI).
 *
 * Every kernel source that defines one of these functions includes this
 * header, so a definition whose signature drifts from its declaration is a
 * compile error ("conflicting declaration of C function") instead of a call
 * through a mismatched prototype at link time. All launchers enqueue on the
 * given stream and return hipGetLastError() of their launches.
 */
#ifndef SERA_LAUNCH_H
#define SERA_LAUNCH_H

#include "q4k_common.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- q8_quantize.hip: activation stages ------------------------------- */
hipError_t sera_launch_q8_1_row(const float *x, int M, int K, void *stage, hipStream_t stream);
hipError_t sera_launch_q8_1_mmq(const float *x, int M, int Mpad, int K, void *stage, hipStream_t stream);
hipError_t sera_launch_q8_1_q6k_stage(const float *x, int M, int Mpad, int K, int row_formula, void *stage,
                                      hipStream_t stream);
hipError_t sera_launch_q8_1_row_p(const float *x, const sera_producer *prod, int M, int K, void *stage,
                                  hipStream_t stream);
hipError_t sera_launch_q8_1_mmq_p(const float *x, const sera_producer *prod, int M, int Mpad, int K, void *stage,
                                  hipStream_t stream);
hipError_t sera_launch_q8_1_q6k_stage_p(const float *x, const sera_producer *prod, int M, int Mpad, int K,
                                        int row_formula, void *stage, hipStream_t stream);

/* ---- q4k_mmvq.hip: dot4 MMVQ ------------------------------------------ */
int sera_mmvq_rows_per_wave(int N, int K, int M);
/* qtype: 12 (GGUF bytes) or SERA_QTYPE_Q4K_TILED (N % 16 == 0) for every
 * Q4_K weight launcher below */
hipError_t sera_launch_q4k_mmvq(uint32_t qtype, const void *W, const void *stage, float *y, int M, int N, int K,
                                int rpw, hipStream_t s);
hipError_t sera_launch_q4k_mmvq_group(uint32_t qtype, int count, const void *const *W, float *const *y, const int *N,
                                      const void *stage, int M, int K, int rows, int accum, hipStream_t s);

/* ---- q4k_mmq.hip: MMQ tiles, split-K reduce, stream-K ------------------ */
int sera_mmq_bm(int M);
int sera_mmq_wgs_per_cu(int M);
int sera_mmq_splits(int M, int N, int K);
int sera_mmq_padded_rows(int M);
/* Sets the message sera_q4k_last_error returns; returns code. */
int sera_report_error(int code, const char *msg);
int sera_mmq_tiles(int M, int N);
int sera_mmq_slot_floats(int M);
hipError_t sera_launch_splitk_reduce(const float *partial, float *y, size_t n, int splits, hipStream_t s);
hipError_t sera_launch_splitk_reduce_acc(const float *partial, float *y, size_t n, int splits, int accum,
                                         hipStream_t s);
hipError_t sera_launch_q4k_mmq(uint32_t qtype, const void *W, const void *stage, float *y, float *partial, int M, int N,
                               int K, int splits, hipStream_t s);
hipError_t sera_launch_q4k_mmq_acc(uint32_t qtype, const void *W, const void *stage, float *y, float *partial, int M,
                                   int N, int K, int splits, int accum, hipStream_t s);
hipError_t sera_launch_q4k_mmq_streamk(uint32_t qtype, const void *W, const void *stage, float *y, float *slots,
                                       int *counters, int M, int N, int K, int P, hipStream_t s);
hipError_t sera_launch_q4k_mmq_streamk_acc(uint32_t qtype, const void *W, const void *stage, float *y, float *slots,
                                           int *counters, int M, int N, int K, int P, int accum, hipStream_t s);
void sera_mmq_tail_plan(int M, int N, int K, int cus, size_t max_slot_floats, int *dp_tiles, int *pieces);
size_t sera_mmq_tail_slot_floats(int M, int N, int dp_tiles, int pieces);
hipError_t sera_launch_q4k_mmq_tail_acc(uint32_t qtype, const void *W, const void *stage, float *y, float *slots,
                                        int *counters, int M, int N, int K, int dp_tiles, int pieces, int accum,
                                        hipStream_t s);

/* ---- q4k_fewtok.hip: few-token MFMA kernel ----------------------------- */
void sera_fewtok_plan(int M, int N, int K, int *nwave, int *chunk);
int sera_fewtok_max_chunk(int M);
int sera_fewtok_groups(int M, int N, int K);
int sera_fewtok_splits(int M, int N, int K, int chunk);
int sera_fewtok_grid(int form, int M, int N, int K, int chunk);
hipError_t sera_launch_q4k_fewtok_acc(uint32_t qtype, int form, const void *W, const void *stage, float *y,
                                      float *slots, int *counters, int M, int N, int K, int chunk, int accum,
                                      hipStream_t s);

/* ---- q6k_mmvq.hip / q6k_mmq.hip / q6k_layout.hip: Q6_K ---------------- */
int sera_q6k_mmvq_rows(int N, int M);
int sera_q6s_mmvq_rows(int N, int M);
hipError_t sera_launch_q6k_mmvq(uint32_t qtype, const void *W, const void *stage, float *y, int M, int N, int K,
                                int rows, hipStream_t s);
hipError_t sera_launch_q6k_mmvq_acc(uint32_t qtype, const void *W, const void *stage, float *y, int M, int N, int K,
                                    int rows, int accum, hipStream_t s);
int sera_q6k_mmq_splits(int M, int N, int K);
int sera_q6k_mmq_tile_tokens(int M, int N, int K);
int sera_q6k_mmq_tiles(int M, int N, int K);
size_t sera_q6k_mmq_tail_slot_floats(int M, int N, int K, int dp_tiles, int pieces);
hipError_t sera_launch_q6k_mmq_tail_acc(uint32_t qtype, const void *W, const void *stage, float *y, float *slots,
                                        int *counters, int M, int N, int K, int dp_tiles, int pieces, int accum,
                                        hipStream_t s);
hipError_t sera_launch_q6k_mmq(uint32_t qtype, const void *W, const void *stage, float *y, float *partial, int M,
                               int N, int K, int splits, hipStream_t s);
hipError_t sera_launch_q6k_mmq_acc(uint32_t qtype, const void *W, const void *stage, float *y, float *partial, int M,
                                   int N, int K, int splits, int accum, hipStream_t s);
hipError_t sera_launch_q6k_split(const void *src, void *dst, uint64_t first, uint64_t count, uint64_t total,
                                 hipStream_t s);

/* ---- q4k_select.hip: gathered rows ------------------------------------ */
hipError_t sera_launch_candidate_logits(int qtype, const void *W, int N, int K, const float *hidden,
                                        const uint32_t *ids, int branches, int per_branch, float *logits,
                                        hipStream_t s);
hipError_t sera_launch_embedding(int qtype, const void *W, int N, int K, const uint32_t *ids, int tokens,
                                 float *hidden, hipStream_t s);

/* ---- q4k_aux.hip: weight quantizer, dequant, integer-dot test hook ----- */
hipError_t sera_launch_q4k_quantize(const float *x, int64_t rows, int64_t K, void *out, hipStream_t s);
hipError_t sera_launch_q4k_dequant(const void *W, int64_t nblocks, float *out, hipStream_t s);
hipError_t sera_launch_q4k_dequant_tiled(const void *W, int64_t N, int64_t K, float *out, hipStream_t s);
hipError_t sera_launch_q4k_tile(const void *src, void *dst, uint64_t row0, uint64_t rows, uint64_t nkb,
                                hipStream_t s);
hipError_t sera_launch_q4k_subblock_dots(const void *W, const int8_t *xq, int32_t *I, int M, int N, int K,
                                         hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif
