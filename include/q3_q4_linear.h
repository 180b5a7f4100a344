/*
 * q3_q4_linear.h - resident Q4_K quantized linear, MI355X (gfx950) build.
 *
 * Drop-in for the reference's src/q3_q4_linear.h (luca-saggese/sera.c):
 * same symbols, same structs (field order and types), same argument
 * meaning and the same bool + message error behaviour, so q3_forward /
 * q3_systemone and the reference's tests link against this library
 * unchanged. The `void *stream` arguments carry a hipStream_t.
 *
 *     resident Q4_K weight [N, K]  (GGUF 144-byte super-blocks, unchanged)
 *          x
 *     fp32 device activation [M, K]
 *          |  Q8_1 activation quantization (HIP)
 *          |  MMVQ (M <= 8) / MMQ on int8 MFMA (M > 8)   (HIP, gfx950)
 *     fp32 device output [M, N], out[token*N + feature]
 *
 * Not carried over: q3_cmd_bench_q4_linear (src/q3_q4_linear.h:110), the
 * CLI bench entry that takes the reference's q3_options; this build's
 * bench driver is bench.py.
 */
#ifndef Q3_Q4_LINEAR_H
#define Q3_Q4_LINEAR_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/q3_q4_linear.h:32-44 */
typedef struct {
    double total_ms;
    double activation_quant_ms;
    double kernel_ms;

    uint64_t weight_bytes;
    uint64_t activation_read_bytes;
    uint64_t activation_write_bytes;

    uint64_t kernel_launches;
    uint64_t cuda_allocations;
    uint64_t host_syncs;
} q3_q4_linear_stats;

/* src/q3_q4_linear.h:49-55. weight = [N, K], input = [M, K], output = [M, N]. */
typedef struct {
    int32_t M;
    int32_t N;
    int32_t K;
    uint32_t qtype;   /* GGUF/GGML quant type of the weight (12 = Q4_K) */
    uint64_t weight_bytes;
} q3_q4_linear_geometry;

/* GGUF dim[0] = K (row length), dim[1] = N (row count). Fails on a qtype
 * other than Q4_K (12) / Q6_K (14) or the two device layouts of
 * include/sera_q4k.h (SERA_QTYPE_Q4K_TILED, which also needs N % 16 == 0,
 * and SERA_QTYPE_Q6K_SPLIT), zero dims, K % 256 != 0 or dims above
 * INT32_MAX. Pure host. Replaces src/q3_q4_linear.h:65-69
 * (src/q3_q4_linear.cu:48-91). */
bool q3_q4_linear_bind_geometry(uint32_t qtype,
                                uint32_t gguf_rows_dim0,
                                uint32_t gguf_cols_dim1,
                                q3_q4_linear_geometry *out,
                                char *error, size_t error_len);

/* Select the device, create timing events, size the workspace. Repeated
 * calls on the same device only grow the requirement. Replaces
 * src/q3_q4_linear.h:75-77 (src/q3_q4_linear.cu:93-124). */
bool q3_cuda_q4k_linear_init(int device, size_t max_tokens,
                             int64_t max_features, int64_t max_k,
                             char *error, size_t error_len);

/* Workspace bytes the caller must reserve (src/q3_q4_linear.h:81). */
size_t q3_cuda_q4k_linear_workspace_bytes(void);

/* Attach caller-owned device scratch of at least the required size
 * (src/q3_q4_linear.h:84-85). */
bool q3_cuda_q4k_linear_set_workspace(void *device_ptr, size_t bytes,
                                      char *error, size_t error_len);

/* "MMVQ" for token_count <= 8, else "MMQ" (src/q3_q4_linear.h:88). */
const char *q3_cuda_q4k_linear_path_for_batch(size_t token_count);

/* Y[M][N] = X[M][K] . W^T with device pointers only; enqueue-only on
 * `stream` (no host sync, no allocation, no host copies). Returns false
 * with `error` filled on any failure. Q4_K (12) and Q6_K (14) geometries
 * both run, as in the reference (src/q3_q4_linear.cu:199-209), and so do
 * geometries bound to the device layouts (SERA_QTYPE_Q4K_TILED,
 * SERA_QTYPE_Q6K_SPLIT, include/sera_q4k.h). Replaces src/q3_q4_linear.h:99-106
 * (src/q3_q4_linear.cu:149-228). */
bool q3_cuda_q4k_linear(const q3_q4_linear_geometry *geometry,
                        const void *weight,
                        const float *device_input,
                        size_t token_count,
                        float *device_output,
                        void *stream,
                        q3_q4_linear_stats *stats,
                        char *error, size_t error_len);

/* Fill the ms fields from the last call's events; call after the caller
 * synchronized the stream (src/q3_q4_linear.h:116). */
void q3_cuda_q4k_linear_read_stats(q3_q4_linear_stats *stats, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* Q3_Q4_LINEAR_H */
