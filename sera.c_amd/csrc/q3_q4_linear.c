/*
 * q3_q4_linear.c - the reference's q3_q4_linear C ABI on the gfx950 kernels.
 *
 * Plain C99 host code; it reaches the GPU only through include/sera_q4k.h.
 * Mirrors src/q3_q4_linear.cu of the reference (binder :48-91, init and
 * workspace :93-143, dispatch :149-228, stats :231-241), with the same
 * process-global, single-device, non-reentrant state: one host thread on
 * one ordered stream, as the reference's server worker guarantees.
 */
#include "../../include/q3_q4_linear.h"
#include "../../include/sera_q4k.h"

#include <stdio.h>
#include <string.h>

enum { QTYPE_Q4_K = 12, QTYPE_Q6_K = 14 };
/* Q6_K in the split device layout and Q4_K in the 16-row tiled one
 * (sera_weight_upload); extensions of the reference's qtype set, accepted
 * wherever Q6_K / Q4_K is. The tiled layout needs N % 16 == 0. */
#define QTYPE_Q6_K_SPLIT SERA_QTYPE_Q6K_SPLIT
#define QTYPE_Q4_K_TILED SERA_QTYPE_Q4K_TILED

static bool known_qtype(uint32_t qtype) {
    return qtype == QTYPE_Q4_K || qtype == QTYPE_Q4_K_TILED || qtype == QTYPE_Q6_K || qtype == QTYPE_Q6_K_SPLIT;
}
#define QK_K 256
#define Q4_K_BLOCK_BYTES 144
#define Q6_K_BLOCK_BYTES 210

static size_t g_workspace_bytes = 0;
static bool g_initialized = false;
static int g_device = -1;

static void set_error(char *error, size_t error_len, const char *message) {
    if (error && error_len) {
        error[0] = '\0';
        snprintf(error, error_len, "%s", message);
    }
}

bool q3_q4_linear_bind_geometry(uint32_t qtype, uint32_t gguf_rows_dim0, uint32_t gguf_cols_dim1,
                                q3_q4_linear_geometry *out, char *error, size_t error_len) {
    if (!out) return false;
    memset(out, 0, sizeof(*out));
    if (!known_qtype(qtype)) {
        set_error(error, error_len, "q3_q4_linear: tensor qtype is not Q4_K/Q6_K");
        return false;
    }
    const uint64_t K = gguf_rows_dim0;   /* contiguous row length */
    const uint64_t N = gguf_cols_dim1;   /* row count */
    if (K == 0 || N == 0) {
        set_error(error, error_len, "q3_q4_linear: degenerate geometry");
        return false;
    }
    if (K % QK_K != 0) {
        char buffer[160];
        snprintf(buffer, sizeof(buffer), "q3_q4_linear: K=%llu must be a multiple of %d",
                 (unsigned long long)K, QK_K);
        set_error(error, error_len, buffer);
        return false;
    }
    if (K > INT32_MAX || N > INT32_MAX) {
        set_error(error, error_len, "q3_q4_linear: geometry exceeds int32");
        return false;
    }
    if (qtype == QTYPE_Q4_K_TILED && N % 16 != 0) {
        set_error(error, error_len, "q3_q4_linear: the tiled Q4_K layout needs a row count divisible by 16");
        return false;
    }
    out->K = (int32_t)K;
    out->N = (int32_t)N;
    out->qtype = qtype;
    out->M = 0;
    out->weight_bytes = N * (K / QK_K) *
                        (qtype == QTYPE_Q4_K || qtype == QTYPE_Q4_K_TILED ? Q4_K_BLOCK_BYTES : Q6_K_BLOCK_BYTES);
    return true;
}

bool q3_cuda_q4k_linear_init(int device, size_t max_tokens, int64_t max_features, int64_t max_k,
                             char *error, size_t error_len) {
    if (g_initialized && g_device == device) {
        /* Several runtimes may share the process; never shrink. */
        const size_t needed = sera_q4k_arena_bytes(max_tokens, max_features, max_k);
        if (needed > g_workspace_bytes) g_workspace_bytes = needed;
        return true;
    }
    if (device < 0) {
        set_error(error, error_len, "q3_q4_linear: invalid device index");
        return false;
    }
    if (sera_q4k_init(device) != 0) {
        char buffer[320];
        snprintf(buffer, sizeof(buffer), "q3_q4_linear: init failed: %s", sera_q4k_last_error());
        set_error(error, error_len, buffer);
        return false;
    }
    g_workspace_bytes = sera_q4k_arena_bytes(max_tokens, max_features, max_k);
    g_device = device;
    g_initialized = true;
    return true;
}

size_t q3_cuda_q4k_linear_workspace_bytes(void) { return g_workspace_bytes; }

bool q3_cuda_q4k_linear_set_workspace(void *device_ptr, size_t bytes, char *error, size_t error_len) {
    if (!device_ptr || bytes < g_workspace_bytes) {
        char buffer[192];
        snprintf(buffer, sizeof(buffer), "q3_q4_linear: workspace too small (%zu < %zu)", bytes,
                 g_workspace_bytes);
        set_error(error, error_len, buffer);
        return false;
    }
    if (sera_q4k_set_arena(device_ptr, bytes) != 0) {
        char buffer[320];
        snprintf(buffer, sizeof(buffer), "q3_q4_linear: arena attach failed: %s", sera_q4k_last_error());
        set_error(error, error_len, buffer);
        return false;
    }
    return true;
}

const char *q3_cuda_q4k_linear_path_for_batch(size_t token_count) {
    return token_count <= SERA_Q4K_MMVQ_MAX_BATCH ? "MMVQ" : "MMQ";
}

bool q3_cuda_q4k_linear(const q3_q4_linear_geometry *geometry, const void *weight,
                        const float *device_input, size_t token_count, float *device_output,
                        void *stream, q3_q4_linear_stats *stats, char *error, size_t error_len) {
    if (!geometry || !weight || !device_input || !device_output) {
        set_error(error, error_len, "q3_q4_linear: null argument");
        return false;
    }
    if (!g_initialized) {
        set_error(error, error_len, "q3_q4_linear: not initialized");
        return false;
    }
    if (token_count == 0 || token_count > INT32_MAX) {
        set_error(error, error_len, "q3_q4_linear: bad token count");
        return false;
    }
    if (geometry->N <= 0 || geometry->K <= 0) {
        set_error(error, error_len, "q3_q4_linear: unresolved geometry");
        return false;
    }
    if (!known_qtype(geometry->qtype)) {
        set_error(error, error_len, "q3_q4_linear: tensor qtype is not Q4_K/Q6_K");
        return false;
    }
    const bool q6 = geometry->qtype == QTYPE_Q6_K || geometry->qtype == QTYPE_Q6_K_SPLIT;

    q3_q4_linear_stats local;
    q3_q4_linear_stats *s = stats ? stats : &local;
    memset(s, 0, sizeof(*s));
    s->weight_bytes = geometry->weight_bytes;

    const int K = geometry->K;
    const int features = geometry->N;
    const int tokens = (int)token_count;
    s->activation_read_bytes = token_count * (size_t)K * sizeof(float);
    s->activation_write_bytes = token_count * (size_t)features * sizeof(float);

    int rc;
    if (tokens <= SERA_Q4K_MMVQ_MAX_BATCH) {
        rc = q6 ? sera_q6k_dense_vec(geometry->qtype, weight, device_input, device_output, tokens, features, K,
                                     stream, stats != NULL)
                : sera_q4k_dense_vec_qt(geometry->qtype, weight, device_input, device_output, tokens, features, K,
                                        stream, stats != NULL);
    } else {
        rc = q6 ? sera_q6k_dense(geometry->qtype, weight, device_input, device_output, tokens, features, K,
                                 stream, stats != NULL)
                : sera_q4k_dense_qt(geometry->qtype, weight, device_input, device_output, tokens, features, K,
                                    stream, stats != NULL);
    }
    s->kernel_launches = (uint64_t)(q6 ? sera_q6k_kernel_launches_qt(geometry->qtype, tokens, features, K)
                                       : sera_q4k_kernel_launches(tokens, features, K));
    if (rc != 0) {
        char buffer[400];
        snprintf(buffer, sizeof(buffer), "q3_q4_linear: %s path failed (rc=%d) for M=%d N=%d K=%d: %s",
                 q3_cuda_q4k_linear_path_for_batch(token_count), rc, tokens, features, K,
                 sera_q4k_last_error());
        set_error(error, error_len, buffer);
        return false;
    }
    return true;
}

void q3_cuda_q4k_linear_read_stats(q3_q4_linear_stats *stats, void *stream) {
    (void)stream;
    if (!stats || !g_initialized) return;
    double q = 0.0, k = 0.0, t = 0.0;
    sera_q4k_read_timings(&q, &k, &t);
    stats->activation_quant_ms = q;
    stats->kernel_ms = k;
    stats->total_ms = t;
}
