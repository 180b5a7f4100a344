/*
 * sera_q4k_bench.hip - timing loops for the bench driver, the counterpart
 * of the reference's --bench-q4-linear mode (src/q3_bench_q4_linear.cu:
 * 181-226), kept in C so host launch cost stays out of the GPU timings.
 *
 * Both loops walk a list of resident weight copies round robin, so a
 * working set larger than the 256 MB last-level (MALL) cache keeps every
 * weight read an HBM read.
 */
#include "sera_launch.h"

#include <stdio.h>

#include "../../include/q3_q4_linear.h"
#include "../../include/sera_q4k.h"

/* `warmup` untimed then `iters` timed calls of q3_cuda_q4k_linear; weight i
 * of the call is weights[i % nweights]. elapsed_ms: first-to-last event of
 * the timed calls (host launch overlaps GPU work). */
extern "C" int sera_q4k_bench_linear(const void *geometry, const void *const *weights,
                                     int nweights, const float *x, size_t M, float *y, void *stream,
                                     int warmup, int iters, double *elapsed_ms) {
    const q3_q4_linear_geometry *g = (const q3_q4_linear_geometry *)geometry;
    if (!g || !weights || nweights <= 0 || iters <= 0 || !elapsed_ms) return -1;
    hipStream_t s = (hipStream_t)stream;
    char err[256];
    for (int i = 0; i < warmup; i++)
        if (!q3_cuda_q4k_linear(g, weights[i % nweights], x, M, y, stream, NULL, err, sizeof(err))) return -3;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1;
    (void)hipEventRecord(a, s);
    for (int i = 0; i < iters; i++)
        if (!q3_cuda_q4k_linear(g, weights[i % nweights], x, M, y, stream, NULL, err, sizeof(err))) return -3;
    (void)hipEventRecord(b, s);
    (void)hipEventSynchronize(b);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, a, b);
    *elapsed_ms = ms;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return 0;
}

/* The achievable read rate of this device: a plain streaming read of a
 * weight copy's bytes with no compute and no output (the floor the MMVQ
 * kernel's time is judged against). Workgroup b reads the 16-byte vectors
 * [b * 256 * LPT, (b + 1) * 256 * LPT) of the buffer, LPT per thread, all
 * loads issued before the first is used; the folded value is stored only in
 * the impossible case that it equals a sentinel, so nothing is written but
 * the loads cannot be dropped. */
template <int LPT>
__global__ __launch_bounds__(256) void sera_stream_read_kernel(const uint4 *__restrict__ p, size_t n16,
                                                               uint32_t *__restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * 256 * LPT + threadIdx.x;
    uint4 v[LPT];
#pragma unroll
    for (int i = 0; i < LPT; i++) {
        const size_t j = base + (size_t)i * 256;
        v[i] = j < n16 ? p[j] : make_uint4(0u, 0u, 0u, 0u);
    }
    uint32_t acc = 0u;
#pragma unroll
    for (int i = 0; i < LPT; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9E3779B9u && threadIdx.x == 0) sink[blockIdx.x & 255] = acc;
}

namespace {
hipError_t launch_stream_read(const void *p, size_t bytes, int lpt, uint32_t *sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    const size_t per = (size_t)256 * lpt;
    const dim3 grid((unsigned)((n16 + per - 1) / per));
    switch (lpt) {
        case 1: hipLaunchKernelGGL(sera_stream_read_kernel<1>, grid, dim3(256), 0, s, (const uint4 *)p, n16, sink); break;
        case 2: hipLaunchKernelGGL(sera_stream_read_kernel<2>, grid, dim3(256), 0, s, (const uint4 *)p, n16, sink); break;
        case 4: hipLaunchKernelGGL(sera_stream_read_kernel<4>, grid, dim3(256), 0, s, (const uint4 *)p, n16, sink); break;
        case 8: hipLaunchKernelGGL(sera_stream_read_kernel<8>, grid, dim3(256), 0, s, (const uint4 *)p, n16, sink); break;
        case 16: hipLaunchKernelGGL(sera_stream_read_kernel<16>, grid, dim3(256), 0, s, (const uint4 *)p, n16, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
}  // namespace

/* Kernel-only loop on a prepared stage: path 0 = MMVQ, 1 = MMQ, 4 = stream-K MMQ (partial = slots, then
 * the zeroed tile counters), 5 = Q6_K MMVQ (param = rows per wave), 6 = Q6_K
 * MMQ (param = splits), 7 / 8 = selected-row LM head on Q6_K / Q4_K rows
 * (stage = fp32 hidden [M][K], partial = the M*param candidate ids,
 * param = candidates per branch, y = logits), 9 / 10 / 11 = paths 5 / 6 / 7
 * on Q6_K weights in the split layout (path 9: param = rows per workgroup),
 * 12 / 13 = few-token kernel on a row stage (MMVQ formula) / an MMQ stage
 * (MMQ formula) (param = chunk, 0 = planned; partial = split slots followed
 * by the zeroed row-group counters). path | 256: the Q4_K paths (0, 1, 4,
 * 8, 12, 13) on weights in the tiled layout (SERA_QTYPE_Q4K_TILED).
 * Path 15: MMQ under the tail schedule (param = dp_tiles * 64 + pieces;
 * partial = slots followed by the zeroed counters). Paths 16 / 17: the
 * Q6_K tile kernel under its tail schedule on GGUF / split-layout weights
 * (param and partial as path 15).
 * Path 14: the plain streaming read of each weight copy's N*K/256*144 bytes
 * (param = 16-byte loads per thread: 1, 2, 4, 8 or 16; y receives nothing but
 * must be 1 KB of device memory).
 * partial_floats: the size of `partial`; a path whose scratch (split-K
 * sums, slots and counters, candidate ids) does not fit returns -2.
 * `iters` launches back to back on `stream` between one pair of events, so
 * no timing packet sits between two launches; avg_kernel_ms is the pair's
 * elapsed time over iters (each launch's duration plus the dispatch gap to
 * the next one), elapsed_ms the pair's elapsed time. */
/* Floats of `partial` a path writes or reads: split-K partial sums, stream-K
 * or tail slots followed by the tile counters, or the candidate ids. */
static size_t bench_partial_floats(int path, int M, int N, int K, int param) {
    switch (path) {
        case 1:
        case 6:
        case 10: return param > 1 ? (size_t)M * N * param : 0;
        case 4: return (size_t)2 * param * sera_mmq_slot_floats(M) + (size_t)sera_mmq_tiles(M, N);
        case 7:
        case 8:
        case 11: return (size_t)M * param;
        case 12:
        case 13: {
            const int sp = sera_fewtok_splits(M, N, K, param);
            return sp > 1 ? (size_t)sp * M * N + (size_t)sera_fewtok_groups(M, N, K) : 0;
        }
        case 15: return sera_mmq_tail_slot_floats(M, N, param / 64, param % 64) + (size_t)sera_mmq_tiles(M, N);
        case 16:
        case 17:
            return sera_q6k_mmq_tail_slot_floats(M, N, K, param / 64, param % 64) +
                   (size_t)sera_q6k_mmq_tiles(M, N, K);
        default: return 0;
    }
}

extern "C" int sera_q4k_bench_kernel(int path, const void *const *weights, int nweights,
                                     const void *stage, float *y, float *partial, size_t partial_floats, int M,
                                     int N, int K, int param, void *stream, int warmup, int iters,
                                     double *avg_kernel_ms, double *elapsed_ms) {
    if (!weights || nweights <= 0 || iters <= 0) return -1;
    hipStream_t s = (hipStream_t)stream;
    const uint32_t q4 = (path & 256) ? SERA_QTYPE_Q4K_TILED : 12u;
    path &= 255;
    /* the kernels trust the scratch they are given: refuse a short one */
    const size_t need = bench_partial_floats(path, M, N, K, param);
    if (need > 0 && (!partial || partial_floats < need)) {
        char msg[160];
        snprintf(msg, sizeof(msg), "sera_q4k_bench_kernel: path %d needs %zu floats of partial, got %zu", path, need,
                 partial ? partial_floats : (size_t)0);
        return sera_report_error(-2, msg);
    }
    auto launch = [&](int i) -> hipError_t {
        const void *w = weights[i % nweights];
        switch (path) {
            case 0: return sera_launch_q4k_mmvq(q4, w, stage, y, M, N, K, param, s);
            case 1: return sera_launch_q4k_mmq(q4, w, stage, y, partial, M, N, K, param, s);
            case 5:
            case 9: return sera_launch_q6k_mmvq(path == 5 ? 14u : SERA_QTYPE_Q6K_SPLIT, w, stage, y, M, N, K, param,
                                                s);
            case 6:
            case 10: return sera_launch_q6k_mmq(path == 6 ? 14u : SERA_QTYPE_Q6K_SPLIT, w, stage, y, partial, M, N, K,
                                                param, s);
            case 7:
            case 8:
            case 11: return sera_launch_candidate_logits(path == 7   ? 14
                                                         : path == 8 ? (int)q4
                                                                     : (int)SERA_QTYPE_Q6K_SPLIT,
                                                         w, N, K, (const float *)stage, (const uint32_t *)partial, M,
                                                         param, y, s);
            case 12:
            case 13: return sera_launch_q4k_fewtok_acc(
                         q4, path - 12, w, stage, y, partial,
                         (int *)(partial + (size_t)sera_fewtok_splits(M, N, K, param) * M * N), M, N, K, param, 0, s);
            case 15: {
                const int dp = param / 64, pc = param % 64;
                return sera_launch_q4k_mmq_tail_acc(
                    q4, w, stage, y, partial, (int *)(partial + sera_mmq_tail_slot_floats(M, N, dp, pc)), M, N, K,
                    dp, pc, 0, s);
            }
            case 16:
            case 17: {
                const int dp = param / 64, pc = param % 64;
                return sera_launch_q6k_mmq_tail_acc(
                    path == 16 ? 14u : SERA_QTYPE_Q6K_SPLIT, w, stage, y, partial,
                    (int *)(partial + sera_q6k_mmq_tail_slot_floats(M, N, K, dp, pc)), M, N, K, dp, pc, 0, s);
            }
            case 14: return launch_stream_read(w, (size_t)N * (K / Q4K_QK) * Q4K_BLOCK_BYTES, param, (uint32_t *)y, s);
            case 4: return sera_launch_q4k_mmq_streamk(
                        q4, w, stage, y, partial, (int *)(partial + (size_t)2 * param * sera_mmq_slot_floats(M)),
                        M, N, K, param, s);
            default: return hipErrorInvalidValue;
        }
    };
    for (int i = 0; i < warmup; i++)
        if (launch(i) != hipSuccess) return -3;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return -1;
    if (hipEventCreate(&b) != hipSuccess) { (void)hipEventDestroy(a); return -1; }
    int rc = 0;
    (void)hipEventRecord(a, s);
    for (int i = 0; i < iters && rc == 0; i++)
        if (launch(i) != hipSuccess) rc = -3;
    (void)hipEventRecord(b, s);
    (void)hipEventSynchronize(b);
    float tot = 0.0f;
    (void)hipEventElapsedTime(&tot, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (rc) return rc;
    if (avg_kernel_ms) *avg_kernel_ms = (double)tot / iters;
    if (elapsed_ms) *elapsed_ms = tot;
    return 0;
}

/* A sequence of q3_cuda_q4k_linear calls (call i: geometries[i], weights[i],
 * xs[i] with Ms[i] rows, ys[i]), issued from C back to back, `warmup` times
 * untimed and `reps` times between one event pair; *ms_per_rep is the pair
 * time over reps. The decode-stream measurement: a token's 64 x 7
 * projections and the LM head without a host language in the loop. With
 * use_graph != 0 the sequence is captured once into a HIP graph (stream
 * must not be the null stream) and the graph is replayed instead. */
namespace {
/* Time `reps` passes of `pass` (after `warmup`), optionally captured once
 * into a HIP graph and replayed. */
template <class Pass>
int time_passes(Pass pass, hipStream_t s, int warmup, int reps, int use_graph, double *ms_per_rep) {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (use_graph) {
        if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return -1;
        const bool ok = pass();
        if (hipStreamEndCapture(s, &graph) != hipSuccess || !ok) return -3;
        if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return -3;
        }
    }
    auto run = [&]() -> bool { return use_graph ? hipGraphLaunch(exec, s) == hipSuccess : pass(); };
    int rc = 0;
    for (int i = 0; i < warmup && rc == 0; i++)
        if (!run()) rc = -3;
    hipEvent_t a = nullptr, b = nullptr;
    if (rc == 0 && (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)) rc = -1;
    if (rc == 0) {
        (void)hipEventRecord(a, s);
        for (int i = 0; i < reps && rc == 0; i++)
            if (!run()) rc = -3;
        (void)hipEventRecord(b, s);
        (void)hipEventSynchronize(b);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, a, b);
        *ms_per_rep = (double)ms / reps;
    }
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
}
}  // namespace

extern "C" int sera_q4k_bench_group_stream(const sera_linear_group_call *calls, int ncalls, void *stream, int warmup,
                                           int reps, int use_graph, double *ms_per_rep) {
    if (!calls || ncalls <= 0 || reps <= 0 || !ms_per_rep) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (use_graph && !s) return -1;
    auto pass = [&]() -> bool {
        for (int i = 0; i < ncalls; i++) {
            const sera_linear_group_call &c = calls[i];
            if (sera_linear_group(c.count, c.geometries, c.weights, c.outputs, c.X, c.X2, c.gamma, c.eps, c.M,
                                  c.flags, stream) != 0)
                return false;
        }
        return true;
    };
    return time_passes(pass, s, warmup, reps, use_graph, ms_per_rep);
}

extern "C" int sera_q4k_bench_stream(const void *const *geometries, const void *const *weights,
                                     const float *const *xs, const size_t *Ms, float *const *ys, int ncalls,
                                     void *stream, int warmup, int reps, int use_graph, double *ms_per_rep) {
    if (!geometries || !weights || !xs || !Ms || !ys || ncalls <= 0 || reps <= 0 || !ms_per_rep) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (use_graph && !s) return -1;
    char err[256];
    auto pass = [&]() -> bool {
        for (int i = 0; i < ncalls; i++)
            if (!q3_cuda_q4k_linear((const q3_q4_linear_geometry *)geometries[i], weights[i], xs[i], Ms[i], ys[i],
                                    stream, NULL, err, sizeof(err)))
                return false;
        return true;
    };
    return time_passes(pass, s, warmup, reps, use_graph, ms_per_rep);
}
