/*
 * sera_q4k_runtime.hip - host side of include/sera_q4k.h: argument checks,
 * the caller-owned scratch arena, hipEvent timings and kernel launches.
 *
 * Replaces the reference's host glue cuda/q3_mmq.cu (arena :95-137,
 * sizing :170-243, dense paths :258-379 and :408-506, timings :45-83).
 * Nothing here allocates device memory or synchronizes: the arena is
 * attached once by the caller, every launch is enqueued on the caller's
 * stream, and timings are read only after the caller has synchronized.
 */
#include "sera_launch.h"
#include "../../include/q3_q4_linear.h"
#include "../../include/sera_q4k.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace {

thread_local char g_err[256];

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

struct Events {
    hipEvent_t quant_begin, quant_end, kernel_begin, kernel_end;
    bool valid;
};

int g_device = -1;
int g_cus = 0;                    /* compute units of the device */
Events g_ev = {};
unsigned char *g_arena = nullptr; /* stage and partial sums (after the counter region) */
int *g_counters = nullptr;        /* stream-K tile counters, zero between calls */
size_t g_arena_bytes = 0;

/* The arena starts with the counters of the stream-K MMQ tiles (first
 * half) and of the few-token kernel's row groups (second half), zeroed when
 * the arena is attached; each call leaves them zero again. */
constexpr size_t kCounterBytes = (size_t)256 << 10;
constexpr int kMaxCounters = (int)(kCounterBytes / sizeof(int));
constexpr int kFewtokCounterBase = kMaxCounters / 2;
constexpr int kFewtokMaxCounters = kMaxCounters - kFewtokCounterBase;

/* The MMVQ path (M <= 8) runs the few-token MFMA kernel (MMVQ formula)
 * instead of the dot4 MMVQ kernel where that is faster. Measured on MI355X
 * per Qwen3-32B shape with the weights streamed from HBM (kernel us, best
 * dot4 / few-token, interleaved runs): the few-token kernel's time is flat
 * in M, dot4's grows with every token and jumps at 6 (2 rows per wave).
 *   gate/up 25600 rows: 3 tokens 19.9 / 19.9, 4: 22.6 / 19.9;
 *   LM head 151936 rows: 3: 96.0 / 93.8;
 *   q 8192 and o 5120 rows: 5 tokens 10.4 / 11.0, 9.2 / 14.7; 6: 16.6 /
 *     11.2, 14.9 / 14.8;
 *   down 5120 rows, K 25600: 5 tokens 26.9 / 25.5;
 *   k/v 1024 rows: 8 tokens 5.3 / 10.5 (dot4 at every batch). */
extern "C" int sera_q4k_vec_uses_fewtok(int M, int N, int K) {
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH || N <= 0) return 0;
    if (N >= 16384) return M >= 3;
    if (N >= 4096) return M >= (K >= 16384 ? 5 : 6);
    return 0;
}

/* The same choice on the tiled layout, where the few-token kernel reads each
 * 16-row group of a super-block as one 2304-byte run (15-19% faster than on
 * GGUF bytes) and dot4 loses 0-6%. Kernel us, dot4 / few-token, both on the
 * tiled bytes: gate/up 2 tokens 17.3 / 15.9; LM head 2: 79.3 / 76.8;
 * down 3: 20.9 / 20.7, 4: 23.1 / 21.3; q 5: 10.8 / 9.8; o 5: 9.3 / 12.1,
 * 6: 14.9 / 12.1; k/v dot4 at every batch (8: 5.3 / 9.2). At one token
 * dot4 stays ahead everywhere (gate/up 14.2 / 15.7). */
extern "C" int sera_q4k_vec_uses_fewtok_qt(uint32_t qtype, int M, int N, int K) {
    if (qtype != SERA_QTYPE_Q4K_TILED) return qtype == 12u ? sera_q4k_vec_uses_fewtok(M, N, K) : 0;
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH || N <= 0) return 0;
    if (N >= 16384) return M >= 2;
    if (N >= 4096) return M >= (K >= 16384 ? 3 : N >= 8192 ? 5 : 6);
    return 0;
}

/* The MMQ path runs the same kernel with the MMQ formula on the MMQ stage
 * at 1-8 tokens, and at 9-16 tokens on the matrices whose rows or K reach
 * 16384 (its 8-wave plan). Against the paired 16-token MMQ tile, measured
 * through the boundary on the Qwen3-32B shapes (weights streamed from HBM,
 * 10-16 tokens, us per call): gate/up 25.5-26 against 33-34, down 34-36
 * against 44-45, LM head 120-124 against 143; on q, o and k/v the paired
 * tile stays ahead (15, 20, 15 against 18-19, 23-24, 17-18), and at 9
 * tokens too (q 15.0 against 17.3). */
#define SERA_Q4K_FEWTOK_MMQ_MAX_BATCH 16
extern "C" int sera_q4k_mmq_uses_fewtok(int M, int N, int K) {
    if (M < 1 || M > SERA_Q4K_FEWTOK_MMQ_MAX_BATCH || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    return M <= 8 || N >= 16384 || K >= 16384;
}

/* Workgroups the stream-K MMQ schedule runs for M tokens: the resident
 * count, a multiple of 8. */
int streamk_wgs(int M) { return g_cus > 0 ? sera_mmq_wgs_per_cu(M) * g_cus / 8 * 8 : 0; }

/* Partial-sum floats never exceed this. Split-K: at most 2048 workgroups
 * (tiles * splits), and an MMQ tile holds at most 64*256 outputs, so
 * splits*M*N <= 2048 * 16384. Stream-K: two tile slots per resident
 * workgroup, at most 2*(2*CUs)*16384 = 4*CUs*16384 (64 x 256 tiles) or
 * 2*(3*CUs)*8192 (32 x 256 tiles). */
size_t partial_floats_bound(size_t max_tokens, int64_t max_features) {
    size_t by_tiles = (size_t)2048 * 16384;
    const size_t by_slots = (size_t)4 * (g_cus > 0 ? g_cus : 256) * 16384;
    if (by_slots > by_tiles) by_tiles = by_slots;
    const size_t by_shape = (size_t)16 * max_tokens * (size_t)(max_features > 0 ? max_features : 0);
    return by_tiles < by_shape ? by_tiles : by_shape;
}

/* Limits of the kernels' index arithmetic, checked before any launch:
 *   - the activation stages are addressed with 32-bit element offsets
 *     (the MMQ staging computes (token * K + k) in 32 bits), so
 *     Mpad * K must stay below 2^31 for the largest token padding (64);
 *   - the quantizers put one activation row per grid row (gridDim.y),
 *     which the device caps at 65535;
 *   - a weight row and a 16-row group of rows stay below 2^31 bytes
 *     (buffer-resource ranges are 32-bit), which K <= 2^24 guarantees. */
constexpr int64_t kMaxStagedElems = (int64_t)1 << 31;
constexpr int kMaxRows = 65535;
constexpr int kMaxK = 1 << 24;

bool stage_ok(const char *tag, int M, int K) {
    if (K > kMaxK) { fail(-1, "%s: K=%d exceeds the supported %d", tag, K, kMaxK); return false; }
    const int64_t mpad = ((int64_t)M + 63) / 64 * 64;
    if (mpad > kMaxRows) {
        fail(-1, "%s: M=%d tokens exceed the %d rows one quantize launch covers", tag, M, kMaxRows);
        return false;
    }
    if (mpad * K >= kMaxStagedElems) {
        fail(-1, "%s: staged activations Mpad*K = %lld reach 2^31 (32-bit stage offsets)", tag,
             (long long)(mpad * K));
        return false;
    }
    return true;
}

bool check_shape(const char *tag, const void *W, const float *X, const float *Y, int M, int N, int K) {
    if (!W || !X || !Y) { fail(-1, "%s: null pointer", tag); return false; }
    if (M <= 0 || N <= 0 || K <= 0) { fail(-1, "%s: bad shape M=%d N=%d K=%d", tag, M, N, K); return false; }
    if (K % Q4K_QK != 0) { fail(-1, "%s: K=%d must be a multiple of 256", tag, K); return false; }
    if (!stage_ok(tag, M, K)) return false;
    if (((uintptr_t)X & 15u) != 0) { fail(-1, "%s: X must be 16-byte aligned", tag); return false; }
    if (((uintptr_t)W & 15u) != 0) { fail(-1, "%s: W must be 16-byte aligned", tag); return false; }
    return true;
}

void record(hipEvent_t e, hipStream_t s) {
    if (g_ev.valid) (void)hipEventRecord(e, s);
}

}  // namespace

/* Records msg as the library's last error (for the other translation units
 * of the library) and returns code. */
int sera_report_error(int code, const char *msg) { return fail(code, "%s", msg); }

extern "C" const char *sera_q4k_last_error(void) { return g_err; }

/* ---- the decode path on a library-owned static scratch ------------------
 * sera_q4k_dense_vec_static keeps its scratch (row-regime counters, the
 * Q8_1 row stage, the few-token kernel's split slots) in this file-scope
 * device array instead of the caller's workspace. Every GPU the library
 * runs on holds its own copy until the process ends; host code never uses
 * the name `scratch` itself (on the host it is a stand-in, not a device
 * address), only the per-device address hipGetSymbolAddress returns. */
static __device__ __align__(256) unsigned char scratch[SERA_Q4K_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
constexpr size_t kStaticCounterBytes = (size_t)16 << 10;   /* row-group counters, zero between calls */
unsigned char *g_scratch_ptr[kMaxDevices];                  /* device address of `scratch`, per device */

__global__ void sera_zero_words_kernel(uint32_t *p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

/* Look up this device's copy of `scratch` (the device must be current) and
 * clear its counter region with a fill kernel on `s`; once per device. */
int static_scratch_setup(int device, hipStream_t s) {
    if (device < 0 || device >= kMaxDevices) return fail(-1, "static scratch: device %d out of range", device);
    if (g_scratch_ptr[device]) return 0;
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
        return fail(-1, "static scratch: hipGetSymbolAddress failed on device %d", device);
    const int words = (int)(kStaticCounterBytes / 4);
    hipLaunchKernelGGL(sera_zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, s, (uint32_t *)p, words);
    if (hipGetLastError() != hipSuccess) return fail(-1, "static scratch: clearing the counters failed");
    g_scratch_ptr[device] = (unsigned char *)p;
    return 0;
}
}  // namespace

extern "C" int sera_q4k_init(int device) {
    if (device < 0) return fail(-1, "sera_q4k_init: invalid device %d", device);
    if (hipSetDevice(device) != hipSuccess) return fail(-1, "sera_q4k_init: hipSetDevice(%d) failed", device);
    if (!g_ev.valid || g_device != device) {
        if (hipEventCreate(&g_ev.quant_begin) != hipSuccess ||
            hipEventCreate(&g_ev.quant_end) != hipSuccess ||
            hipEventCreate(&g_ev.kernel_begin) != hipSuccess ||
            hipEventCreate(&g_ev.kernel_end) != hipSuccess)
            return fail(-1, "sera_q4k_init: hipEventCreate failed");
        g_ev.valid = true;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
        return fail(-1, "sera_q4k_init: cannot read the compute-unit count of device %d", device);
    g_cus = cus;
    g_device = device;
    /* the static scratch of sera_q4k_dense_vec_static, set up while this
     * device is current; the clearing kernel runs on the null stream, and
     * init waits for it (a caller's non-blocking stream is not ordered after
     * the null stream) */
    if (!g_scratch_ptr[device]) {
        if (static_scratch_setup(device, nullptr) != 0) return -1;
        if (hipStreamSynchronize(nullptr) != hipSuccess)
            return fail(-1, "sera_q4k_init: clearing the static scratch failed");
    }
    return 0;
}

extern "C" size_t sera_q8_1_row_stage_bytes(int M, int K) {
    if (M <= 0 || K <= 0) return 0;
    return sera_row_stage_layout((size_t)M, (size_t)K).total;
}

extern "C" void sera_q8_1_row_stage_offsets(int M, int K, size_t *qs, size_t *ds, size_t *dsf) {
    const sera_stage_layout L = sera_row_stage_layout((size_t)(M > 0 ? M : 0), (size_t)(K > 0 ? K : 0));
    if (qs) *qs = L.qs;
    if (ds) *ds = L.ds;
    if (dsf) *dsf = L.dsf;
}

extern "C" int sera_q8_1_mmq_padded_rows(int M) { return M > 0 ? sera_mmq_padded_rows(M) : 0; }

extern "C" size_t sera_q8_1_mmq_stage_bytes(int M, int K) {
    if (M <= 0 || K <= 0) return 0;
    return sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K).total;
}

extern "C" void sera_q8_1_mmq_stage_offsets(int M, int K, size_t *qs, size_t *ds) {
    const size_t mp = M > 0 ? (size_t)sera_mmq_padded_rows(M) : 0;
    const sera_stage_layout L = sera_mmq_stage_layout(mp, (size_t)(K > 0 ? K : 0));
    if (qs) *qs = L.qs;
    if (ds) *ds = L.ds;
}

extern "C" size_t sera_q4k_arena_bytes(size_t max_tokens, int64_t max_features, int64_t max_k) {
    if (max_tokens == 0 || max_k <= 0) return (size_t)1 << 21;  /* unspecified geometry floor */
    const int mt = (int)(max_tokens > 0x7fffffff ? 0x7fffffff : max_tokens);
    const size_t row = sera_row_stage_layout((size_t)(mt < SERA_Q4K_MMVQ_MAX_BATCH ? mt : SERA_Q4K_MMVQ_MAX_BATCH),
                                             (size_t)max_k).total;
    const size_t mmq = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(mt), (size_t)max_k).total;
    const size_t q6 = sera_q6k_mmq_stage_layout((size_t)sera_q6k_mmq_padded_rows(mt), (size_t)max_k).total;
    size_t stage = row > mmq ? row : mmq;
    if (q6 > stage) stage = q6;
    size_t partial_floats = partial_floats_bound(max_tokens, max_features);
    /* the few-token kernel's split partials: at most 16 splits, or one per
     * 10 super-blocks of a longer K */
    const size_t few_splits = (size_t)((max_k / Q4K_QK + 9) / 10 > 16 ? (max_k / Q4K_QK + 9) / 10 : 16);
    const size_t few = few_splits * (size_t)(mt < SERA_Q4K_FEWTOK_MMQ_MAX_BATCH ? mt : SERA_Q4K_FEWTOK_MMQ_MAX_BATCH) *
                       (size_t)(max_features > 0 ? max_features : 0);
    if (few > partial_floats) partial_floats = few;
    const size_t partial = sera_align256(partial_floats * sizeof(float));
    return kCounterBytes + stage + partial;
}

extern "C" int sera_q4k_set_arena(void *device_ptr, size_t bytes) {
    if (!device_ptr || bytes <= kCounterBytes) return fail(-1, "sera_q4k_set_arena: null or too small arena");
    if (((uintptr_t)device_ptr & 255u) != 0) return fail(-1, "sera_q4k_set_arena: arena must be 256-byte aligned");
    if (hipMemset(device_ptr, 0, kCounterBytes) != hipSuccess)
        return fail(-1, "sera_q4k_set_arena: clearing the tile counters failed");
    g_counters = (int *)device_ptr;
    g_arena = (unsigned char *)device_ptr + kCounterBytes;
    g_arena_bytes = bytes - kCounterBytes;
    return 0;
}

extern "C" int sera_q8_1_quantize_row(const float *X, int M, int K, void *stage, void *stream) {
    if (!X || !stage || M <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q8_1_quantize_row: bad arguments");
    if (!stage_ok("sera_q8_1_quantize_row", M, K)) return -1;
    return sera_launch_q8_1_row(X, M, K, stage, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-2, "sera_q8_1_quantize_row: launch failed");
}

extern "C" int sera_q8_1_quantize_mmq(const float *X, int M, int K, void *stage, void *stream) {
    if (!X || !stage || M <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q8_1_quantize_mmq: bad arguments");
    if (!stage_ok("sera_q8_1_quantize_mmq", M, K)) return -1;
    if (((uintptr_t)X & 15u) != 0) return fail(-1, "sera_q8_1_quantize_mmq: X must be 16-byte aligned");
    return sera_launch_q8_1_mmq(X, M, sera_mmq_padded_rows(M), K, stage, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-2, "sera_q8_1_quantize_mmq: launch failed");
}

extern "C" int sera_q4k_mmvq_rows_per_tile(int M, int N, int K) {
    return sera_mmvq_rows_per_wave(N, K, M);
}

namespace {
/* The weight layouts of the Q4_K path: 12 (GGUF bytes) or the 16-row tiled
 * layout, which needs N % 16 == 0. */
bool q4k_layout_ok(const char *tag, uint32_t qtype, int N) {
    if (qtype != 12u && qtype != SERA_QTYPE_Q4K_TILED) {
        fail(-1, "%s: qtype %u is not Q4_K (12) or Q4_K tiled (%u)", tag, qtype, SERA_QTYPE_Q4K_TILED);
        return false;
    }
    if (qtype == SERA_QTYPE_Q4K_TILED && N % Q4K_TILE_ROWS) {
        fail(-1, "%s: the tiled layout needs N %% 16 == 0 (N=%d)", tag, N);
        return false;
    }
    return true;
}
}  // namespace

extern "C" int sera_q4k_mmvq(const void *W, const void *row_stage, float *Y, int M, int N, int K,
                             int rows_per_tile, void *stream) {
    return sera_q4k_mmvq_qt(12u, W, row_stage, Y, M, N, K, rows_per_tile, stream);
}

extern "C" int sera_q4k_mmvq_qt(uint32_t qtype, const void *W, const void *row_stage, float *Y, int M, int N, int K,
                                int rows_per_tile, void *stream) {
    if (!W || !row_stage || !Y) return fail(-1, "sera_q4k_mmvq: null pointer");
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH) return fail(-1, "sera_q4k_mmvq: batch M=%d outside 1..8", M);
    if (N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q4k_mmvq: bad shape N=%d K=%d", N, K);
    if (!stage_ok("sera_q4k_mmvq", M, K)) return -1;
    if (rows_per_tile != 0 && rows_per_tile != 2 && rows_per_tile != 4 && rows_per_tile != 8 &&
        rows_per_tile != 16)
        return fail(-1, "sera_q4k_mmvq: rows_per_tile=%d not in {0,2,4,8,16}", rows_per_tile);
    if (!q4k_layout_ok("sera_q4k_mmvq", qtype, N)) return -1;
    return sera_launch_q4k_mmvq(qtype, W, row_stage, Y, M, N, K, rows_per_tile, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q4k_mmvq: launch failed");
}

extern "C" int sera_q4k_mmq_splits(int M, int N, int K) { return sera_mmq_splits(M, N, K); }

extern "C" int sera_q4k_fewtok_splits(int M, int N, int K, int chunk) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK || chunk < 0) return 0;
    return sera_fewtok_splits(M, N, K, chunk);
}

extern "C" int sera_q4k_fewtok_groups(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    return sera_fewtok_groups(M, N, K);
}

extern "C" int sera_q4k_fewtok_grid(int form, int M, int N, int K, int chunk) {
    if (M <= 0 || M > SERA_Q4K_FEWTOK_MMQ_MAX_BATCH || (form == 0 && M > 8) || (form != 0 && form != 1) || N <= 0 ||
        K <= 0 || K % Q4K_QK || chunk < 0)
        return 0;
    return sera_fewtok_grid(form, M, N, K, chunk);
}

extern "C" int sera_q4k_fewtok(int form, const void *W, const void *stage, float *Y, float *slots, int *counters,
                               int M, int N, int K, int chunk, int accum, void *stream) {
    return sera_q4k_fewtok_qt(12u, form, W, stage, Y, slots, counters, M, N, K, chunk, accum, stream);
}

extern "C" int sera_q4k_fewtok_qt(uint32_t qtype, int form, const void *W, const void *stage, float *Y, float *slots,
                                  int *counters, int M, int N, int K, int chunk, int accum, void *stream) {
    if (!W || !stage || !Y) return fail(-1, "sera_q4k_fewtok: null pointer");
    if (form != 0 && form != 1) return fail(-1, "sera_q4k_fewtok: form=%d not 0 (row stage) or 1 (MMQ stage)", form);
    const int mmax = form == 0 ? SERA_Q4K_MMVQ_MAX_BATCH : SERA_Q4K_FEWTOK_MAX_BATCH;
    if (M < 1 || M > mmax) return fail(-1, "sera_q4k_fewtok: batch M=%d outside 1..%d", M, mmax);
    if (N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q4k_fewtok: bad shape N=%d K=%d", N, K);
    if (!stage_ok("sera_q4k_fewtok", M, K)) return -1;
    if (((uintptr_t)W & 15u) || ((uintptr_t)stage & 15u))
        return fail(-1, "sera_q4k_fewtok: W and the stage must be 16-byte aligned");
    if (chunk < 0 || chunk > sera_fewtok_max_chunk(M))
        return fail(-1, "sera_q4k_fewtok: chunk=%d outside 0..%d", chunk, sera_fewtok_max_chunk(M));
    if (sera_fewtok_splits(M, N, K, chunk) > 1 && (!slots || !counters))
        return fail(-1, "sera_q4k_fewtok: a split K needs slots and counters");
    if (!q4k_layout_ok("sera_q4k_fewtok", qtype, N)) return -1;
    return sera_launch_q4k_fewtok_acc(qtype, form, W, stage, Y, slots, counters, M, N, K, chunk, accum ? 1 : 0,
                                      (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q4k_fewtok: launch failed");
}

extern "C" int sera_q4k_mmq(const void *W, const void *mmq_stage, float *Y, float *partial, int M, int N,
                            int K, int splits, void *stream) {
    return sera_q4k_mmq_qt(12u, W, mmq_stage, Y, partial, M, N, K, splits, stream);
}

extern "C" int sera_q4k_mmq_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *partial, int M,
                               int N, int K, int splits, void *stream) {
    if (!W || !mmq_stage || !Y) return fail(-1, "sera_q4k_mmq: null pointer");
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q4k_mmq: bad shape M=%d N=%d K=%d", M, N, K);
    if (!stage_ok("sera_q4k_mmq", M, K)) return -1;
    if (splits == 0) splits = sera_mmq_splits(M, N, K);
    if (splits < 1 || splits > K / Q4K_QK) return fail(-1, "sera_q4k_mmq: splits=%d outside 1..K/256", splits);
    if (splits > 1 && (!partial || ((size_t)M * N) % 4 != 0))
        return fail(-1, "sera_q4k_mmq: split-K needs a partial buffer and M*N %% 4 == 0");
    if (!q4k_layout_ok("sera_q4k_mmq", qtype, N)) return -1;
    return sera_launch_q4k_mmq(qtype, W, mmq_stage, Y, partial, M, N, K, splits, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q4k_mmq: launch failed");
}

namespace {
/* The schedule rule, from MI355X measurements over the Qwen3-32B shapes.
 * For 64-token tiles the fitted split-K choice beats stream-K on all 43
 * measured shapes (q, k/v, o, gate/up, down at 48-2048 tokens; stream-K
 * 0.3-90% slower), so 64-token tiles never take it. 32-token tiles (M <= 32)
 * take stream-K from one full round of tiles on (the 151936-row LM head);
 * below that split-K wins, since each tile would be cut into many short
 * pieces. */
bool streamk_rule(int M, int N, int K) {
    const int P = streamk_wgs(M);
    if (P < 8 || M > 32) return false;
    const int tiles = sera_mmq_tiles(M, N);
    return tiles >= P && tiles < 4 * P && tiles <= kFewtokCounterBase && (int64_t)tiles * (K / Q4K_QK) >= P;
}
bool use_streamk(int M, int N, int K) { return g_counters && streamk_rule(M, N, K); }

/* The tail schedule (whole tiles, then the last round's tiles cut along K)
 * serves the 64-token tile (M > 32) from more than P/8 tiles (P = 2 * CUs
 * resident workgroups); below that the fitted split-K with its reduce
 * launch was faster on every measured shape (k/v at 256-1024 tokens, q at
 * 96-128: split-K 22.7-30.3 us against the best tail 24.1-34.3; from 80
 * tiles the tail won: o at 256 tokens 50.6 against 54.4, gate/up at 64
 * 44.1 against 48.8, at 512 215.9 against 232.9, down at 512 206.5 against
 * 217.9). Its counters share the stream-K half of the counter region (the
 * two never run at once; both leave it zero). */
bool tail_rule(int M, int N) {
    return g_cus > 0 && sera_mmq_bm(M) == 64 && sera_mmq_tiles(M, N) * 8 > 2 * g_cus;
}

struct MmqPlan {
    int kind;        /* 0 split-K (splits), 1 stream-K, 2 tail (dp_tiles, pieces) */
    int splits, dp_tiles, pieces;
    size_t partial_floats;
};

/* The MMQ schedule for M x N x K with cap floats of partial/slot scratch. */
MmqPlan mmq_plan(int M, int N, int K, size_t cap, bool have_counters) {
    MmqPlan p = {0, 1, 0, 1, 0};
    if (have_counters && tail_rule(M, N)) {
        sera_mmq_tail_plan(M, N, K, g_cus, cap, &p.dp_tiles, &p.pieces);
        const int R = sera_mmq_tiles(M, N) - p.dp_tiles;
        if (p.pieces == 1 || R <= kFewtokCounterBase) {
            p.kind = 2;
            p.partial_floats = sera_mmq_tail_slot_floats(M, N, p.dp_tiles, p.pieces);
            return p;
        }
    }
    const size_t slot_floats = (size_t)2 * streamk_wgs(M) * sera_mmq_slot_floats(M);
    if (have_counters && streamk_rule(M, N, K) && slot_floats <= cap) {
        p.kind = 1;
        p.partial_floats = slot_floats;
        return p;
    }
    int sp = ((size_t)M * N) % 4 == 0 ? sera_mmq_splits(M, N, K) : 1;
    if ((size_t)sp * M * N > cap) sp = 1;
    p.splits = sp;
    p.partial_floats = sp > 1 ? (size_t)sp * M * N : 0;
    return p;
}

hipError_t mmq_launch(const MmqPlan &p, uint32_t qt, const void *W, const void *stage, float *Y, float *partial,
                      int M, int N, int K, int accum, hipStream_t s) {
    if (p.kind == 2)
        return sera_launch_q4k_mmq_tail_acc(qt, W, stage, Y, partial, g_counters, M, N, K, p.dp_tiles, p.pieces,
                                            accum, s);
    if (p.kind == 1)
        return sera_launch_q4k_mmq_streamk_acc(qt, W, stage, Y, partial, g_counters, M, N, K, streamk_wgs(M), accum,
                                               s);
    return sera_launch_q4k_mmq_acc(qt, W, stage, Y, partial, M, N, K, p.splits, accum, s);
}
}  // namespace


namespace {
/* The few-token kernel on `stage` (form 0: row stage, 1: MMQ stage): split
 * partials go to `slots` (cap floats), row-group counters to `counters`
 * (ncounters ints, zero between calls). */
int fewtok_launch_on(const char *tag, uint32_t qtype, int form, const void *W, const void *stage, float *Y,
                     float *slots, size_t cap, int *counters, int ncounters, int M, int N, int K, int accum,
                     hipStream_t s) {
    const int splits = sera_fewtok_splits(M, N, K, 0);
    if (splits > 1) {
        if ((size_t)splits * M * N > cap)
            return fail(-1, "%s: scratch too small for %d split partials of %dx%d", tag, splits, M, N);
        if (sera_fewtok_groups(M, N, K) > ncounters)
            return fail(-1, "%s: N=%d needs more row-group counters than the scratch holds", tag, N);
    }
    return sera_launch_q4k_fewtok_acc(qtype, form, W, stage, Y, slots, counters, M, N, K, 0, accum, s) == hipSuccess
               ? 0 : fail(-3, "%s: few-token kernel launch failed", tag);
}

/* The same on the caller's arena: the stage at its start, the counters in
 * the second half of the counter region. */
int fewtok_launch(const char *tag, uint32_t qtype, int form, const void *W, float *Y, float *slots, size_t cap, int M,
                  int N, int K, int accum, hipStream_t s) {
    return fewtok_launch_on(tag, qtype, form, W, g_arena, Y, slots, cap, g_counters + kFewtokCounterBase,
                            kFewtokMaxCounters, M, N, K, accum, s);
}

/* The MMVQ path (quantize + dot4 MMVQ or the few-token kernel) on explicit
 * scratch: the row stage at `stage`, split slots after it (slot_cap
 * floats), row-group counters at `counters`. */
int dense_vec_on(const char *tag, uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                 hipStream_t s, int timed, unsigned char *stage, size_t stage_cap, int *counters, int ncounters) {
    const size_t stage_bytes = sera_row_stage_layout((size_t)M, (size_t)K).total;
    if (stage_bytes > stage_cap) return fail(-1, "%s: scratch too small (%zu > %zu)", tag, stage_bytes, stage_cap);
    if (timed) record(g_ev.quant_begin, s);
    if (sera_launch_q8_1_row(X, M, K, stage, s) != hipSuccess) return fail(-2, "%s: quantize launch failed", tag);
    if (timed) record(g_ev.quant_end, s);
    if (timed) record(g_ev.kernel_begin, s);
    if (sera_q4k_vec_uses_fewtok_qt(qtype, M, N, K)) {
        const int rc = fewtok_launch_on(tag, qtype, 0, W, stage, Y, (float *)(stage + stage_bytes),
                                        (stage_cap - stage_bytes) / sizeof(float), counters, ncounters, M, N, K, 0, s);
        if (rc) return rc;
    } else if (sera_launch_q4k_mmvq(qtype, W, stage, Y, M, N, K, 0, s) != hipSuccess) {
        return fail(-3, "%s: mmvq launch failed", tag);
    }
    if (timed) record(g_ev.kernel_end, s);
    return 0;
}
}  // namespace


extern "C" int sera_q4k_dense(const void *W, const float *X, float *Y, int M, int N, int K, void *stream,
                              int timed) {
    return sera_q4k_dense_qt(12u, W, X, Y, M, N, K, stream, timed);
}

extern "C" int sera_q4k_dense_qt(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                                 void *stream, int timed) {
    if (!check_shape("sera_q4k_dense", W, X, Y, M, N, K)) return -1;
    if (!q4k_layout_ok("sera_q4k_dense", qtype, N)) return -1;
    if (!g_arena) return fail(-1, "sera_q4k_dense: no arena attached");
    hipStream_t s = (hipStream_t)stream;
    const int Mpad = sera_mmq_padded_rows(M);
    const size_t stage_bytes = sera_mmq_stage_layout((size_t)Mpad, (size_t)K).total;
    if (sera_q4k_mmq_uses_fewtok(M, N, K)) {
        /* few tokens: the few-token kernel with the MMQ formula on the MMQ stage */
        if (stage_bytes > g_arena_bytes)
            return fail(-1, "sera_q4k_dense: arena too small (%zu > %zu)", stage_bytes, g_arena_bytes);
        if (timed) record(g_ev.quant_begin, s);
        if (sera_launch_q8_1_mmq(X, M, Mpad, K, g_arena, s) != hipSuccess)
            return fail(-2, "sera_q4k_dense: quantize launch failed");
        if (timed) record(g_ev.quant_end, s);
        if (timed) record(g_ev.kernel_begin, s);
        const int rc = fewtok_launch("sera_q4k_dense", qtype, 1, W, Y, (float *)(g_arena + stage_bytes),
                                     (g_arena_bytes - stage_bytes) / sizeof(float), M, N, K, 0, s);
        if (rc) return rc;
        if (timed) record(g_ev.kernel_end, s);
        return 0;
    }
    if (stage_bytes > g_arena_bytes)
        return fail(-1, "sera_q4k_dense: arena too small (%zu > %zu)", stage_bytes, g_arena_bytes);
    const MmqPlan plan = mmq_plan(M, N, K, (g_arena_bytes - stage_bytes) / sizeof(float), g_counters != nullptr);
    void *stage = g_arena;
    float *partial = plan.partial_floats ? (float *)(g_arena + stage_bytes) : nullptr;
    if (timed) record(g_ev.quant_begin, s);
    if (sera_launch_q8_1_mmq(X, M, Mpad, K, stage, s) != hipSuccess)
        return fail(-2, "sera_q4k_dense: quantize launch failed");
    if (timed) record(g_ev.quant_end, s);
    if (timed) record(g_ev.kernel_begin, s);
    const hipError_t e = mmq_launch(plan, qtype, W, stage, Y, partial, M, N, K, 0, s);
    if (e != hipSuccess) return fail(-3, "sera_q4k_dense: mmq launch failed");
    if (timed) record(g_ev.kernel_end, s);
    return 0;
}

extern "C" int sera_q4k_mmq_streamk_wgs(int M) { return M > 0 ? streamk_wgs(M) : 0; }

extern "C" int sera_q4k_mmq_schedule(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return -1;
    if (tail_rule(M, N)) return 2;
    return streamk_rule(M, N, K) ? 1 : 0;
}

extern "C" int sera_q4k_mmq_tail_plan(int M, int N, int K, size_t max_slot_floats, int *dp_tiles, int *pieces) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK || !dp_tiles || !pieces)
        return fail(-1, "sera_q4k_mmq_tail_plan: bad arguments");
    if (g_cus <= 0) return fail(-1, "sera_q4k_mmq_tail_plan: not initialised (the CU count is unknown)");
    if (max_slot_floats == 0) {
        /* what sera_q4k_dense would use: the attached arena after the stage */
        const size_t stage = sera_mmq_stage_layout((size_t)sera_mmq_padded_rows(M), (size_t)K).total;
        max_slot_floats = g_arena && g_arena_bytes > stage ? (g_arena_bytes - stage) / sizeof(float) : 0;
    }
    sera_mmq_tail_plan(M, N, K, g_cus, max_slot_floats, dp_tiles, pieces);
    return 0;
}

extern "C" size_t sera_q4k_mmq_tail_slot_floats(int M, int N, int dp_tiles, int pieces) {
    if (M <= 0 || N <= 0) return 0;
    return sera_mmq_tail_slot_floats(M, N, dp_tiles, pieces);
}

extern "C" int sera_q4k_mmq_tail_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *slots,
                                    int *counters, int M, int N, int K, int dp_tiles, int pieces, int accum,
                                    void *stream) {
    const char *tag = "sera_q4k_mmq_tail";
    if (!W || !mmq_stage || !Y) return fail(-1, "%s: null pointer", tag);
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "%s: bad shape M=%d N=%d K=%d", tag, M, N, K);
    if (!stage_ok(tag, M, K)) return -1;
    const int T = sera_mmq_tiles(M, N);
    if (dp_tiles < 0 || dp_tiles > T) return fail(-1, "%s: dp_tiles=%d outside 0..%d", tag, dp_tiles, T);
    if (pieces < 1 || pieces > K / Q4K_QK) return fail(-1, "%s: pieces=%d outside 1..K/256", tag, pieces);
    if (pieces > 1 && dp_tiles < T && (!slots || !counters))
        return fail(-1, "%s: a split tail needs slots and counters", tag);
    if (!q4k_layout_ok(tag, qtype, N)) return -1;
    return sera_launch_q4k_mmq_tail_acc(qtype, W, mmq_stage, Y, slots, counters, M, N, K, dp_tiles, pieces,
                                        accum ? 1 : 0, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "%s: launch failed", tag);
}

extern "C" int sera_q4k_mmq_streamk(const void *W, const void *mmq_stage, float *Y, float *slots, int *counters,
                                    int M, int N, int K, int wgs, void *stream) {
    return sera_q4k_mmq_streamk_qt(12u, W, mmq_stage, Y, slots, counters, M, N, K, wgs, stream);
}

extern "C" int sera_q4k_mmq_streamk_qt(uint32_t qtype, const void *W, const void *mmq_stage, float *Y, float *slots,
                                       int *counters, int M, int N, int K, int wgs, void *stream) {
    if (!W || !mmq_stage || !Y || !slots || !counters) return fail(-1, "sera_q4k_mmq_streamk: null pointer");
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK)
        return fail(-1, "sera_q4k_mmq_streamk: bad shape M=%d N=%d K=%d", M, N, K);
    if (!stage_ok("sera_q4k_mmq_streamk", M, K)) return -1;
    if (wgs == 0) wgs = streamk_wgs(M);
    if (wgs < 8 || wgs % 8)
        return fail(-1, "sera_q4k_mmq_streamk: workgroups=%d must be a positive multiple of 8", wgs);
    if ((int64_t)sera_mmq_tiles(M, N) * (K / Q4K_QK) < wgs)
        return fail(-1, "sera_q4k_mmq_streamk: fewer (tile, super-block) units than workgroups=%d", wgs);
    if (!q4k_layout_ok("sera_q4k_mmq_streamk", qtype, N)) return -1;
    return sera_launch_q4k_mmq_streamk(qtype, W, mmq_stage, Y, slots, counters, M, N, K, wgs, (hipStream_t)stream) ==
                   hipSuccess
               ? 0 : fail(-3, "sera_q4k_mmq_streamk: launch failed");
}

extern "C" int sera_q4k_mmq_tiles(int M, int N) { return M > 0 && N > 0 ? sera_mmq_tiles(M, N) : 0; }
extern "C" int sera_q4k_mmq_slot_floats(int M) { return M > 0 ? sera_mmq_slot_floats(M) : 0; }

extern "C" int sera_q4k_kernel_launches(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    if (sera_q4k_mmq_uses_fewtok(M, N, K)) return 2;   /* the few-token kernel sums split K inside */
    if (g_counters && tail_rule(M, N)) return 2;
    if (use_streamk(M, N, K)) return 2;
    return sera_mmq_splits(M, N, K) > 1 && ((size_t)M * N) % 4 == 0 ? 3 : 2;
}

extern "C" int sera_q4k_dense_vec(const void *W, const float *X, float *Y, int M, int N, int K, void *stream,
                                  int timed) {
    return sera_q4k_dense_vec_qt(12u, W, X, Y, M, N, K, stream, timed);
}

extern "C" int sera_q4k_dense_vec_qt(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                                     void *stream, int timed) {
    if (!check_shape("sera_q4k_dense_vec", W, X, Y, M, N, K)) return -1;
    if (!q4k_layout_ok("sera_q4k_dense_vec", qtype, N)) return -1;
    if (M > SERA_Q4K_MMVQ_MAX_BATCH)
        return fail(-1, "sera_q4k_dense_vec: batch M=%d exceeds MMVQ cap %d", M, SERA_Q4K_MMVQ_MAX_BATCH);
    if (!g_arena) return fail(-1, "sera_q4k_dense_vec: no arena attached");
    return dense_vec_on("sera_q4k_dense_vec", qtype, W, X, Y, M, N, K, (hipStream_t)stream, timed, g_arena,
                        g_arena_bytes, g_counters + kFewtokCounterBase, kFewtokMaxCounters);
}

extern "C" size_t sera_q4k_dense_vec_static_bytes(int M, int N, int K) {
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    size_t bytes = kStaticCounterBytes + sera_row_stage_layout((size_t)M, (size_t)K).total;
    if (sera_q4k_vec_uses_fewtok(M, N, K)) {
        const int splits = sera_fewtok_splits(M, N, K, 0);
        if (splits > 1) bytes += (size_t)splits * M * N * sizeof(float);
    }
    return bytes;
}

extern "C" int sera_q4k_dense_vec_static(const void *W, const float *X, float *Y, int M, int N, int K, void *stream) {
    const char *tag = "sera_q4k_dense_vec_static";
    if (!check_shape(tag, W, X, Y, M, N, K)) return -1;
    if (M > SERA_Q4K_MMVQ_MAX_BATCH) return fail(-1, "%s: batch M=%d exceeds MMVQ cap %d", tag, M, SERA_Q4K_MMVQ_MAX_BATCH);
    const size_t need = sera_q4k_dense_vec_static_bytes(M, N, K);
    if (need > SERA_Q4K_STATIC_SCRATCH_BYTES)
        return fail(-1, "%s: M=%d N=%d K=%d needs %zu bytes of scratch, more than the static %zu", tag, M, N, K, need,
                    (size_t)SERA_Q4K_STATIC_SCRATCH_BYTES);
    if (sera_q4k_vec_uses_fewtok(M, N, K) && sera_fewtok_splits(M, N, K, 0) > 1 &&
        sera_fewtok_groups(M, N, K) > (int)(kStaticCounterBytes / sizeof(int)))
        return fail(-1, "%s: N=%d needs more row-group counters than the static scratch holds", tag, N);
    hipStream_t s = (hipStream_t)stream;
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess) return fail(-1, "%s: hipGetDevice failed", tag);
    if (static_scratch_setup(device, s) != 0) return -1;
    unsigned char *base = g_scratch_ptr[device];
    return dense_vec_on(tag, 12u, W, X, Y, M, N, K, s, 0, base + kStaticCounterBytes,
                        SERA_Q4K_STATIC_SCRATCH_BYTES - kStaticCounterBytes, (int *)base,
                        (int)(kStaticCounterBytes / sizeof(int)));
}

/* ---- Q6_K ---------------------------------------------------------------- */

namespace {
/* Q6_K rows are K/256 * 210 bytes; the kernels address a row's bytes with
 * 32-bit offsets from the start of a group of rows. qtype: 14 (GGUF bytes)
 * or SERA_QTYPE_Q6K_SPLIT. */
bool q6k_shape_ok(const char *tag, uint32_t qtype, int K) {
    if (qtype != 14u && qtype != SERA_QTYPE_Q6K_SPLIT) {
        fail(-1, "%s: qtype %u is not Q6_K (14) or Q6_K split (%u)", tag, qtype, SERA_QTYPE_Q6K_SPLIT);
        return false;
    }
    if ((uint64_t)(K / Q4K_QK) * 210u * 256u >= (1ull << 31)) {
        fail(-1, "%s: K=%d too long for 32-bit row offsets", tag, K);
        return false;
    }
    return true;
}
}  // namespace

extern "C" int sera_q6k_mmvq_rows_per_wave(int M, int N) {
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH || N <= 0) return 0;
    return sera_q6k_mmvq_rows(N, M);
}

extern "C" int sera_q6k_mmvq(uint32_t qtype, const void *W, const void *row_stage, float *Y, int M, int N, int K,
                             int rows, void *stream) {
    if (!W || !row_stage || !Y) return fail(-1, "sera_q6k_mmvq: null pointer");
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH) return fail(-1, "sera_q6k_mmvq: batch M=%d outside 1..8", M);
    if (N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q6k_mmvq: bad shape N=%d K=%d", N, K);
    if (!stage_ok("sera_q6k_mmvq", M, K)) return -1;
    if (!q6k_shape_ok("sera_q6k_mmvq", qtype, K)) return -1;
    if (qtype == SERA_QTYPE_Q6K_SPLIT) {
        if (rows != 0 && rows != 2 && rows != 4)
            return fail(-1, "sera_q6k_mmvq: rows=%d not in {0,2,4} for the split layout", rows);
    } else {
        if (rows != 0 && rows != 1 && rows != 2 && rows != 4)
            return fail(-1, "sera_q6k_mmvq: rows_per_wave=%d not in {0,1,2,4}", rows);
        if (rows == 4 && M > 4) return fail(-1, "sera_q6k_mmvq: rows_per_wave=4 needs M <= 4");
    }
    if (((uintptr_t)W & 15u) != 0) return fail(-1, "sera_q6k_mmvq: W must be 16-byte aligned");
    return sera_launch_q6k_mmvq(qtype, W, row_stage, Y, M, N, K, rows, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q6k_mmvq: launch failed");
}

namespace {
/* Q6_K tile kernel schedule: the tail (every tile cut into K pieces handed
 * off through counters, no reduce launch) when one round of resident
 * workgroups (P = 2 per CU) gives each tile at least 4 pieces of at least 5
 * super-blocks; split-K with its reduce launch otherwise. Measured on
 * MI355X, split layout, kernel us tail / split-K: down 5120 x 25600 at 8
 * tokens 41.8 (12 pieces) / 48.5 (16 splits), at 64 61.6 / 67.1, at 128
 * 97.3 (6) / 102.5 (16); at 512, the same 4 K ranges both ways, 335 / 314
 * (the hand-off's write-through slot traffic costs more than the reduce);
 * q 8192 x 5120 at 8 (8 pieces of 2.5 super-blocks) 18.5 / 17.4. */
bool q6k_tail_plan(int M, int N, int K, size_t cap, int *dp, int *pieces) {
    if (!g_counters || g_cus <= 0) return false;
    const int T = sera_q6k_mmq_tiles(M, N, K);
    const int p = 2 * g_cus / T, nkb = K / Q4K_QK;
    if (T > kFewtokCounterBase || p < 4 || nkb < 5 * p) return false;
    const int pc = p < 63 ? p : 63;
    if (sera_q6k_mmq_tail_slot_floats(M, N, K, 0, pc) > cap) return false;
    *dp = 0;
    *pieces = pc;
    return true;
}

/* The Q6_K tile kernel on stage (Mpad rows) with cap floats of scratch at
 * partial: the tail schedule or split-K (splits as sera_q6k_mmq_splits, 1
 * when M*N % 4 or cap does not allow). */
hipError_t q6k_tile_launch(uint32_t qt, const void *W, const void *stage, float *Y, float *partial, size_t cap, int M,
                           int N, int K, int accum, hipStream_t s) {
    int dp, pieces;
    if (q6k_tail_plan(M, N, K, cap, &dp, &pieces))
        return sera_launch_q6k_mmq_tail_acc(qt, W, stage, Y, partial, g_counters, M, N, K, dp, pieces, accum, s);
    int sp = ((size_t)M * N) % 4 == 0 ? sera_q6k_mmq_splits(M, N, K) : 1;
    if ((size_t)sp * M * N > cap) sp = 1;
    return sera_launch_q6k_mmq_acc(qt, W, stage, Y, partial, M, N, K, sp, accum, s);
}

/* launches of q6k_tile_launch: 1, or 2 with a reduce */
int q6k_tile_launches(int M, int N, int K) {
    int dp, pieces;
    if (q6k_tail_plan(M, N, K, (size_t)-1, &dp, &pieces)) return 1;
    return (((size_t)M * N) % 4 == 0 && sera_q6k_mmq_splits(M, N, K) > 1) ? 2 : 1;
}
}  // namespace

/* Q6_K batches on the MMVQ path (M <= 8) run the MFMA tile kernel on a
 * row-formula stage (the MMVQ arithmetic) instead of the MMVQ kernel where
 * that is faster. Measured on MI355X per shape (kernel us, MMVQ / tile):
 * the tile kernel's time is flat in M, MMVQ's grows.
 *   GGUF bytes: LM head 151936 rows: 3 tokens 219 / 222, 4: 200-253 / 202-220;
 *     q 8192 x 5120: 5: 20.0 / 20.0, 6: 21.6 / 19.5; down 5120 x 25600
 *     (tail schedule): 4: 46.9 / 47.7, 5: 51.8 / 46.3;
 *   split layout (its own MMVQ kernel is faster): LM head 4 tokens 178 /
 *     174; q 6: 16.4 / 18.4, 7: 20.0 / 17.8; down 5: 42.5 / 44.0, 6: 45.4 /
 *     43.7;
 *   v 1024 rows: 8 tokens 8.2 / 13.7 (MMVQ at every batch, both layouts).
 * On 4096-16383 rows a K of 16384 or more (down) lets the tile kernel run
 * its tail schedule, one token earlier. */
extern "C" int sera_q6k_vec_uses_tile_qt(uint32_t qtype, int M, int N, int K) {
    if (qtype != 14u && qtype != SERA_QTYPE_Q6K_SPLIT) return 0;
    if (M < 1 || M > SERA_Q4K_MMVQ_MAX_BATCH || N <= 0) return 0;
    if (N >= 16384) return M >= 4;
    if (N >= 4096) return M >= (qtype == 14u ? 6 : 7) - (K >= 16384 ? 1 : 0);
    return 0;
}

extern "C" int sera_q6k_vec_uses_tile(int M, int N, int K) { return sera_q6k_vec_uses_tile_qt(14u, M, N, K); }

extern "C" int sera_q6k_dense_vec(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                                  void *stream, int timed) {
    if (!check_shape("sera_q6k_dense_vec", W, X, Y, M, N, K)) return -1;
    if (M > SERA_Q4K_MMVQ_MAX_BATCH)
        return fail(-1, "sera_q6k_dense_vec: batch M=%d exceeds MMVQ cap %d", M, SERA_Q4K_MMVQ_MAX_BATCH);
    if (!q6k_shape_ok("sera_q6k_dense_vec", qtype, K)) return -1;
    if (!g_arena) return fail(-1, "sera_q6k_dense_vec: no arena attached");
    hipStream_t s = (hipStream_t)stream;
    const bool mfma = sera_q6k_vec_uses_tile_qt(qtype, M, N, K) != 0;
    const int Mpad = sera_q6k_mmq_padded_rows(M);
    const size_t stage_bytes = mfma ? sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K).total
                                    : sera_row_stage_layout((size_t)M, (size_t)K).total;
    if (stage_bytes > g_arena_bytes)
        return fail(-1, "sera_q6k_dense_vec: arena too small (%zu > %zu)", stage_bytes, g_arena_bytes);
    if (timed) record(g_ev.quant_begin, s);
    const hipError_t qe = mfma ? sera_launch_q8_1_q6k_stage(X, M, Mpad, K, 1, g_arena, s)
                               : sera_launch_q8_1_row(X, M, K, g_arena, s);
    if (qe != hipSuccess) return fail(-2, "sera_q6k_dense_vec: quantize launch failed");
    if (timed) record(g_ev.quant_end, s);
    if (timed) record(g_ev.kernel_begin, s);
    if (mfma) {
        if (q6k_tile_launch(qtype, W, g_arena, Y, (float *)(g_arena + stage_bytes),
                            (g_arena_bytes - stage_bytes) / sizeof(float), M, N, K, 0, s) != hipSuccess)
            return fail(-3, "sera_q6k_dense_vec: tile kernel launch failed");
    } else if (sera_launch_q6k_mmvq(qtype, W, g_arena, Y, M, N, K, 0, s) != hipSuccess) {
        return fail(-3, "sera_q6k_dense_vec: mmvq launch failed");
    }
    if (timed) record(g_ev.kernel_end, s);
    return 0;
}

namespace {
int q6k_splits(int M, int N, int K) {
    return ((size_t)M * N) % 4 == 0 ? sera_q6k_mmq_splits(M, N, K) : 1;
}
}  // namespace

extern "C" int sera_q6k_kernel_launches_qt(uint32_t qtype, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    if (M <= SERA_Q4K_MMVQ_MAX_BATCH && !sera_q6k_vec_uses_tile_qt(qtype, M, N, K)) return 2;
    return 1 + q6k_tile_launches(M, N, K);
}

extern "C" int sera_q6k_kernel_launches(int M, int N, int K) { return sera_q6k_kernel_launches_qt(14u, M, N, K); }

extern "C" int sera_q8_1_q6k_mmq_padded_rows(int M) { return M > 0 ? sera_q6k_mmq_padded_rows(M) : 0; }

extern "C" size_t sera_q8_1_q6k_mmq_stage_bytes(int M, int K) {
    if (M <= 0 || K <= 0) return 0;
    return sera_q6k_mmq_stage_layout((size_t)sera_q6k_mmq_padded_rows(M), (size_t)K).total;
}

extern "C" void sera_q8_1_q6k_mmq_stage_offsets(int M, int K, size_t *qs, size_t *d) {
    const size_t mp = M > 0 ? (size_t)sera_q6k_mmq_padded_rows(M) : 0;
    const sera_stage_layout L = sera_q6k_mmq_stage_layout(mp, (size_t)(K > 0 ? K : 0));
    if (qs) *qs = L.qs;
    if (d) *d = L.ds;
}

extern "C" int sera_q8_1_quantize_mmq_d4(const float *X, int M, int K, void *stage, void *stream) {
    if (!X || !stage || M <= 0 || K <= 0 || K % Q4K_QK)
        return fail(-1, "sera_q8_1_quantize_mmq_d4: bad arguments");
    if (!stage_ok("sera_q8_1_quantize_mmq_d4", M, K)) return -1;
    if (((uintptr_t)X & 15u) != 0) return fail(-1, "sera_q8_1_quantize_mmq_d4: X must be 16-byte aligned");
    return sera_launch_q8_1_q6k_stage(X, M, sera_q6k_mmq_padded_rows(M), K, 0, stage, (hipStream_t)stream) ==
                   hipSuccess
               ? 0 : fail(-2, "sera_q8_1_quantize_mmq_d4: launch failed");
}

extern "C" int sera_q8_1_quantize_row_q6k(const float *X, int M, int K, void *stage, void *stream) {
    if (!X || !stage || M <= 0 || K <= 0 || K % Q4K_QK)
        return fail(-1, "sera_q8_1_quantize_row_q6k: bad arguments");
    if (!stage_ok("sera_q8_1_quantize_row_q6k", M, K)) return -1;
    if (((uintptr_t)X & 15u) != 0) return fail(-1, "sera_q8_1_quantize_row_q6k: X must be 16-byte aligned");
    return sera_launch_q8_1_q6k_stage(X, M, sera_q6k_mmq_padded_rows(M), K, 1, stage, (hipStream_t)stream) ==
                   hipSuccess
               ? 0 : fail(-2, "sera_q8_1_quantize_row_q6k: launch failed");
}

extern "C" int sera_q6k_mmq_splits_for(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    return q6k_splits(M, N, K);
}

extern "C" int sera_q6k_mmq(uint32_t qtype, const void *W, const void *q6k_mmq_stage, float *Y, float *partial,
                            int M, int N, int K, int splits, void *stream) {
    if (!W || !q6k_mmq_stage || !Y) return fail(-1, "sera_q6k_mmq: null pointer");
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q6k_mmq: bad shape M=%d N=%d K=%d", M, N, K);
    if (!stage_ok("sera_q6k_mmq", M, K)) return -1;
    if (((uintptr_t)W & 15u) != 0) return fail(-1, "sera_q6k_mmq: W must be 16-byte aligned");
    if (!q6k_shape_ok("sera_q6k_mmq", qtype, K)) return -1;
    if (splits == 0) splits = q6k_splits(M, N, K);
    if (splits < 1 || splits > K / Q4K_QK) return fail(-1, "sera_q6k_mmq: splits=%d outside 1..K/256", splits);
    if (splits > 1 && (!partial || ((size_t)M * N) % 4 != 0))
        return fail(-1, "sera_q6k_mmq: split-K needs a partial buffer and M*N %% 4 == 0");
    return sera_launch_q6k_mmq(qtype, W, q6k_mmq_stage, Y, partial, M, N, K, splits, (hipStream_t)stream) ==
                   hipSuccess
               ? 0 : fail(-3, "sera_q6k_mmq: launch failed");
}

extern "C" int sera_q6k_mmq_tail(uint32_t qtype, const void *W, const void *q6k_mmq_stage, float *Y, float *slots,
                                 int *counters, int M, int N, int K, int dp_tiles, int pieces, int accum, void *stream) {
    const char *tag = "sera_q6k_mmq_tail";
    if (!W || !q6k_mmq_stage || !Y) return fail(-1, "%s: null pointer", tag);
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "%s: bad shape M=%d N=%d K=%d", tag, M, N, K);
    if (!stage_ok(tag, M, K)) return -1;
    if (((uintptr_t)W & 15u) != 0) return fail(-1, "%s: W must be 16-byte aligned", tag);
    if (!q6k_shape_ok(tag, qtype, K)) return -1;
    const int T = sera_q6k_mmq_tiles(M, N, K);
    if (dp_tiles < 0 || dp_tiles > T) return fail(-1, "%s: dp_tiles=%d outside 0..%d", tag, dp_tiles, T);
    if (pieces < 1 || pieces > K / Q4K_QK) return fail(-1, "%s: pieces=%d outside 1..K/256", tag, pieces);
    if (pieces > 1 && dp_tiles < T && (!slots || !counters))
        return fail(-1, "%s: a split tail needs slots and counters", tag);
    return sera_launch_q6k_mmq_tail_acc(qtype, W, q6k_mmq_stage, Y, slots, counters, M, N, K, dp_tiles, pieces,
                                        accum ? 1 : 0, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "%s: launch failed", tag);
}

extern "C" int sera_q6k_mmq_tail_plan(int M, int N, int K, size_t max_slot_floats, int *dp_tiles, int *pieces) {
    if (M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q6k_mmq_tail_plan: bad shape");
    int dp = 0, pc = 1;
    const size_t cap = max_slot_floats ? max_slot_floats : (size_t)-1;
    const int tail = q6k_tail_plan(M, N, K, cap, &dp, &pc) ? 1 : 0;
    if (dp_tiles) *dp_tiles = tail ? dp : 0;
    if (pieces) *pieces = tail ? pc : 0;
    return tail;
}

extern "C" int sera_q6k_dense(uint32_t qtype, const void *W, const float *X, float *Y, int M, int N, int K,
                              void *stream, int timed) {
    if (!check_shape("sera_q6k_dense", W, X, Y, M, N, K)) return -1;
    if (!q6k_shape_ok("sera_q6k_dense", qtype, K)) return -1;
    if (!g_arena) return fail(-1, "sera_q6k_dense: no arena attached");
    hipStream_t s = (hipStream_t)stream;
    const int Mpad = sera_q6k_mmq_padded_rows(M);
    const size_t stage_bytes = sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K).total;
    if (stage_bytes > g_arena_bytes)
        return fail(-1, "sera_q6k_dense: arena too small (%zu > %zu)", stage_bytes, g_arena_bytes);
    if (timed) record(g_ev.quant_begin, s);
    if (sera_launch_q8_1_q6k_stage(X, M, Mpad, K, 0, g_arena, s) != hipSuccess)
        return fail(-2, "sera_q6k_dense: quantize launch failed");
    if (timed) record(g_ev.quant_end, s);
    if (timed) record(g_ev.kernel_begin, s);
    if (q6k_tile_launch(qtype, W, g_arena, Y, (float *)(g_arena + stage_bytes),
                        (g_arena_bytes - stage_bytes) / sizeof(float), M, N, K, 0, s) != hipSuccess)
        return fail(-3, "sera_q6k_dense: mmq launch failed");
    if (timed) record(g_ev.kernel_end, s);
    return 0;
}

/* ---- device layouts at upload ------------------------------------------ */

namespace {
bool layout_args_ok(const char *tag, uint32_t qtype, int N, int K) {
    if (qtype != 12u && qtype != SERA_QTYPE_Q4K_TILED && qtype != 14u && qtype != SERA_QTYPE_Q6K_SPLIT) {
        fail(-1, "%s: qtype %u is not Q4_K (12), Q4_K tiled (%u), Q6_K (14) or Q6_K split (%u)", tag, qtype,
             SERA_QTYPE_Q4K_TILED, SERA_QTYPE_Q6K_SPLIT);
        return false;
    }
    if (N <= 0 || K <= 0 || K % Q4K_QK) {
        fail(-1, "%s: bad shape N=%d K=%d", tag, N, K);
        return false;
    }
    if (qtype == SERA_QTYPE_Q4K_TILED && N % Q4K_TILE_ROWS) {
        fail(-1, "%s: the tiled layout needs N %% 16 == 0 (N=%d)", tag, N);
        return false;
    }
    return true;
}
}  // namespace

extern "C" size_t sera_weight_bytes(uint32_t qtype, int N, int K) {
    const bool q4 = qtype == 12u || qtype == SERA_QTYPE_Q4K_TILED;
    if ((!q4 && qtype != 14u && qtype != SERA_QTYPE_Q6K_SPLIT) || N <= 0 || K <= 0 || K % Q4K_QK) return 0;
    if (qtype == SERA_QTYPE_Q4K_TILED && N % Q4K_TILE_ROWS) return 0;
    return (size_t)N * (size_t)(K / Q4K_QK) * (q4 ? Q4K_BLOCK_BYTES : Q6K_GGUF_BYTES);
}

extern "C" int sera_weight_to_device_layout(uint32_t qtype, int N, int K, const void *gguf, void *dst, void *stream) {
    const char *tag = "sera_weight_to_device_layout";
    if (!gguf || !dst) return fail(-1, "%s: null pointer", tag);
    if (!layout_args_ok(tag, qtype, N, K)) return -1;
    const size_t bytes = sera_weight_bytes(qtype, N, K);
    hipStream_t s = (hipStream_t)stream;
    if (qtype == 12u || qtype == 14u) {
        if (gguf == dst) return 0;
        return hipMemcpyAsync(dst, gguf, bytes, hipMemcpyDeviceToDevice, s) == hipSuccess
                   ? 0 : fail(-3, "%s: copy failed", tag);
    }
    const char *a = (const char *)gguf, *b = (const char *)dst;
    if (a < b + bytes && b < a + bytes) return fail(-1, "%s: source and destination overlap", tag);
    if (qtype == SERA_QTYPE_Q4K_TILED) {
        if (((uintptr_t)gguf & 15u) || ((uintptr_t)dst & 15u))
            return fail(-1, "%s: GGUF bytes and dst must be 16-byte aligned", tag);
        return sera_launch_q4k_tile(gguf, dst, 0, (uint64_t)N, (uint64_t)(K / Q4K_QK), s) == hipSuccess
                   ? 0 : fail(-3, "%s: launch failed", tag);
    }
    if (((uintptr_t)gguf & 1u) || ((uintptr_t)dst & 15u))
        return fail(-1, "%s: GGUF bytes must be 2-byte and dst 16-byte aligned", tag);
    const uint64_t total = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    return sera_launch_q6k_split(gguf, dst, 0, total, total, s) == hipSuccess ? 0 : fail(-3, "%s: launch failed", tag);
}

extern "C" int sera_weight_upload(uint32_t qtype, int N, int K, const void *host_gguf, void *dst, void *staging,
                                  size_t staging_bytes, void *stream) {
    const char *tag = "sera_weight_upload";
    if (!host_gguf || !dst) return fail(-1, "%s: null pointer", tag);
    if (!layout_args_ok(tag, qtype, N, K)) return -1;
    const size_t bytes = sera_weight_bytes(qtype, N, K);
    hipStream_t s = (hipStream_t)stream;
    if (qtype == 12u || qtype == 14u)
        return hipMemcpyAsync(dst, host_gguf, bytes, hipMemcpyHostToDevice, s) == hipSuccess
                   ? 0 : fail(-3, "%s: host-to-device copy failed", tag);
    if (qtype == SERA_QTYPE_Q4K_TILED) {
        /* whole 16-row groups through the staging buffer */
        const uint64_t nkb = (uint64_t)(K / Q4K_QK);
        const uint64_t group_bytes = Q4K_TILE_ROWS * nkb * Q4K_BLOCK_BYTES;
        if (!staging || staging_bytes < group_bytes)
            return fail(-1, "%s: the tiled layout needs a device staging buffer of at least %llu bytes", tag,
                        (unsigned long long)group_bytes);
        if (((uintptr_t)staging & 15u) || ((uintptr_t)dst & 15u))
            return fail(-1, "%s: staging and dst must be 16-byte aligned", tag);
        const uint64_t per = (staging_bytes / group_bytes) * Q4K_TILE_ROWS;
        const char *src = (const char *)host_gguf;
        for (uint64_t row0 = 0; row0 < (uint64_t)N; row0 += per) {
            const uint64_t rows = (uint64_t)N - row0 < per ? (uint64_t)N - row0 : per;
            if (hipMemcpyAsync(staging, src + row0 * nkb * Q4K_BLOCK_BYTES, rows * nkb * Q4K_BLOCK_BYTES,
                               hipMemcpyHostToDevice, s) != hipSuccess)
                return fail(-3, "%s: host-to-device copy failed", tag);
            if (sera_launch_q4k_tile(staging, dst, row0, rows, nkb, s) != hipSuccess)
                return fail(-3, "%s: repack launch failed", tag);
        }
        return 0;
    }
    if (!staging || staging_bytes < Q6K_GGUF_BYTES)
        return fail(-1, "%s: the split layout needs a device staging buffer of at least %d bytes", tag,
                    Q6K_GGUF_BYTES);
    if (((uintptr_t)staging & 15u) || ((uintptr_t)dst & 15u))
        return fail(-1, "%s: staging and dst must be 16-byte aligned", tag);
    const uint64_t total = (uint64_t)N * (uint64_t)(K / Q4K_QK);
    const uint64_t per = staging_bytes / Q6K_GGUF_BYTES;
    const char *src = (const char *)host_gguf;
    /* one stream: the copy into the staging buffer waits for the repack that
     * last read it */
    for (uint64_t first = 0; first < total; first += per) {
        const uint64_t count = total - first < per ? total - first : per;
        if (hipMemcpyAsync(staging, src + first * Q6K_GGUF_BYTES, count * Q6K_GGUF_BYTES, hipMemcpyHostToDevice,
                           s) != hipSuccess)
            return fail(-3, "%s: host-to-device copy failed", tag);
        if (sera_launch_q6k_split(staging, dst, first, count, total, s) != hipSuccess)
            return fail(-3, "%s: repack launch failed", tag);
    }
    return 0;
}

/* ---- gathered rows ----------------------------------------------------- */

namespace {
bool rows_shape_ok(const char *tag, int qtype, const void *W, int N, int K) {
    if (!W) { fail(-1, "%s: null weight pointer", tag); return false; }
    if (qtype != 12 && qtype != (int)SERA_QTYPE_Q4K_TILED && qtype != 14 && qtype != (int)SERA_QTYPE_Q6K_SPLIT) {
        fail(-1, "%s: qtype %d is not Q4_K (12), Q4_K tiled (%u), Q6_K (14) or Q6_K split (%u)", tag, qtype,
             SERA_QTYPE_Q4K_TILED, SERA_QTYPE_Q6K_SPLIT);
        return false;
    }
    if (qtype == (int)SERA_QTYPE_Q4K_TILED && N % Q4K_TILE_ROWS) {
        fail(-1, "%s: the tiled layout needs N %% 16 == 0 (N=%d)", tag, N);
        return false;
    }
    if (N <= 0 || K <= 0 || K % Q4K_QK) { fail(-1, "%s: bad shape N=%d K=%d", tag, N, K); return false; }
    if (((uintptr_t)W & 15u) != 0) { fail(-1, "%s: W must be 16-byte aligned", tag); return false; }
    if ((uint64_t)(K / Q4K_QK) * 210u >= (1ull << 30)) { fail(-1, "%s: K=%d too long", tag, K); return false; }
    return true;
}
}  // namespace

extern "C" int sera_candidate_logits(int qtype, const void *W, int N, int K, const float *hidden, int branches,
                                     const uint32_t *ids, int per_branch, float *logits, void *stream) {
    if (!rows_shape_ok("sera_candidate_logits", qtype, W, N, K)) return -1;
    if (!hidden || !ids || !logits) return fail(-1, "sera_candidate_logits: null pointer");
    if (branches <= 0 || per_branch <= 0 || (int64_t)branches * per_branch > (1 << 28))
        return fail(-1, "sera_candidate_logits: bad counts branches=%d per_branch=%d", branches, per_branch);
    if (((uintptr_t)hidden & 15u) != 0) return fail(-1, "sera_candidate_logits: hidden must be 16-byte aligned");
    return sera_launch_candidate_logits(qtype, W, N, K, hidden, ids, branches, per_branch, logits,
                                        (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_candidate_logits: launch failed");
}

extern "C" int sera_embedding(int qtype, const void *W, int N, int K, const uint32_t *ids, int tokens, float *hidden,
                              void *stream) {
    if (!rows_shape_ok("sera_embedding", qtype, W, N, K)) return -1;
    if (!ids || !hidden || tokens <= 0) return fail(-1, "sera_embedding: bad arguments");
    if (((uintptr_t)hidden & 15u) != 0) return fail(-1, "sera_embedding: hidden must be 16-byte aligned");
    return sera_launch_embedding(qtype, W, N, K, ids, tokens, hidden, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_embedding: launch failed");
}

/* ---- fused linear group ----------------------------------------------- */

extern "C" int sera_linear_group(int count, const void *const *geometries, const void *const *weights,
                                 float *const *outputs, const float *X, const float *X2, const float *gamma, float eps,
                                 size_t M_, unsigned flags, void *stream) {
    const char *tag = "sera_linear_group";
    if (count < 1 || count > SERA_LINEAR_GROUP_MAX || !geometries || !weights || !outputs || !X)
        return fail(-1, "%s: bad arguments (count=%d)", tag, count);
    if (!g_arena) return fail(-1, "%s: no arena attached", tag);
    if (M_ == 0 || M_ > 0x7fffffff) return fail(-1, "%s: bad token count", tag);
    if (flags & ~(SERA_LIN_ACCUMULATE | SERA_LIN_RMSNORM | SERA_LIN_SILU_MUL))
        return fail(-1, "%s: unknown flags 0x%x", tag, flags);
    if ((flags & SERA_LIN_RMSNORM) && (flags & SERA_LIN_SILU_MUL))
        return fail(-1, "%s: RMSNORM and SILU_MUL are exclusive", tag);
    if ((flags & SERA_LIN_RMSNORM) && (!gamma || ((uintptr_t)gamma & 15u)))
        return fail(-1, "%s: RMSNORM needs a 16-byte aligned gamma", tag);
    if ((flags & SERA_LIN_SILU_MUL) && (!X2 || ((uintptr_t)X2 & 15u)))
        return fail(-1, "%s: SILU_MUL needs a 16-byte aligned X2", tag);
    const int M = (int)M_;
    const q3_q4_linear_geometry *g0 = (const q3_q4_linear_geometry *)geometries[0];
    if (!g0) return fail(-1, "%s: null geometry", tag);
    const int K = g0->K;
    const uint32_t qt = g0->qtype;
    int N[SERA_LINEAR_GROUP_MAX];
    for (int i = 0; i < count; i++) {
        const q3_q4_linear_geometry *g = (const q3_q4_linear_geometry *)geometries[i];
        if (!g || g->K != K || g->qtype != qt || g->N <= 0)
            return fail(-1, "%s: geometry %d differs in K/qtype or is unresolved", tag, i);
        if (!check_shape(tag, weights[i], X, outputs[i], M, g->N, K)) return -1;
        N[i] = g->N;
    }
    if (qt != 12 && qt != SERA_QTYPE_Q4K_TILED && qt != 14 && qt != SERA_QTYPE_Q6K_SPLIT)
        return fail(-1, "%s: qtype %u is not Q4_K/Q6_K", tag, qt);
    /* q4: the Q4_K kernels, on GGUF bytes or the tiled layout */
    const bool q4 = qt == 12 || qt == SERA_QTYPE_Q4K_TILED;
    if (q4)
        for (int i = 0; i < count; i++)
            if (!q4k_layout_ok(tag, qt, N[i])) return -1;
    if (!q4 && !q6k_shape_ok(tag, qt, K)) return -1;
    hipStream_t s = (hipStream_t)stream;
    const int accum = (flags & SERA_LIN_ACCUMULATE) ? 1 : 0;
    sera_producer prod = {0, X2, gamma, eps};
    if (flags & SERA_LIN_RMSNORM) prod.kind = 1;
    if (flags & SERA_LIN_SILU_MUL) prod.kind = 2;

    /* Q6_K: one stage serves the whole group, so the largest matrix picks
     * between the MMVQ kernel (row stage) and the tile kernel */
    int n_max = 0;
    for (int i = 0; i < count; i++) n_max = N[i] > n_max ? N[i] : n_max;
    const bool q6_tile = M > SERA_Q4K_MMVQ_MAX_BATCH || sera_q6k_vec_uses_tile_qt(qt, M, n_max, K);

    /* stage, then per-matrix split-K partials or stream-K slots */
    size_t stage_bytes;
    int Mpad = M;
    if (q4) {
        if (M <= SERA_Q4K_MMVQ_MAX_BATCH) {
            stage_bytes = sera_row_stage_layout((size_t)M, (size_t)K).total;
        } else {
            Mpad = sera_mmq_padded_rows(M);
            stage_bytes = sera_mmq_stage_layout((size_t)Mpad, (size_t)K).total;
        }
    } else if (!q6_tile) {
        stage_bytes = sera_row_stage_layout((size_t)M, (size_t)K).total;
    } else {
        Mpad = sera_q6k_mmq_padded_rows(M);
        stage_bytes = sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K).total;
    }
    if (stage_bytes > g_arena_bytes) return fail(-1, "%s: arena too small for the stage", tag);
    float *partial = (float *)(g_arena + stage_bytes);
    const size_t partial_cap = (g_arena_bytes - stage_bytes) / sizeof(float);

    /* quantize once */
    hipError_t qe;
    if (q4)
        qe = M <= SERA_Q4K_MMVQ_MAX_BATCH ? sera_launch_q8_1_row_p(X, &prod, M, K, g_arena, s)
                                          : sera_launch_q8_1_mmq_p(X, &prod, M, Mpad, K, g_arena, s);
    else
        qe = !q6_tile
                 ? sera_launch_q8_1_row_p(X, &prod, M, K, g_arena, s)
                 : sera_launch_q8_1_q6k_stage_p(X, &prod, M, Mpad, K, M <= SERA_Q4K_MMVQ_MAX_BATCH ? 1 : 0,
                                                g_arena, s);
    if (qe != hipSuccess) return fail(-2, "%s: quantize launch failed", tag);

    /* the products */
    if (q4 && M <= SERA_Q4K_MMVQ_MAX_BATCH) {
        /* the matrices the dot4 kernel takes share one grouped launch; the
         * few-token kernel runs the others one by one */
        const void *gw[SERA_LINEAR_GROUP_MAX];
        float *gy[SERA_LINEAR_GROUP_MAX];
        int gn[SERA_LINEAR_GROUP_MAX];
        int g = 0;
        for (int i = 0; i < count; i++)
            if (!sera_q4k_vec_uses_fewtok_qt(qt, M, N[i], K)) {
                gw[g] = weights[i];
                gy[g] = outputs[i];
                gn[g] = N[i];
                g++;
            }
        if (g > 0 && sera_launch_q4k_mmvq_group(qt, g, gw, gy, gn, g_arena, M, K, 0, accum, s) != hipSuccess)
            return fail(-3, "%s: grouped mmvq launch failed", tag);
        for (int i = 0; i < count; i++)
            if (sera_q4k_vec_uses_fewtok_qt(qt, M, N[i], K)) {
                const int rc = fewtok_launch(tag, qt, 0, weights[i], outputs[i], partial, partial_cap, M, N[i], K,
                                             accum, s);
                if (rc) return rc;
            }
        return 0;
    }
    for (int i = 0; i < count; i++) {
        hipError_t e;
        const int n = N[i];
        if (q4 && sera_q4k_mmq_uses_fewtok(M, n, K)) {
            const int rc = fewtok_launch(tag, qt, 1, weights[i], outputs[i], partial, partial_cap, M, n, K, accum, s);
            if (rc) return rc;
            continue;
        } else if (q4) {
            const MmqPlan plan = mmq_plan(M, n, K, partial_cap, g_counters != nullptr);
            e = mmq_launch(plan, qt, weights[i], g_arena, outputs[i], partial, M, n, K, accum, s);
        } else if (!q6_tile) {
            e = sera_launch_q6k_mmvq_acc(qt, weights[i], g_arena, outputs[i], M, n, K, 0, accum, s);
        } else {
            e = q6k_tile_launch(qt, weights[i], g_arena, outputs[i], partial, partial_cap, M, n, K, accum, s);
        }
        if (e != hipSuccess) return fail(-3, "%s: product %d launch failed", tag, i);
    }
    return 0;
}

extern "C" void sera_q4k_read_timings(double *quant_ms, double *kernel_ms, double *total_ms) {
    float q = 0.0f, k = 0.0f, t = 0.0f;
    if (g_ev.valid) {
        if (hipEventElapsedTime(&q, g_ev.quant_begin, g_ev.quant_end) != hipSuccess) q = 0.0f;
        if (hipEventElapsedTime(&k, g_ev.kernel_begin, g_ev.kernel_end) != hipSuccess) k = 0.0f;
        if (hipEventElapsedTime(&t, g_ev.quant_begin, g_ev.kernel_end) != hipSuccess) t = 0.0f;
    }
    if (quant_ms) *quant_ms = q;
    if (kernel_ms) *kernel_ms = k;
    if (total_ms) *total_ms = t;
}

extern "C" int sera_q4k_dequantize(const void *W, size_t nblocks, float *out, void *stream) {
    if (!W || !out || nblocks == 0) return fail(-1, "sera_q4k_dequantize: bad arguments");
    return sera_launch_q4k_dequant(W, (int64_t)nblocks, out, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q4k_dequantize: launch failed");
}

extern "C" int sera_q4k_dequantize_qt(uint32_t qtype, const void *W, int N, int K, float *out, void *stream) {
    if (!W || !out || N <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q4k_dequantize: bad arguments");
    if (!q4k_layout_ok("sera_q4k_dequantize", qtype, N)) return -1;
    const hipError_t e = qtype == SERA_QTYPE_Q4K_TILED
                             ? sera_launch_q4k_dequant_tiled(W, N, K, out, (hipStream_t)stream)
                             : sera_launch_q4k_dequant(W, (int64_t)N * (K / Q4K_QK), out, (hipStream_t)stream);
    return e == hipSuccess ? 0 : fail(-3, "sera_q4k_dequantize: launch failed");
}

extern "C" int sera_q4k_subblock_dots(const void *W, const void *stage_qs, int32_t *I, int M, int N, int K,
                                      void *stream) {
    if (!W || !stage_qs || !I || M <= 0 || N <= 0 || K <= 0 || K % Q4K_QK)
        return fail(-1, "sera_q4k_subblock_dots: bad arguments");
    return sera_launch_q4k_subblock_dots(W, (const int8_t *)stage_qs, I, M, N, K, (hipStream_t)stream) ==
                   hipSuccess
               ? 0 : fail(-3, "sera_q4k_subblock_dots: launch failed");
}

extern "C" int sera_q4k_quantize(const float *X, int64_t rows, int64_t K, void *out, void *stream) {
    if (!X || !out || rows <= 0 || K <= 0 || K % Q4K_QK) return fail(-1, "sera_q4k_quantize: bad arguments");
    return sera_launch_q4k_quantize(X, rows, K, out, (hipStream_t)stream) == hipSuccess
               ? 0 : fail(-3, "sera_q4k_quantize: launch failed");
}
