/*
 * q8_quantize.hip - fp32 activations -> Q8_1 (32 values per scale).
 *
 * Two quantizers, each bit-exact with one of the reference's formulas:
 *
 *  row (MMVQ activations), cuda/mmq/quantize.cu:4-48
 *     amax = max|x|, sum = xor-butterfly over offsets 16,8,4,2,1 of the 32
 *     values, d = amax/127, q = amax == 0 ? 0 : roundf(x/d),
 *     ds = (fp16(d), fp16(sum))
 *
 *  mmq (MMQ activations, DS4 layout), cuda/mmq/quantize.cu:271-367
 *     8 lanes hold 4 consecutive values each, lane sum ((x0+x1)+x2)+x3,
 *     then xor 4,2,1 across the 8 lanes; d_inv = 127/amax,
 *     q = roundf(x*d_inv), d = 1/d_inv; amax == 0 gives q = 0, d = 0.
 *
 *  mmq D4 (MMQ activations for Q6_K weights), the same kernel with the D4
 *     layout the reference selects for Q6_K (cuda/mmq/mmq.cuh:64-103,
 *     cuda/q3_mmq.cu:303-316): quants as above, fp32 d = 1/d_inv, no sum.
 *     This library stores 16 * quant as fp16 (exact) for the fp16-MFMA
 *     Q6_K kernel and d transposed per 256-wide K step (see q4k_common.h).
 *
 * Producers (sera_producer): each quantizer can compute its input row on the
 * fly instead of reading a materialized one, fusing the reference's
 * rms_norm_batched_kernel (src/q3_forward.cu:117-146) or silu_mul_kernel
 * (:154-161) into the quantize that follows it. RMSNorm: every workgroup of
 * a row first reduces the row's sum of squares in a fixed order (thread t
 * adds x[t + 256i]^2 in i order, the square exact in double and each sum
 * rounded to fp32 as the reference's float += double does; then an xor
 * butterfly over the wave and the four wave sums left to right), then
 * inv = 1 / sqrt(sum / K + eps) with IEEE division and square root (the
 * reference's rsqrtf is an approximation), x = (x * inv) * gamma. SiLU:
 * (g / (1 + expf(-g))) * u with the device expf.
 *
 * Division is IEEE correctly rounded (hipcc default), roundf rounds half
 * away from zero, fp16 conversion rounds to nearest even. The float sums are
 * pure additions in a fixed pairing, so they cannot be contracted or
 * reassociated by the compiler.
 */
#include "sera_launch.h"
#include "sera_dpp.h"

/* No floating-point contraction in this file: the values here must follow
 * the reference's separately rounded multiplies and adds (hipcc fuses a * b
 * + c into one FMA by default, and the _rn intrinsics are plain operators
 * that do not prevent it). Explicit fmaf calls are unaffected. */
#pragma clang fp contract(off)

/* 1 / sqrt(mean(x^2) + eps) of one row, computed by all 256 threads of the
 * workgroup (every thread returns the same value). Thread t adds x[t+256i]^2
 * in i order; the loads go out 32 at a time, so a row of up to 8192 values
 * costs one memory round trip. Past K a load reads the last element (a
 * valid address, no branch) and its value is replaced by zero, which the
 * non-negative running sum absorbs unchanged; a branch around each load
 * made the compiler wait for every load on its own. */
__device__ __forceinline__ float q8_row_inv_rms(const float *__restrict__ xr, int K, float eps) {
    __shared__ float s_red[4];
    float s = 0.0f;
    for (int k0 = threadIdx.x; k0 < K; k0 += 32 * 256) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float t = xr[min(k0 + 256 * j, K - 1)];
            v[j] = k0 + 256 * j < K ? t : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const double d = (double)v[j];
            s = (float)((double)s + d * d);
        }
    }
    s = __fadd_rn(s, xor_partner<32>(s));
    s = __fadd_rn(s, xor_partner<16>(s));
    s = __fadd_rn(s, xor_partner<8>(s));
    s = __fadd_rn(s, xor_partner<4>(s));
    s = __fadd_rn(s, xor_partner<2>(s));
    s = __fadd_rn(s, xor_partner<1>(s));
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float tot = __fadd_rn(__fadd_rn(__fadd_rn(s_red[0], s_red[1]), s_red[2]), s_red[3]);
    /* sqrtf is correctly rounded with hipcc defaults (__fsqrt_rn is not on gfx950) */
    return __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)K), eps)));
}

__device__ __forceinline__ float q8_silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

/* The producer's value at (row, k). For RMSNorm the element and its gamma
 * are loaded before the row's sum of squares (q8_produce_rms), so both
 * travel in the same memory round trip as the reduction's loads. */
template <int PK>
__device__ __forceinline__ float q8_produce(const float *__restrict__ x, const sera_producer &p, size_t idx) {
    const float v = x[idx];
    if (PK == 2) return q8_silu_mul(v, p.x2[idx]);
    return v;
}

__device__ __forceinline__ float q8_produce_rms(const float *__restrict__ x, const sera_producer &p, int row, int K,
                                                int k) {
    const float v = x[(size_t)row * K + k];
    const float g = p.gamma[k];
    const float inv = q8_row_inv_rms(x + (size_t)row * K, K, p.eps);
    return __fmul_rn(__fmul_rn(v, inv), g);
}

template <int PK>
__device__ __forceinline__ float4 q8_produce4(const float *__restrict__ x, const sera_producer &p, size_t idx) {
    const float4 v = *(const float4 *)(x + idx);
    if (PK == 2) {
        const float4 u = *(const float4 *)(p.x2 + idx);
        return make_float4(q8_silu_mul(v.x, u.x), q8_silu_mul(v.y, u.y), q8_silu_mul(v.z, u.z),
                           q8_silu_mul(v.w, u.w));
    }
    return v;
}

/* Four consecutive producer values (row, k..k+3) for the DS4 / Q6_K stage
 * kernels: zeros for padding rows (row >= M) and for k >= K. Every thread
 * of the workgroup takes part in the RMSNorm reduction, and its own values
 * and gammas are loaded before it. */
template <int PK>
__device__ __forceinline__ float4 q8_produce4_row(const float *__restrict__ x, const sera_producer &p, int row, int M,
                                                  int K, int k) {
    const bool live = row < M && k < K;
    if (PK == 1) {
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f), g = v;
        if (live) {
            v = *(const float4 *)(x + (size_t)row * K + k);
            g = *(const float4 *)(p.gamma + k);
        }
        const float inv = row < M ? q8_row_inv_rms(x + (size_t)row * K, K, p.eps) : 0.0f;
        return make_float4(__fmul_rn(__fmul_rn(v.x, inv), g.x), __fmul_rn(__fmul_rn(v.y, inv), g.y),
                           __fmul_rn(__fmul_rn(v.z, inv), g.z), __fmul_rn(__fmul_rn(v.w, inv), g.w));
    }
    return live ? q8_produce4<PK>(x, p, (size_t)row * K + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

/* One wave-64 handles two consecutive Q8_1 blocks (lanes 0-31 and 32-63);
 * a 256-thread workgroup covers 256 values of one activation row.
 * grid = (K/256, M). Writes qs, ds and the MMVQ helper dsf. */
template <int PK>
__global__ __launch_bounds__(256) void sera_q8_1_row_kernel(
        const float *__restrict__ x, sera_producer prod, int K, int8_t *__restrict__ qs,
        uint32_t *__restrict__ ds, float4 *__restrict__ dsf) {
    const int row = blockIdx.y;
    const int k = blockIdx.x * 256 + threadIdx.x;
    const float xi = PK == 1 ? q8_produce_rms(x, prod, row, K, k) : q8_produce<PK>(x, prod, (size_t)row * K + k);

    /* the 32-lane xor butterfly 16, 8, 4, 2, 1 of the reference (each lane
     * adds its partner's value; addition is commutative, so own + partner is
     * the reference's sum bit for bit) */
    float amax = fabsf(xi);
    float sum = xi;
    amax = fmaxf(amax, xor_partner<16>(amax));
    sum = sum + xor_partner<16>(sum);
    amax = fmaxf(amax, xor_partner<8>(amax));
    sum = sum + xor_partner<8>(sum);
    amax = fmaxf(amax, xor_partner<4>(amax));
    sum = sum + xor_partner<4>(sum);
    amax = fmaxf(amax, xor_partner<2>(amax));
    sum = sum + xor_partner<2>(sum);
    amax = fmaxf(amax, xor_partner<1>(amax));
    sum = sum + xor_partner<1>(sum);
    const float d = amax / 127.0f;
    const float qf = amax == 0.0f ? 0.0f : roundf(xi / d);
    const int q = (int)qf;
    qs[(size_t)row * K + k] = (int8_t)q;

    /* S = sum of the 32 quants (exact integer), for the MMVQ min term. */
    int s = q;
    s += xor_partner<16>(s);
    s += xor_partner<8>(s);
    s += xor_partner<4>(s);
    s += xor_partner<2>(s);
    s += xor_partner<1>(s);

    const uint32_t dh = f2h_bits(d);
    const uint32_t sh = f2h_bits(sum);
    const int lane = threadIdx.x & 63;
    const size_t blk = (size_t)row * (K / 32) + (k >> 5);
    if ((lane & 31) == 0) ds[blk] = dh | (sh << 16);

    /* dsf pairs block 2p (lanes 0-31) with block 2p+1 (lanes 32-63). */
    const float d8 = h2f_bits(dh);
    const float dS = d8 * (float)s;
    const float d8_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(d8), 32));
    const float dS_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dS), 32));
    if (lane == 0) {
        dsf[(size_t)row * (K / 64) + (k >> 6)] = make_float4(d8, d8_hi, dS, dS_hi);
    }
}

/* DS4 quantizer. Each thread holds 4 consecutive values (one float4); a
 * 256-thread workgroup covers 1024 values of one row. grid = (ceil(K/1024),
 * Mpad). Rows >= M (padding up to the MMQ tile) are written as zeros. */
template <int PK>
__global__ __launch_bounds__(256) void sera_q8_1_mmq_kernel(
        const float *__restrict__ x, sera_producer prod, int M, int K, int8_t *__restrict__ qs,
        uint32_t *__restrict__ ds) {
    const int row = blockIdx.y;
    const int k = (blockIdx.x * 256 + threadIdx.x) * 4;
    const float4 v = q8_produce4_row<PK>(x, prod, row, M, K, k);
    if (k >= K) return;

    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float sum = ((v.x + v.y) + v.z) + v.w;
    amax = fmaxf(amax, xor_partner<4>(amax));
    sum = sum + xor_partner<4>(sum);
    amax = fmaxf(amax, xor_partner<2>(amax));
    sum = sum + xor_partner<2>(sum);
    amax = fmaxf(amax, xor_partner<1>(amax));
    sum = sum + xor_partner<1>(sum);
    int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        const float d_inv = 127.0f / amax;
        q0 = (int)roundf(v.x * d_inv);
        q1 = (int)roundf(v.y * d_inv);
        q2 = (int)roundf(v.z * d_inv);
        q3 = (int)roundf(v.w * d_inv);
        d = 1.0f / d_inv;
    }
    const uint32_t packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                            ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
    *(uint32_t *)(qs + (size_t)row * K + k) = packed;
    if ((threadIdx.x & 7) == 0) {
        ds[(size_t)row * (K / 32) + (k >> 5)] = f2h_bits(d) | (f2h_bits(sum) << 16);
    }
}

/* Q6_K MMQ-layout stage: 16 * quant as fp16 [Mpad][K], fp32 d as
 * [K/256][8][Mpad]; grid = (ceil(K/1024), Mpad); rows >= M are zero.
 * ROW = false: the D4 quantizer (MMQ arithmetic): d_inv = 127/amax,
 *   q = roundf(x*d_inv), d = 1/d_inv in fp32.
 * ROW = true: the row quantizer's values (MMVQ arithmetic, the same as
 *   sera_q8_1_row_kernel): d = amax/127, q = roundf(x/d), and the scale
 *   kept as fp32(fp16(d)), the d8 the MMVQ formula multiplies by. */
template <bool ROW, int PK>
__global__ __launch_bounds__(256) void sera_q8_1_q6k_stage_kernel(
        const float *__restrict__ x, sera_producer prod, int M, int Mpad, int K, _Float16 *__restrict__ xh,
        float *__restrict__ d8t) {
    const int row = blockIdx.y;
    const int k = (blockIdx.x * 256 + threadIdx.x) * 4;
    const float4 v = q8_produce4_row<PK>(x, prod, row, M, K, k);
    if (k >= K) return;

    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, xor_partner<4>(amax));
    amax = fmaxf(amax, xor_partner<2>(amax));
    amax = fmaxf(amax, xor_partner<1>(amax));
    float q0 = 0.0f, q1 = 0.0f, q2 = 0.0f, q3 = 0.0f, d = 0.0f;
    if (amax != 0.0f) {
        if (ROW) {
            const float dr = amax / 127.0f;
            q0 = roundf(v.x / dr);
            q1 = roundf(v.y / dr);
            q2 = roundf(v.z / dr);
            q3 = roundf(v.w / dr);
            d = h2f_bits(f2h_bits(dr));
        } else {
            const float d_inv = 127.0f / amax;
            q0 = roundf(v.x * d_inv);
            q1 = roundf(v.y * d_inv);
            q2 = roundf(v.z * d_inv);
            q3 = roundf(v.w * d_inv);
            d = 1.0f / d_inv;
        }
    }
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    /* stored as 16*q: |16q| <= 2032 is exact in fp16 */
    const h4 hq = {(_Float16)(16.0f * q0), (_Float16)(16.0f * q1), (_Float16)(16.0f * q2), (_Float16)(16.0f * q3)};
    *(h4 *)(xh + (size_t)row * K + k) = hq;
    if ((threadIdx.x & 7) == 0)
        d8t[((size_t)(k >> 8) * 8 + ((k >> 5) & 7)) * Mpad + row] = d;
}

#define Q8_DISPATCH_PK(KIND, ...)                                                                         \
    switch (KIND) {                                                                                        \
        case 1: { constexpr int PK = 1; __VA_ARGS__; } break;                                              \
        case 2: { constexpr int PK = 2; __VA_ARGS__; } break;                                              \
        default: { constexpr int PK = 0; __VA_ARGS__; } break;                                             \
    }

/* row_formula = 0: D4 (MMQ) values, 1: row-quantizer (MMVQ) values. */
extern "C" hipError_t sera_launch_q8_1_q6k_stage_p(const float *x, const sera_producer *prod, int M, int Mpad, int K,
                                                   int row_formula, void *stage, hipStream_t stream) {
    const sera_stage_layout L = sera_q6k_mmq_stage_layout((size_t)Mpad, (size_t)K);
    char *base = (char *)stage;
    const sera_producer p = prod ? *prod : sera_producer{0, nullptr, nullptr, 0.0f};
    dim3 grid((K + 1023) / 1024, Mpad);
    Q8_DISPATCH_PK(p.kind,
        if (row_formula)
            hipLaunchKernelGGL((sera_q8_1_q6k_stage_kernel<true, PK>), grid, dim3(256), 0, stream, x, p, M, Mpad, K,
                               (_Float16 *)(base + L.qs), (float *)(base + L.ds));
        else
            hipLaunchKernelGGL((sera_q8_1_q6k_stage_kernel<false, PK>), grid, dim3(256), 0, stream, x, p, M, Mpad,
                               K, (_Float16 *)(base + L.qs), (float *)(base + L.ds)))
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q8_1_row_p(const float *x, const sera_producer *prod, int M, int K, void *stage,
                                             hipStream_t stream) {
    const sera_stage_layout L = sera_row_stage_layout((size_t)M, (size_t)K);
    char *base = (char *)stage;
    const sera_producer p = prod ? *prod : sera_producer{0, nullptr, nullptr, 0.0f};
    dim3 grid(K / 256, M);
    Q8_DISPATCH_PK(p.kind,
        hipLaunchKernelGGL((sera_q8_1_row_kernel<PK>), grid, dim3(256), 0, stream, x, p, K,
                           (int8_t *)(base + L.qs), (uint32_t *)(base + L.ds), (float4 *)(base + L.dsf)))
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q8_1_mmq_p(const float *x, const sera_producer *prod, int M, int Mpad, int K,
                                             void *stage, hipStream_t stream) {
    const sera_stage_layout L = sera_mmq_stage_layout((size_t)Mpad, (size_t)K);
    char *base = (char *)stage;
    const sera_producer p = prod ? *prod : sera_producer{0, nullptr, nullptr, 0.0f};
    dim3 grid((K + 1023) / 1024, Mpad);
    Q8_DISPATCH_PK(p.kind,
        hipLaunchKernelGGL((sera_q8_1_mmq_kernel<PK>), grid, dim3(256), 0, stream, x, p, M, K,
                           (int8_t *)(base + L.qs), (uint32_t *)(base + L.ds)))
    return hipGetLastError();
}

extern "C" hipError_t sera_launch_q8_1_q6k_stage(const float *x, int M, int Mpad, int K, int row_formula,
                                                 void *stage, hipStream_t stream) {
    return sera_launch_q8_1_q6k_stage_p(x, nullptr, M, Mpad, K, row_formula, stage, stream);
}

extern "C" hipError_t sera_launch_q8_1_row(const float *x, int M, int K, void *stage, hipStream_t stream) {
    return sera_launch_q8_1_row_p(x, nullptr, M, K, stage, stream);
}

extern "C" hipError_t sera_launch_q8_1_mmq(const float *x, int M, int Mpad, int K, void *stage,
                                           hipStream_t stream) {
    return sera_launch_q8_1_mmq_p(x, nullptr, M, Mpad, K, stage, stream);
}
