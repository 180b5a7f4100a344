/*
 * q6k_layout.hip - Q6_K weights from GGUF bytes to the split device layout.
 *
 * The reference's loader copies each GGUF tensor verbatim into one device
 * allocation through pinned staging buffers
 * (cuda/q3_model_loader_cuda.cu:232-261,290-342). A GGUF Q6_K block is 210
 * bytes (ql[128], qh[64], sc[16], fp16 d; src/q3_quant.c:78-103), so blocks
 * and rows sit at 2-byte alignment and no lane can fetch its fields with
 * aligned 16-byte loads. The split layout (q4k_common.h) keeps the same
 * bytes but moves every block's d into an array after the blocks, so each
 * block's remaining 208 bytes start on a 16-byte boundary.
 *
 * The repack runs on the device once the GGUF bytes have landed: thread
 * (block b, chunk c) reads chunk c of block b as eight 2-byte loads (the
 * source is 2-byte aligned) and writes it with one 16-byte store; chunk 13
 * writes d. Memory-bound, one pass.
 */
#include "sera_launch.h"

/* src: GGUF blocks [first, first + count) of a matrix of `total` blocks,
 * back to back; dst: the whole matrix in the split layout. */
__global__ __launch_bounds__(256) void sera_q6k_split_kernel(const uint16_t *__restrict__ src,
                                                             uint8_t *__restrict__ dst, uint64_t first,
                                                             uint64_t count, uint64_t total) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t b = i / 14;
    const int c = (int)(i - b * 14);
    if (b >= count) return;
    const uint16_t *s = src + b * (Q6K_GGUF_BYTES / 2);
    if (c < 13) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = (uint32_t)s[8 * c + 2 * k] | ((uint32_t)s[8 * c + 2 * k + 1] << 16);
        *(uint4 *)(dst + (first + b) * Q6K_SPLIT_QBYTES + 16 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        ((uint16_t *)(dst + total * Q6K_SPLIT_QBYTES))[first + b] = s[Q6K_SPLIT_QBYTES / 2];
    }
}

extern "C" hipError_t sera_launch_q6k_split(const void *src, void *dst, uint64_t first, uint64_t count,
                                            uint64_t total, hipStream_t s) {
    if (count == 0) return hipSuccess;
    const uint64_t threads = count * 14;
    hipLaunchKernelGGL(sera_q6k_split_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       (const uint16_t *)src, (uint8_t *)dst, first, count, total);
    return hipGetLastError();
}
