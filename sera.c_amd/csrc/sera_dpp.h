/*
 * sera_dpp.h - cross-lane helpers for wave64 kernels on gfx950 (device code
 * only).
 */
#ifndef SERA_DPP_H
#define SERA_DPP_H

#include <hip/hip_runtime.h>

/* The value of lane (lane ^ OFF) for xor butterflies, in VALU cross-lane
 * operations instead of LDS permutes: DPP inside a 16-lane row
 * (quad_perm for 1 and 2, row_ror:8 for 8, and for 4 two row shifts, each
 * written only to the banks of four lanes whose partner it reaches), and for
 * 16 and 32 the gfx950 row and half swaps (v_permlane16_swap /
 * v_permlane32_swap: with both operands the same value, one result holds the
 * partner where the lane's row (half) is odd, the other where it is even). */
template <int OFF>
__device__ __forceinline__ int xor_partner(int v) {
    if constexpr (OFF == 1) {
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);     /* quad_perm [1,0,3,2] */
    } else if constexpr (OFF == 2) {
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);     /* quad_perm [2,3,0,1] */
    } else if constexpr (OFF == 4) {
        const int p = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0x5, false);   /* row_shl:4, banks 0, 2 */
        return __builtin_amdgcn_update_dpp(p, v, 0x114, 0xF, 0xA, false);          /* row_shr:4, banks 1, 3 */
    } else if constexpr (OFF == 8) {
        return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);    /* row_ror:8 */
    } else if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (threadIdx.x & 16) ? (int)r[0] : (int)r[1];
    } else {
        static_assert(OFF == 32, "xor partner offset");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? (int)r[0] : (int)r[1];
    }
}

template <int OFF>
__device__ __forceinline__ float xor_partner(float v) { return __int_as_float(xor_partner<OFF>(__float_as_int(v))); }

#endif
