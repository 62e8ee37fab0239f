// Device-side helpers shared by the gfx950 kernels: wave64 lane exchanges and exp2.
#pragma once

#include <hip/hip_runtime.h>

namespace eb {

constexpr float kLog2e = 1.4426950408889634f;

// DPP lane exchange within a 16-lane row (CDNA DPP control codes).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i within each 16 lanes

// Sum over aligned groups of N consecutive lanes (N in 1, 2, 4, 8, 16); every lane of a
// group ends with the group's total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group of 1..16 lanes");
    if constexpr (N >= 2) x += dpp<kDppQuadXor1>(x);
    if constexpr (N >= 4) x += dpp<kDppQuadXor2>(x);
    if constexpr (N >= 8) x += dpp<kDppRowHalfMirror>(x);
    if constexpr (N >= 16) x += dpp<kDppRowMirror>(x);
    return x;
}

// 2^x on the hardware transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace eb
