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

// The value held by lane i ^ 16 (v_permlane16_swap exchanges the odd 16-lane rows of one
// operand with the even rows of the other; with both operands x, the first result holds
// the lower neighbour's row on odd rows, the second the upper neighbour's on even rows).
__device__ __forceinline__ float lane_xor16(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    unsigned r1 = r[1];
    asm volatile("" : "+v"(r1));  // keep the two results distinct (see swap_sum32)
    const bool odd_row = (__lane_id() >> 4) & 1;
    return __builtin_bit_cast(float, odd_row ? r[0] : r1);
}

// The value held by lane i ^ 32 (v_permlane32_swap exchanges the wave's two halves).
__device__ __forceinline__ float lane_xor32(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    unsigned r1 = r[1];
    asm volatile("" : "+v"(r1));  // keep the two results distinct (see swap_sum32)
    const bool upper = __lane_id() >= 32;
    return __builtin_bit_cast(float, upper ? r[0] : r1);
}

// Reduce-scatter halves with the swaps: a + b over lane pairs i, i ^ 32 (swap_sum32) or
// i, i ^ 16 (swap_sum16), where lanes 0-31 (even 16-lane rows) end with the pair's sum of
// a and lanes 32-63 (odd rows) with the pair's sum of b. The empty asm keeps the second
// result opaque: the ROCm 7.2 compiler folds the f32 add of a swap's two results into
// an add of the first result to itself.
__device__ __forceinline__ float swap_sum32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, b), false, false);
    unsigned r1 = r[1];
    asm volatile("" : "+v"(r1));
    return __builtin_bit_cast(float, r[0]) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a),
                                                    __builtin_bit_cast(unsigned, b), false, false);
    unsigned r1 = r[1];
    asm volatile("" : "+v"(r1));
    return __builtin_bit_cast(float, r[0]) + __builtin_bit_cast(float, r1);
}

// Reduce (sum or max) over the lanes that share lane bits [0, log2(FROM)): every lane
// ends with the reduction over its class {i' : i' % FROM == i % FROM}. VALU lane
// permutes only (DPP row rotations within 16 lanes, then the 16- and 32-lane swaps): a
// rotation by 8 within a row pairs lane i with i ^ 8, and the rotations by 1, 2, 4 fold
// a class's members within a row in any order, which a sum or max does not notice.
template <int FROM, bool MAX>
__device__ __forceinline__ float row_class_reduce(float x) {
    static_assert(FROM == 1 || FROM == 2 || FROM == 4 || FROM == 8 || FROM == 16 ||
                      FROM == 32 || FROM == 64, "power of two");
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    if constexpr (FROM <= 1) x = op(x, dpp<0x121>(x));  // row_ror:1
    if constexpr (FROM <= 2) x = op(x, dpp<0x122>(x));  // row_ror:2
    if constexpr (FROM <= 4) x = op(x, dpp<0x124>(x));  // row_ror:4
    if constexpr (FROM <= 8) x = op(x, dpp<0x128>(x));  // row_ror:8
    return x;
}

template <int FROM, bool MAX>
__device__ __forceinline__ float class_reduce(float x) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    x = row_class_reduce<FROM, MAX>(x);  // the members within each 16-lane row
    if constexpr (FROM <= 16) x = op(x, lane_xor16(x));
    if constexpr (FROM <= 32) x = op(x, lane_xor32(x));
    return x;
}

// 2^x on the hardware transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- OCP FP8 E4M3 ("e4m3fn": sign, 4 exponent bits with bias 7, 3 fraction bits, no
// infinities, S.1111.111 NaN, largest finite 448) -------------------------------------

// The E4M3 pattern (low 8 bits) of x: the nearest value, ties to the even fraction; finite
// values at or beyond 448 saturate to +-448; inf and NaN become NaN (0x7F with the sign).
// From the f32 fields: below 2^-6 the value is a count of 2^-9 steps (x * 512 rounded to
// nearest even, exact scaling; a count of 8 is the smallest normal 2^-6); above, the f32
// fraction is rounded to 3 bits (adding 2^19 - 1 plus the kept lowest bit, a carry
// moving the exponent) and the exponent rebased from 127 to 7.
__device__ __forceinline__ unsigned f8e4m3_bits(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const unsigned s = (u >> 24) & 0x80u;
    const unsigned a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return s | 0x7Fu;  // inf, NaN
    if (a >= 0x43E00000u) return s | 0x7Eu;  // 448 and beyond
    if (a < 0x3C800000u)                      // below 2^-6
        return s | (unsigned)__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
    return s | ((((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20)) - (120u << 3));
}

// Four E4M3 values (bytes 0..3 of w, lowest first) as f32, exact (v_cvt_pk_f32_fp8, which
// reads the OCP E4M3 format on gfx950).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4_t f8x4_to_f32(unsigned w) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    return f32x4_t{lo[0], lo[1], hi[0], hi[1]};
}

// Four f32 values as E4M3 bytes of one word (lowest first).
__device__ __forceinline__ unsigned f8x4_bits(f32x4_t x) {
    return f8e4m3_bits(x[0]) | (f8e4m3_bits(x[1]) << 8) | (f8e4m3_bits(x[2]) << 16) |
           (f8e4m3_bits(x[3]) << 24);
}

// Raw buffer resource over [p, p + nbytes) (gfx9 raw buffer: 32-bit data, range checked:
// a load at or past nbytes reads zeros without touching memory). The operands are made
// wave-uniform explicitly so that the descriptor lives in scalar registers (a per-lane
// descriptor costs a loop per load); p and nbytes must be the same in every lane.
constexpr int kRawBufferFlags = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, int nbytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(p);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    void *u = reinterpret_cast<void *>(((unsigned long long)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, __builtin_amdgcn_readfirstlane(nbytes),
                                             kRawBufferFlags);
}

}  // namespace eb
