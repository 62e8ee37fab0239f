// Greedy sampling for gfx950: the index of the largest logit.
//
// Replaces argmax (crates/eyebrowse-kernels/src/sampling.rs:6-53), one 256-thread
// workgroup in which lane t scans i = t, t+256, ... keeping its first strictly larger
// value (start -3e38), followed by a tree over the lanes that moves the right value left
// only if strictly larger. That order fixes which index wins a tie: the one whose lane
// (i mod 256) comes first in bit-reversed order (two lanes first meet at the stride of
// their lowest differing bit, the lane with that bit clear sitting on the left), then the
// smallest i. NaN and values <= -3e38 never win; with no candidate the result is 0.
//
// Here every element gets a 64-bit key whose order is exactly that choice: the high 32
// bits are the value's bits made monotonic (-0.0 taken as +0.0), the low 32 bits 255 - bitrev8(i mod 256) and
// 2^24 - 1 - i / 256 (so vocab < 2^32); non-candidates get key 0. The maximum key is the
// reference's winner whatever order the keys are reduced in, so the work can be spread
// over many workgroups: pass 1 reduces slices to one key each (workspace), pass 2 reduces
// those and decodes the index. A vocabulary of one slice (up to 4096) is one launch: its
// single workgroup decodes the index itself.
#include "eb_common.h"
#include "eb_internal.h"

#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kPerThread = 16;  // elements per thread per workgroup (4 x 16-byte loads)
constexpr int kSlice = kThreads * kPerThread;

__device__ __forceinline__ uint64_t key_of(float v, uint32_t i) {
    if (!(v > -3.0e38f)) return 0;  // NaN and values the reference's start never beats
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    // -0.0 and +0.0 compare equal under the reference's strict `>`, so they tie: both
    // take +0.0's key, and the tie order below decides between them.
    if ((u & 0x7FFFFFFFu) == 0) u = 0;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t lane_rank = 255u - (__builtin_bitreverse32(i & 255u) >> 24);
    const uint32_t tb = (lane_rank << 24) | (0xFFFFFFu - (i >> 8));
    return ((uint64_t)u << 32) | tb;
}

__device__ __forceinline__ uint32_t index_of(uint64_t key) {
    if (key == 0) return 0;
    const uint32_t tb = (uint32_t)key;
    const uint32_t lane = __builtin_bitreverse32(255u - (tb >> 24)) >> 24;
    return (0xFFFFFFu - (tb & 0xFFFFFFu)) * 256u + lane;
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The key of another lane: both 32-bit halves through the same exchange.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t k) {
    const unsigned lo = (unsigned)k, hi = (unsigned)(k >> 32);
    const unsigned lo2 = __builtin_bit_cast(unsigned, eb::dpp<CTRL>(__builtin_bit_cast(float, lo)));
    const unsigned hi2 = __builtin_bit_cast(unsigned, eb::dpp<CTRL>(__builtin_bit_cast(float, hi)));
    return ((uint64_t)hi2 << 32) | lo2;
}
__device__ __forceinline__ uint64_t xor64(uint64_t k, int mask) {
    const unsigned lo = __shfl_xor((unsigned)k, mask), hi = __shfl_xor((unsigned)(k >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

// Workgroup maximum of one key per thread: within each wave by lane exchanges (the row's
// 16 lanes by DPP, then across rows), the waves' maxima through LDS with one barrier. The
// maximum key does not depend on the order it is taken in.
__device__ __forceinline__ uint64_t block_max(uint64_t k) {
    __shared__ uint64_t s[kThreads / 64];
    k = umax64(k, dpp64<eb::kDppQuadXor1>(k));
    k = umax64(k, dpp64<eb::kDppQuadXor2>(k));
    k = umax64(k, dpp64<eb::kDppRowHalfMirror>(k));
    k = umax64(k, dpp64<eb::kDppRowMirror>(k));
    k = umax64(k, xor64(k, 16));
    k = umax64(k, xor64(k, 32));
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = k;
    __syncthreads();
    uint64_t r = s[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = umax64(r, s[w]);
    return r;
}

// Pass 1: workgroup b reduces elements [b*kSlice, (b+1)*kSlice) to one key (with one
// workgroup, the winner's index goes straight to out).
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const float *__restrict__ x,
                                                                  uint32_t n, bool vec,
                                                                  uint64_t *__restrict__ part,
                                                                  uint32_t *__restrict__ out) {
    const uint32_t base = blockIdx.x * (uint32_t)kSlice;
    uint64_t best = 0;
    if (vec) {  // x 16-byte aligned, n % 4 == 0: 4 loads of 4 per thread, issued first
        f32x4 v[kPerThread / 4];
        uint32_t at[kPerThread / 4];
#pragma unroll
        for (int j = 0; j < kPerThread / 4; ++j) {
            at[j] = base + 4u * (threadIdx.x + j * kThreads);
            v[j] = *reinterpret_cast<const f32x4 *>(x + (at[j] < n ? at[j] : 0));
        }
#pragma unroll
        for (int j = 0; j < kPerThread / 4; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (at[j] < n) best = umax64(best, key_of(v[j][c], at[j] + c));
    } else {
        for (int j = 0; j < kPerThread; ++j) {
            const uint32_t i = base + threadIdx.x + j * kThreads;
            if (i < n) best = umax64(best, key_of(x[i], i));
        }
    }
    best = block_max(best);
    if (threadIdx.x == 0) {
        if (gridDim.x == 1)
            out[0] = index_of(best);
        else
            part[blockIdx.x] = best;
    }
}

// Pass 2: one workgroup reduces the partial keys and writes the index.
__global__ __launch_bounds__(kThreads) void argmax_final_kernel(const uint64_t *__restrict__ part,
                                                                int nparts,
                                                                uint32_t *__restrict__ out) {
    uint64_t best = 0;
    for (int i = threadIdx.x; i < nparts; i += kThreads) best = umax64(best, part[i]);
    best = block_max(best);
    if (threadIdx.x == 0) out[0] = index_of(best);
}

}  // namespace

namespace eb {

size_t argmax_workspace_floats(size_t n) {
    const size_t parts = (n + kSlice - 1) / kSlice;
    return 2 * (parts > 0 ? parts : 1);  // one u64 per part
}

eb_status launch_argmax(hipStream_t st, const float *x, size_t n, uint32_t *out, float *ws,
                        size_t ws_floats) {
    const size_t parts = (n + kSlice - 1) / kSlice;
    if (n >= ((size_t)1 << 31)) return fail(EB_UNSUPPORTED_CONFIG, "argmax: vocab %zu too large", n);
    if (!ws || (reinterpret_cast<uintptr_t>(ws) & 7) != 0 || ws_floats < argmax_workspace_floats(n))
        return fail(EB_SHAPE_MISMATCH, "argmax: workspace too small or not 8-byte aligned");
    uint64_t *part = reinterpret_cast<uint64_t *>(ws);
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && n % 4 == 0 && n >= 4;
    const unsigned blocks = (unsigned)(parts > 0 ? parts : 1);
    argmax_partial_kernel<<<blocks, kThreads, 0, st>>>(x, (uint32_t)n, vec, part, out);
    if (blocks > 1) argmax_final_kernel<<<1, kThreads, 0, st>>>(part, (int)blocks, out);
    return check_launch("argmax");
}

}  // namespace eb
