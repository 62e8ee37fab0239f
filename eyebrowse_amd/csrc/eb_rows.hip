// Per-head pre-attention rows for gfx950: the part of Attention::prefill between the
// projections and the attention (crates/eyebrowse-nn/src/attention.rs:62-97: q/k/v
// RMSNorm, RoPE of q and k, kv_write of K and V) as one launch, and RoPE on its own
// (crates/eyebrowse-kernels/src/rope.rs:38-69).
//
// A head row is the HD values of one head of one token. A launch walks up to three
// segments of head rows (q, k, v: [rows, nh, HD] each) and for each row does
//  - RMSNorm with a gain when the segment has one: y = x * (1 / sqrt(sum x^2 / HD + eps)) * w
//    (kernels/src/rmsnorm.rs:6-38, per head: rows * heads rows of HD),
//  - RoPE at table row rope_row0 + token when the segment asks for it: dims p and p + HD/2
//    become (x1 c - x2 s, x2 c + x1 s) with the table's angle p (kernels/src/rope.rs:6-32;
//    pass-through pairs have c = 1, s = 0),
//  - a store into row dst_row0 + token of a [*, nh, HD] destination of f32, IEEE-half or
//    OCP FP8 E4M3 elements (the KV caches at base_pos, or the rotated q).
// The rotation is computed without contraction (two roundings, then the difference), as the
// reference computes it in f32, so RoPE alone is bit-exact against the reference's CPU path.
//
// Lane layout (HD a multiple of 8, up to 256): a head row sits on LPR lanes, LPR the power of
// two at or above HD/8; lane j < HD/8 holds dims 4j..4j+3 and HD/2+4j..HD/2+4j+3, both halves
// of its RoPE pairs, so the rotation needs no lane exchange and every access is one 16-byte
// load or store (8 bytes for half, 4 for E4M3). The row's sum of squares meets over the LPR lanes by DPP
// and lane swaps. Other even head dims (and unaligned buffers) take one wave per head row.
#include "eb_common.h"
#include "eb_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// Sum over aligned groups of N lanes, N a power of two up to 32.
template <int N>
__device__ __forceinline__ float lanes_sum(float x) {
    if constexpr (N <= 16) {
        return eb::group_sum<N>(x);
    } else {
        x = eb::group_sum<16>(x);
        return x + eb::lane_xor16(x);
    }
}

// The segment a head row belongs to, its fields selected (not indexed) so that the kernel
// arguments stay in scalar registers.
struct SegView {
    const float *src;
    void *dst;
    const float *gain;
    int nh, dst_row0, local;
    bool rope;
    int elem;  // bytes per destination element
};

__device__ __forceinline__ SegView seg_of(const eb::RowsArgs &a, int t) {
    const int s = (a.nseg > 2 && t >= a.start[2]) ? 2 : (a.nseg > 1 && t >= a.start[1]) ? 1 : 0;
    auto pick = [s](auto x0, auto x1, auto x2) { return s == 0 ? x0 : s == 1 ? x1 : x2; };
    SegView v;
    v.src = pick(a.seg[0].src, a.seg[1].src, a.seg[2].src);
    v.dst = pick(a.seg[0].dst, a.seg[1].dst, a.seg[2].dst);
    v.gain = pick(a.seg[0].gain, a.seg[1].gain, a.seg[2].gain);
    v.nh = pick(a.seg[0].nh, a.seg[1].nh, a.seg[2].nh);
    v.dst_row0 = pick(a.seg[0].dst_row0, a.seg[1].dst_row0, a.seg[2].dst_row0);
    v.rope = pick(a.seg[0].rope, a.seg[1].rope, a.seg[2].rope);
    v.elem = pick(a.seg[0].elem, a.seg[1].elem, a.seg[2].elem);
    v.local = t - pick(a.start[0], a.start[1], a.start[2]);
    return v;
}

template <int LPR>
__global__ __launch_bounds__(kThreads) void rows_vec_kernel(eb::RowsArgs a) {
#pragma clang fp contract(off)
    constexpr int RPW = 64 / LPR;  // head rows per wave
    const int lane = threadIdx.x & 63;
    const int j = lane % LPR;
    const int t = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * RPW + lane / LPR;
    const int hd = a.hd;
    const int half = hd / 2;
    const bool row_on = t < a.start[a.nseg];
    const bool on = row_on && j < hd / 8;
    const SegView sv = seg_of(a, row_on ? t : 0);
    const int tok = sv.local / sv.nh;
    const int hh = sv.local % sv.nh;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const float *src = sv.src + ((size_t)tok * sv.nh + hh) * hd + 4 * j;
    f32x4 x1 = on ? *reinterpret_cast<const f32x4 *>(src) : z;
    f32x4 x2 = on ? *reinterpret_cast<const f32x4 *>(src + half) : z;
    // Every lane joins the reduction (rows of one group share their segment).
    float ss = (x1.x * x1.x + x1.y * x1.y) + (x1.z * x1.z + x1.w * x1.w) +
               ((x2.x * x2.x + x2.y * x2.y) + (x2.z * x2.z + x2.w * x2.w));
    ss = lanes_sum<LPR>(ss);
    if (!on) return;
    if (sv.gain) {
        const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
        x1 = x1 * inv * *reinterpret_cast<const f32x4 *>(sv.gain + 4 * j);
        x2 = x2 * inv * *reinterpret_cast<const f32x4 *>(sv.gain + half + 4 * j);
    }
    if (sv.rope) {
        const size_t trow = (size_t)(a.rope_row0 + tok) * half + 4 * j;
        const f32x4 c = *reinterpret_cast<const f32x4 *>(a.cosb + trow);
        const f32x4 s = *reinterpret_cast<const f32x4 *>(a.sinb + trow);
        const f32x4 y1 = x1 * c - x2 * s;
        const f32x4 y2 = x2 * c + x1 * s;
        x1 = y1;
        x2 = y2;
    }
    const size_t d = ((size_t)(sv.dst_row0 + tok) * sv.nh + hh) * hd + 4 * j;
    if (sv.elem == 2) {
        _Float16 *p = static_cast<_Float16 *>(sv.dst) + d;
        *reinterpret_cast<f16x4 *>(p) = __builtin_convertvector(x1, f16x4);
        *reinterpret_cast<f16x4 *>(p + half) = __builtin_convertvector(x2, f16x4);
    } else if (sv.elem == 1) {
        uint8_t *p = static_cast<uint8_t *>(sv.dst) + d;
        *reinterpret_cast<unsigned *>(p) = eb::f8x4_bits(x1);
        *reinterpret_cast<unsigned *>(p + half) = eb::f8x4_bits(x2);
    } else {
        float *p = static_cast<float *>(sv.dst) + d;
        *reinterpret_cast<f32x4 *>(p) = x1;
        *reinterpret_cast<f32x4 *>(p + half) = x2;
    }
}

// Any even head dim: one wave per head row, lanes striding its RoPE pairs.
__global__ __launch_bounds__(kThreads) void rows_wave_kernel(eb::RowsArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (t >= a.start[a.nseg]) return;  // (wave-uniform)
    const SegView sv = seg_of(a, t);
    const int hd = a.hd;
    const int half = hd / 2;
    const int tok = sv.local / sv.nh;
    const int hh = sv.local % sv.nh;
    const float *src = sv.src + ((size_t)tok * sv.nh + hh) * hd;
    float inv = 1.0f;
    if (sv.gain) {
        float ss = 0.0f;
        for (int i = lane; i < hd; i += 64) ss += src[i] * src[i];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
    }
    const size_t d = ((size_t)(sv.dst_row0 + tok) * sv.nh + hh) * hd;
    const size_t trow = (size_t)(a.rope_row0 + tok) * half;
    for (int p = lane; p < half; p += 64) {
        float x1 = src[p], x2 = src[p + half];
        if (sv.gain) {
            x1 = x1 * inv * sv.gain[p];
            x2 = x2 * inv * sv.gain[p + half];
        }
        if (sv.rope) {
            const float c = a.cosb[trow + p], s = a.sinb[trow + p];
            const float y1 = x1 * c - x2 * s;
            const float y2 = x2 * c + x1 * s;
            x1 = y1;
            x2 = y2;
        }
        if (sv.elem == 2) {
            _Float16 *o = static_cast<_Float16 *>(sv.dst) + d;
            o[p] = (_Float16)x1;
            o[p + half] = (_Float16)x2;
        } else if (sv.elem == 1) {
            uint8_t *o = static_cast<uint8_t *>(sv.dst) + d;
            o[p] = (uint8_t)eb::f8e4m3_bits(x1);
            o[p + half] = (uint8_t)eb::f8e4m3_bits(x2);
        } else {
            float *o = static_cast<float *>(sv.dst) + d;
            o[p] = x1;
            o[p + half] = x2;
        }
    }
}

bool aligned(const void *p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

}  // namespace

namespace eb {

eb_status launch_attn_rows(hipStream_t st, const RowsArgs &args) {
    RowsArgs a = args;
    a.start[0] = 0;
    for (int s = 0; s < a.nseg; ++s) a.start[s + 1] = a.start[s] + a.rows * a.seg[s].nh;
    for (int s = a.nseg; s < 3; ++s) a.start[s + 1] = a.start[a.nseg];
    const int total = a.start[a.nseg];
    if (total == 0) return EB_OK;
    bool vec = a.hd % 8 == 0 && a.hd <= 256;
    for (int s = 0; s < a.nseg && vec; ++s) {
        const RowSeg &g = a.seg[s];
        vec = aligned(g.src, 16) && aligned(g.dst, 4 * (uintptr_t)g.elem) && aligned(g.gain, 16);
    }
    vec = vec && aligned(a.cosb, 16) && aligned(a.sinb, 16);
    if (!vec) {
        rows_wave_kernel<<<(unsigned)((total + kWaves - 1) / kWaves), kThreads, 0, st>>>(a);
        return check_launch("attention rows");
    }
    int lpr = 1;
    while (lpr < a.hd / 8) lpr *= 2;
    const int per_block = kWaves * (64 / lpr);
    const unsigned grid = (unsigned)((total + per_block - 1) / per_block);
    switch (lpr) {
        case 1: rows_vec_kernel<1><<<grid, kThreads, 0, st>>>(a); break;
        case 2: rows_vec_kernel<2><<<grid, kThreads, 0, st>>>(a); break;
        case 4: rows_vec_kernel<4><<<grid, kThreads, 0, st>>>(a); break;
        case 8: rows_vec_kernel<8><<<grid, kThreads, 0, st>>>(a); break;
        case 16: rows_vec_kernel<16><<<grid, kThreads, 0, st>>>(a); break;
        default: rows_vec_kernel<32><<<grid, kThreads, 0, st>>>(a); break;
    }
    return check_launch("attention rows");
}

eb_status launch_rope(hipStream_t st, const float *x, const float *cosb, const float *sinb,
                      float *out, size_t seq, size_t n_heads, size_t hd, size_t base_pos) {
    RowsArgs a{};
    a.nseg = 1;
    a.seg[0] = RowSeg{x, out, nullptr, (int)n_heads, 0, true, 4};
    a.rows = (int)seq;
    a.hd = (int)hd;
    a.cosb = cosb;
    a.sinb = sinb;
    a.rope_row0 = (int)base_pos;
    return launch_attn_rows(st, a);
}

}  // namespace eb
