// Batch-1 decode attention for gfx950: split-KV ("flash-decoding") over the seq-major
// cache [max_seq, Hkv, HD], then a log-sum-exp merge.
//
// Replaces attn_decode (crates/eyebrowse-kernels/src/attention.rs:52-90,124-162), which
// runs one thread per query head and streams the whole cache serially, and optionally
// folds in the two kv_write calls that precede it in Attention::decode
// (crates/eyebrowse-nn/src/attention.rs:149-183).
//
// Pass 1, grid (Hkv * nsub) x nsplit, 256 threads per workgroup. Workgroup (col, split)
// reduces a 1/nsplit share of the keys for KV head col % Hkv and the G query heads that
// share it (GQA: every K/V row is read once for all of them):
//  - a key row of HD elements (f32, IEEE half or OCP FP8 E4M3, converted to f32 as loaded)
//    is spread over LPK = HD/DPL lanes (DPL = 16 dims per lane; 8 for f32 head_dim 128
//    with 4 query heads per workgroup),
//    so a wave covers KPW = 64/LPK keys per step; the keys are dealt to the splits in
//    superblocks of one step of every wave, kWaves * KPW rows (split s owns superblocks
//    s, s + nsplit, ...; the E4M3 matrix-core kernel deals tiles of KPW rows), so that
//    all workgroups together stream one contiguous stretch of the cache at a time;
//  - loads are 128-bit raw buffer loads (64-bit over E4M3 caches, so that a lane holds the
//    same dims as over f16 ones) whose range check turns rows past the end into
//    zeros (no clamping, no branches); two register buffers per wave keep the next
//    iteration's loads in flight while the current one is consumed;
//  - scores are lane-partial dot products summed across the LPK lanes with DPP;
//  - each lane group keeps an online softmax (running max m, sum l, acc[DPL]) in the log2
//    domain (scores times scale*log2(e), exponentials on v_exp_f32), with the rescale of
//    l and acc skipped until a score exceeds the running max by a slack;
//  - the lane groups' states meet in LDS, where the workgroup combines them per head;
//  - with one split the workgroup writes o directly; otherwise it writes its partial
//    (m, l, acc[HD]) per head and pass 2 (decode_merge_kernel) computes
//    o = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M). A second launch is cheaper here
//    than merging in the last-arriving workgroup: on the 8-XCD part that needs an L2
//    write-back fence in every workgroup.
// Fused new-token write: when knew/vnew are given, rows 0..pos-1 come from the cache and
// key `pos` from knew/vnew, folded in after the loop by the split that owns its rows;
// that split's first head-subgroup workgroup also copies knew/vnew into cache row `pos`.
// Nothing else touches that row in the launch, so the copy is exact and race free.
//
// E4M3 caches at head dims 64, 128 and 256 run decode_mx_kernel instead (below): the same
// grid, split plan, partials and merge, with both products on the matrix cores.
//
// The result is softmax(scale * q K^T) V over keys 0..=pos; it differs from the
// reference's 3-pass f32 softmax only by rounding (summation order, exp2 vs expf).
#include "eb_common.h"
#include "eb_internal.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

// Wave steps per iteration (and per softmax update); a positive EB_DECODE_U overrides
// the default of one.
#ifndef EB_DECODE_U
#define EB_DECODE_U 0
#endif
// Wave steps per iteration over IEEE-half caches. Two would keep the bytes in flight of
// one f32 step, but measured slower than one at Mistral 32k keys (26.0 -> 27.3 us per
// step): per byte the f16 kernel does twice the f32 arithmetic (v_fma_mix per dim and
// head), which then dominates.
#ifndef EB_DECODE_U16
#define EB_DECODE_U16 1
#endif
// Dims per lane of the head_dim 128 IEEE-half kernel with 4 heads (16 or 8). 8 frees half
// of the q and accumulator registers but doubles the lanes a score sums over; measured at
// Mistral 32k keys (us per step): 16: 26.0; 8 with 1, 2, 3 wave steps per iteration: 35.1,
// 27.4, 26.8 (27.3 and 28.8 at two workgroups per CU).
#ifndef EB_DECODE_DPL16
#define EB_DECODE_DPL16 16
#endif
// Wave steps per iteration over E4M3 caches (a wave step's loads hold half the bytes of
// an f16 one). Measured at Mistral 32k keys: 1: 28.8 us, 2: 25.3 us, 4: 25.6 us per step.
#ifndef EB_DECODE_U8
#define EB_DECODE_U8 2
#endif
// Workgroups per CU the register allocation must allow (launch-bounds minimum); 0 picks
// 2 when at most 2 query heads share a workgroup (then everything fits 256 VGPRs), else 1.
#ifndef EB_DECODE_MINB
#define EB_DECODE_MINB 0
#endif

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplits = 256;  // per column
constexpr float kSlack = 8.0f;  // log2-units a score may exceed the reference max by

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int HD, int G, int UDEF = 1, int DPLDEF = 16>
struct DecodeShape {
    static constexpr int DPL = HD >= DPLDEF ? DPLDEF : HD;  // dims per lane
    static constexpr int LPK = HD / DPL;            // lanes holding a key row's dims
    // Lanes per row group: LPK rounded up to a power of two (head dims 48, 80, 96, ...: the
    // extra lanes hold zeros), so that a row's lanes meet by DPP and lane swaps.
    static constexpr int LPK2 = LPK <= 1 ? 1 : LPK <= 2 ? 2 : LPK <= 4 ? 4 : LPK <= 8 ? 8 : 16;
    static constexpr int KPW = 64 / LPK2;           // keys per wave step
    static constexpr int NV4 = DPL / 4;             // 16-byte loads per lane per row
    // Wave steps per iteration: each of the two register buffers holds U*NV4*2 16-byte
    // loads per lane (half that over f16 caches). One f32 step per buffer keeps everything
    // in VGPRs; with the workgroups of a CU that is as much in flight as the HBM rewards.
    static constexpr int U = EB_DECODE_U > 0 ? EB_DECODE_U : UDEF;
    static constexpr int KEYS_PER_ITER = kWaves * KPW * U;
    // Epilogue LDS: one state per wave, WS floats (G heads of HD, padded by 4 floats so
    // that the waves' rows start in different banks), plus m and l per head and wave.
    static constexpr int WS = G * HD + 4;
    static constexpr size_t LDS_BYTES = sizeof(float) * ((size_t)kWaves * WS + 2 * G * kWaves);
    static_assert(DPL % 4 == 0 && HD % DPL == 0 && LPK <= 16,
                  "head_dim: 4, a multiple of 8 up to 128, or a multiple of 16 up to 256");
};

// Bytes per load over a cache of EB-byte elements: 16 (4 f32 or 8 f16 dims), 8 for E4M3
// (8 dims), so that a lane's loads hold the same dims over f16 and E4M3 caches.
template <int EB>
constexpr int load_bytes() { return EB == 1 ? 8 : 16; }

// Byte offset (within a row) of load number j of dim slice `ls` (LPK lanes per row).
template <int LPK, int EB>
__device__ __forceinline__ int dim_byte(int j, int ls) {
    return (j * LPK + ls) * load_bytes<EB>();
}

// First dim of the lane's f32x4 unit i (4 dims): a load holds 4 dims of an f32 cache row
// and 8 of an f16 or E4M3 one, so unit i of a narrow lane is half of load i/2.
template <int LPK, int EB>
__device__ __forceinline__ int dim_of(int i, int ls) {
    if constexpr (EB < 4)
        return (i / 2 * LPK + ls) * 8 + (i % 2) * 4;
    else
        return dim_byte<LPK, EB>(i, ls) / 4;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// A lane's raw load of one row: 16 bytes, 8 for E4M3 caches.
template <int EB>
using RawLoad = std::conditional_t<EB == 1, u32x2, f32x4>;

// Unit i (4 dims, as f32) of a lane's raw loads of one row.
template <int EB>
__device__ __forceinline__ f32x4 unit_f32(const RawLoad<EB> *raw, int i) {
    if constexpr (EB == 2) {
        const f16x8 h = __builtin_bit_cast(f16x8, raw[i / 2]);
        return (i % 2) ? f32x4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]}
                       : f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    } else if constexpr (EB == 1) {
        return eb::f8x4_to_f32(raw[i / 2][i % 2]);
    } else {
        return raw[i];
    }
}

// The value a cache of EB-byte elements holds for x: f32 -> IEEE half -> f32 (nearest
// even), or f32 -> E4M3 -> f32 (nearest even, saturating).
template <int EB>
__device__ __forceinline__ f32x4 through_cache(f32x4 x) {
    if constexpr (EB == 2)
        return __builtin_convertvector(__builtin_convertvector(x, f16x4), f32x4);
    else if constexpr (EB == 1)
        return eb::f8x4_to_f32(eb::f8x4_bits(x));
    else
        return x;
}

// Stores 4 dims (f32) of a cache row at element offset off, in the cache's element type.
template <int EB>
__device__ __forceinline__ void store_cache4(void *base, size_t off, f32x4 x) {
    if constexpr (EB == 2)
        *reinterpret_cast<f16x4 *>(static_cast<_Float16 *>(base) + off) =
            __builtin_convertvector(x, f16x4);
    else if constexpr (EB == 1)
        *reinterpret_cast<unsigned *>(static_cast<uint8_t *>(base) + off) = eb::f8x4_bits(x);
    else
        *reinterpret_cast<f32x4 *>(static_cast<float *>(base) + off) = x;
}

using eb::make_rsrc;

// Cache policy of the K/V stream's loads: non-temporal (nt). Each cache row is read once
// per step and the step's bytes exceed the L2s and the Infinity Cache, so keeping them only
// evicts lines for nothing. Measured against the default policy, A/B on one box (GB/s per
// step): Mistral 32k keys 5705 -> 6143, Gemma-4 16k 5656 -> 6160, Qwen L=8191 4045 ->
// 4419, Qwen L=2048 1947 -> 2034, the half cache at Mistral 32k keys 27.7 -> 26.6 us; sc0
// or sc1 alone: no change; either with nt: as nt alone.
constexpr int kStreamPolicy = 2;  // gfx950 cache-policy bits: 1 sc0, 2 nt, 16 sc1

__device__ __forceinline__ f32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int voffset,
                                               int soffset = 0) {
    return __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, kStreamPolicy));
}

// One raw load of a row slice: 16 bytes, or 8 over E4M3 caches.
template <int EB>
__device__ __forceinline__ RawLoad<EB> buffer_load_row(__amdgpu_buffer_rsrc_t r, int voffset,
                                                       int soffset) {
    if constexpr (EB == 1)
        return __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, kStreamPolicy));
    else
        return buffer_load16(r, voffset, soffset);
}

struct DecodeArgs {
    const float *q;
    const void *kc;    // cache rows read (and row `pos` written when knew != null),
    const void *vc;    // f32 or IEEE half elements
    void *kc_w;        // same as kc, writable
    void *vc_w;
    const float *knew; // [Hkv, HD] new token K (or null)
    const float *vnew;
    float *o;
    float *part_acc;   // [nsplit, h, HD]
    float *part_ml;    // [nsplit, h, 2]
    int h, hkv, g, keys, nsplit;
    float scale_log2;
    // Optional prologue (the step of Attention::decode between the projections and the
    // attention, attention.rs:133-168): per-head RMSNorm of q / knew / vnew with these
    // gains (null: no norm), then RoPE of q and knew at table row rope_row (null tables:
    // no RoPE). With it, the new row is written from the processed knew / vnew.
    bool prologue;
    const float *qn_w, *kn_w, *vn_w;
    float eps;
    const float *rcos, *rsin;  // [max_seq, HD/2]
    int rope_row;
};

// RMSNorm of one head held in a lane group's units (attention.rs:62-73 via
// kernels/src/rmsnorm.rs:6-38): y = x * (1/sqrt(sum x^2 / HD + eps)) * w.
// LPK lanes hold the row's dims, LPK2 (a power of two) lanes form its group; lanes
// ls >= LPK hold zeros and keep them.
template <int HD, int EB, int NV4, int LPK, int LPK2>
__device__ __forceinline__ void norm_units(f32x4 (&u)[NV4], const float *__restrict__ w,
                                           float eps, int ls) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV4; ++i) ss += (u[i].x * u[i].x + u[i].y * u[i].y) +
                                       (u[i].z * u[i].z + u[i].w * u[i].w);
    ss = eb::group_sum<LPK2>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
    if (LPK == LPK2 || ls < LPK) {
#pragma unroll
        for (int i = 0; i < NV4; ++i)
            u[i] = u[i] * inv * *reinterpret_cast<const f32x4 *>(w + dim_of<LPK, EB>(i, ls));
    }
}

// RoPE of one head (kernels/src/rope.rs:6-32): dims p and p + HD/2 rotate by the table
// row's angle p. In the lane layout, unit i + NV4/2 holds the partners of unit i's dims
// (both cache layouts), so each lane rotates its own units.
template <int HD, int EB, int NV4, int LPK>
__device__ __forceinline__ void rope_units(f32x4 (&u)[NV4], const float *__restrict__ cs,
                                           const float *__restrict__ sn, int ls) {
    if constexpr (NV4 == 1) {  // HD 4: pairs (0, 2) and (1, 3) inside the unit
        const float c0 = cs[0], c1 = cs[1], s0 = sn[0], s1 = sn[1];
        const f32x4 x = u[0];
        u[0] = f32x4{x.x * c0 - x.z * s0, x.y * c1 - x.w * s1, x.z * c0 + x.x * s0,
                     x.w * c1 + x.y * s1};
    } else {
#pragma unroll
        for (int i = 0; i < NV4 / 2; ++i) {
            const int d = dim_of<LPK, EB>(i, ls);
            const f32x4 c = *reinterpret_cast<const f32x4 *>(cs + d);
            const f32x4 sv = *reinterpret_cast<const f32x4 *>(sn + d);
            const f32x4 x1 = u[i], x2 = u[i + NV4 / 2];
            u[i] = x1 * c - x2 * sv;
            u[i + NV4 / 2] = x2 * c + x1 * sv;
        }
    }
}

// Two wave steps per iteration for f32 head_dim 256 (4 rows per wave step there): measured
// +4 % at 16k keys; head_dim 128 measured slower with two (its query heads per workgroup
// then fill the register file).
// f32 head_dim 128 with 4 query heads per workgroup (GQA 4, Mistral) runs 8 dims per lane
// (a row over 16 lanes, 4 rows per wave step): at 16 dims per lane the q fragments and
// accumulators of 4 heads leave the two load buffers no registers (256 VGPRs and spills);
// at 8 they take half (160 VGPRs, none spilled). Measured at 32k keys: 5.48 -> 5.77 TB/s;
// more wave steps per iteration on the freed registers measured slower (2: 5.40, 3: 5.35,
// 4: 5.26 TB/s). 2 heads per workgroup (Qwen) measured slower at 8 dims per lane with
// the default cache policy and faster with the non-temporal loads (L=8191 4.43 -> 4.52
// TB/s, 2048 keys +1 %), so head_dim 128 f32 runs 8 dims per lane from 2 heads up.
// Head dims that are odd multiples of 8 (24, 40, ..., 120) run 8 dims per lane for every
// cache type: a row over hd / 8 lanes, padded to a power-of-two group.
// SHORT (f32 head_dim 256 only, chosen by the planner for caches of at most kShortKeys
// keys): one wave step per iteration instead of two. A/B on one box, two rounds, us per
// step at Gemma-4 width, two against one: 1024 keys 8.46 -> 7.60, 2048 9.92 -> 9.83, 4096
// 14.47 -> 14.33, 8192 23.89 -> 24.02, 16384 43.11 -> 43.31 (the local layers' windows of
// Gemma-4 are 1024 keys).
template <int HD, int G, int EB, bool SHORT = false>
using DecodeShapeOf = DecodeShape<HD, G,
                                  EB == 2 ? EB_DECODE_U16 : EB == 1 ? EB_DECODE_U8
                                                                    : (HD == 256 && !SHORT ? 2 : 1),
                                  ((EB == 4 && HD == 128 && G >= 2) || HD % 16 == 8 ||
                                   (EB == 2 && HD == 128 && G >= 4 && EB_DECODE_DPL16 == 8))
                                      ? 8
                                      : 16>;

// Whether the online-softmax update is written once per branch of the wave-uniform rescale
// test. With one copy after the branch, the compiler gives the rescaled accumulators of the
// half-cache kernels with 4 heads new registers and copies them all on the common path
// that skips the rescale (head_dim 128: 485 VALU instructions per loop pass, 82 of them
// copies); with a copy in each branch the pass is 422 instructions, and a Mistral step at
// 32k keys measured 26.9 -> 26.1 us (A/B on one box, two rounds each; head_dim 72 and up;
// the smaller head dims and the other kernels keep their accumulators in place already,
// and a second copy of the update costs them registers and instructions: E4M3 with 4
// heads spills 34 registers to AGPRs).
template <int HD, int EB, int G>
constexpr bool kUpdatePerBranch = EB == 2 && G == 4 && HD >= 72;

// EB: bytes per cache element: 4 (f32), 2 (IEEE half) or 1 (OCP FP8 E4M3), converted to f32
// as loaded. A narrow lane's loads hold 8 dims each (16 bytes of halves, 8 of E4M3), in the
// same dim layout for both.
template <int HD, int G, int EB, bool SHORT = false>
__global__ __launch_bounds__(kThreads, (EB_DECODE_MINB > 0 ? EB_DECODE_MINB : (G <= 2 ? 2 : 1))) void decode_kernel(DecodeArgs a) {
    using S = DecodeShapeOf<HD, G, EB, SHORT>;
    using Raw = RawLoad<EB>;
    constexpr int U = S::U;
    constexpr int NV4 = S::NV4;
    constexpr int LB = load_bytes<EB>();
    constexpr int NL = EB < 4 ? NV4 / 2 : NV4;  // loads per lane per row
    static_assert(EB == 4 || NV4 % 2 == 0, "f16 and e4m3 caches need head_dim >= 8");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // Column col = sub * hkv + kvh: workgroup ids that differ by a multiple of hkv share a
    // KV head, so with hkv a multiple of the 8 XCDs (ids dealt round robin) every column and
    // split of one KV head lands on the same XCD, and the head subgroups that read the same
    // rows share that XCD's L2.
    const int col = blockIdx.x;
    const int kvh = col % a.hkv;
    const int sub = col / a.hkv;
    const int head0 = kvh * a.g + sub * G;
    const int split = blockIdx.y;
    const int kg = lane / S::LPK2;
    const int ls = lane % S::LPK2;
    const bool dims_on = S::LPK == S::LPK2 || ls < S::LPK;  // lane holds dims of its row
    const int pos = a.keys - 1;
    // Keys are dealt to the splits in superblocks of kWaves * KPW rows (one step of every
    // wave of the workgroup): split s owns superblocks s, s + nsplit, s + 2*nsplit, ...
    // At any moment the workgroups of all splits and KV heads together stream one
    // contiguous stretch of the cache, which the HBM serves faster than nsplit separate
    // chunks, and every split gets the same share; within a superblock wave w takes block
    // w, so a workgroup's wave steps read adjacent rows. (Blocks of one wave step dealt
    // round the splits measured 0.4 % slower at 16k-32k keys, A/B on one box, f32 and
    // half caches.) With a new token, rows [0, pos) come from the cache and key `pos`
    // from knew/vnew, folded in by the split that owns its superblock.
    const int ce = a.knew != nullptr ? pos : a.keys;
    const bool tail_new = a.knew != nullptr && split == (pos / S::KPW / kWaves) % a.nsplit;
    const int nsb = (ce + S::KPW * kWaves - 1) / (S::KPW * kWaves);
    const int my_blk = kWaves * (nsb > split ? (nsb - split + a.nsplit - 1) / a.nsplit : 0);
    const int row_bytes = a.hkv * HD * EB;

    f32x4 qr[G][NV4];
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < NV4; ++i)
            qr[gi][i] = dims_on ? *reinterpret_cast<const f32x4 *>(
                                      a.q + (size_t)(head0 + gi) * HD + dim_of<S::LPK, EB>(i, ls))
                                : f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    if (a.prologue) {
        const float *cs = a.rcos ? a.rcos + (size_t)a.rope_row * (HD / 2) : nullptr;
        const float *sn = a.rsin ? a.rsin + (size_t)a.rope_row * (HD / 2) : nullptr;
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            if (a.qn_w) norm_units<HD, EB, NV4, S::LPK, S::LPK2>(qr[gi], a.qn_w, a.eps, ls);
            if (cs && dims_on) rope_units<HD, EB, NV4, S::LPK>(qr[gi], cs, sn, ls);
        }
    }

    float m[G], l[G];
    f32x4 acc[G][NV4];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
#pragma unroll
        for (int i = 0; i < NV4; ++i) acc[gi][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // Iteration `it` covers the split's local superblocks it*U .. +U; wave step (u, wave)
    // reads block `wave` of local superblock it*U + u, i.e. global rows
    // (((it*U + u)*nsplit + split)*kWaves + wave)*KPW + kg. Each iteration gets buffer
    // resources based at its first global row (64-bit pointer arithmetic on the scalar
    // unit), so the per-lane offsets are the same for every iteration and stay far below
    // 2^31; rows at or past `ce` are out of range and read as zeros without touching
    // memory.
    const int blk_stride = U * kWaves * a.nsplit;  // global blocks per iteration
    int rowof[U], voff[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        rowof[u] = ((u * a.nsplit + split) * kWaves + wave) * S::KPW + kg;  // minus it0
        // (lanes without dims read past every range check: zeros, no memory access)
        voff[u] = dims_on ? rowof[u] * row_bytes + dim_byte<S::LPK, EB>(0, ls) : 0x7FFF0000;
    }
    const char *kbase = static_cast<const char *>(a.kc) + (size_t)kvh * HD * EB;
    const char *vbase = static_cast<const char *>(a.vc) + (size_t)kvh * HD * EB;
    auto rows_from = [&](int it) { return it * blk_stride * S::KPW; };
    auto load_iter = [&](int it, Raw (&kv)[U][NL], Raw (&vv)[U][NL]) {
        const int r0 = rows_from(it);
        const int left = min(ce - r0, blk_stride * S::KPW);  // rows in range, window-capped
        const int nbytes = left > 0 ? (left - 1) * row_bytes + HD * EB : 0;
        const size_t off = (size_t)r0 * row_bytes;
        const __amdgpu_buffer_rsrc_t kres = make_rsrc(kbase + off, nbytes);
        const __amdgpu_buffer_rsrc_t vres = make_rsrc(vbase + off, nbytes);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                // The dim offset goes in the scalar offset: the row offsets stay the only
                // per-lane values (a hoisted per-load address would cost a VGPR each).
                // Range checks decide by row either way, since a row's dims end within
                // its HD*EB bytes.
                kv[u][j] = buffer_load_row<EB>(kres, voff[u], j * S::LPK * LB);
                vv[u][j] = buffer_load_row<EB>(vres, voff[u], j * S::LPK * LB);
            }
    };
    // Online-softmax update of every head with the U rows of one iteration (rows at or
    // past `ce` are masked out).
    auto consume_iter = [&](int it, const Raw (&kv)[U][NL], const Raw (&vv)[U][NL]) {
        const int r0 = rows_from(it);
        // Scores of every head first (their DPP chains interleave).
        float sc[G][U];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                f32x4 t = qr[gi][0] * unit_f32<EB>(kv[u], 0);
#pragma unroll
                for (int i = 1; i < NV4; ++i) t += qr[gi][i] * unit_f32<EB>(kv[u], i);
                float sv = (t.x + t.y) + (t.z + t.w);
                sv = eb::group_sum<S::LPK2>(sv);
                sc[gi][u] = (r0 + rowof[u] < ce) ? sv * a.scale_log2 : -INFINITY;
            }
        // Lazy rescale: a head's reference max m moves only when a score exceeds it by more
        // than kSlack (log2 units), and the rescale of l and acc is skipped for the whole
        // wave when no lane group needs it. Terms 2^(s - m) then stay below 2^kSlack; the
        // result is the same up to rounding, since l and acc always share the reference.
        float mloc[G];
        bool grow[G];
        bool any = false;
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            mloc[gi] = sc[gi][0];
#pragma unroll
            for (int u = 1; u < U; ++u) mloc[gi] = fmaxf(mloc[gi], sc[gi][u]);
            grow[gi] = mloc[gi] > m[gi] + kSlack;
            any = any || grow[gi];
        }
        auto rescale = [&]() {
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                // 0 when m was -inf; exactly 1 for the lane groups that keep their max
                const float corr = grow[gi] ? eb::fast_exp2(m[gi] - mloc[gi]) : 1.0f;
                l[gi] *= corr;
#pragma unroll
                for (int i = 0; i < NV4; ++i) acc[gi][i] *= corr;
                m[gi] = grow[gi] ? mloc[gi] : m[gi];
            }
        };
        auto accumulate = [&]() {
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                const float mref = (m[gi] == -INFINITY) ? 0.0f : m[gi];
                float p[U];
                float psum = 0.0f;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    p[u] = eb::fast_exp2(sc[gi][u] - mref);
                    psum += p[u];
                }
                l[gi] += psum;
#pragma unroll
                for (int i = 0; i < NV4; ++i) {
                    f32x4 t = acc[gi][i];
#pragma unroll
                    for (int u = 0; u < U; ++u) t += p[u] * unit_f32<EB>(vv[u], i);
                    acc[gi][i] = t;
                }
            }
        };
        if constexpr (kUpdatePerBranch<HD, EB, G>) {
            if (__builtin_amdgcn_ballot_w64(any) != 0) {
                rescale();
                accumulate();
                // (a step only this path has, so that the compiler does not merge the two
                // copies of the update back into one after the branch)
                asm volatile("" : "+v"(l[0]));
            } else {
                accumulate();
            }
        } else {
            if (__builtin_amdgcn_ballot_w64(any) != 0) rescale();
            accumulate();
        }
    };

    // Iterations run in pairs (A, B): both buffers are loaded before the first is used
    // and each is refilled right after it is consumed. The loop is counted and its loads
    // unconditional (a load under a branch is sunk next to its use by the compiler,
    // draining the queue); an iteration past the split's blocks reads zeros and is masked.
    const int n_iter = (my_blk + U * kWaves - 1) / (U * kWaves);
    const int n_pairs = (n_iter + 1) / 2;
    if (n_pairs > 0) {
        Raw kA[U][NL], vA[U][NL], kB[U][NL], vB[U][NL];
        load_iter(0, kA, vA);
        load_iter(1, kB, vB);
        for (int pr = 1; pr < n_pairs; ++pr) {
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(2 * pr - 2, kA, vA);
            load_iter(2 * pr, kA, vA);
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(2 * pr - 1, kB, vB);
            load_iter(2 * pr + 1, kB, vB);
        }
        __builtin_amdgcn_sched_barrier(0);
        consume_iter(2 * n_pairs - 2, kA, vA);
        consume_iter(2 * n_pairs - 1, kB, vB);
    }

    // Key `pos` from knew/vnew, folded into the first lane group of wave 0.
    if (tail_new && wave == 0) {
        f32x4 kn[NV4], vn[NV4];
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            kn[i] = dims_on ? *reinterpret_cast<const f32x4 *>(a.knew + (size_t)kvh * HD +
                                                               dim_of<S::LPK, EB>(i, ls))
                            : z;
            vn[i] = dims_on ? *reinterpret_cast<const f32x4 *>(a.vnew + (size_t)kvh * HD +
                                                               dim_of<S::LPK, EB>(i, ls))
                            : z;
        }
        if (a.prologue) {
            if (a.kn_w) norm_units<HD, EB, NV4, S::LPK, S::LPK2>(kn, a.kn_w, a.eps, ls);
            if (a.vn_w) norm_units<HD, EB, NV4, S::LPK, S::LPK2>(vn, a.vn_w, a.eps, ls);
            if (a.rcos && dims_on)
                rope_units<HD, EB, NV4, S::LPK>(kn, a.rcos + (size_t)a.rope_row * (HD / 2),
                                         a.rsin + (size_t)a.rope_row * (HD / 2), ls);
        }
        // The new cache row (after the prologue's norm and RoPE), one lane group per KV
        // head. No workgroup reads cache row `pos` in this launch. Written here rather than
        // before the stream, where the first wave of these workgroups waited on the row's
        // loads before issuing its own (these workgroups then ended last).
        if (sub == 0 && kg == 0 && dims_on) {
            const size_t dst = (size_t)pos * a.hkv * HD + (size_t)kvh * HD;
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                const int d = dim_of<S::LPK, EB>(i, ls);
                store_cache4<EB>(a.kc_w, dst + d, kn[i]);
                store_cache4<EB>(a.vc_w, dst + d, vn[i]);
            }
        }
        if constexpr (EB < 4) {  // the value the cache row now holds
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                kn[i] = through_cache<EB>(kn[i]);
                vn[i] = through_cache<EB>(vn[i]);
            }
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            f32x4 t = qr[gi][0] * kn[0];
#pragma unroll
            for (int i = 1; i < NV4; ++i) t += qr[gi][i] * kn[i];
            const float s = eb::group_sum<S::LPK2>((t.x + t.y) + (t.z + t.w)) * a.scale_log2;
            if (kg == 0) {
                const float mnew = fmaxf(m[gi], s);
                const float corr = eb::fast_exp2(m[gi] - mnew);
                const float p = eb::fast_exp2(s - mnew);
                l[gi] = l[gi] * corr + p;
#pragma unroll
                for (int i = 0; i < NV4; ++i) acc[gi][i] = acc[gi][i] * corr + p * vn[i];
                m[gi] = mnew;
            }
        }
    }

    // Epilogue, in two levels. Within a wave the KPW lane groups' states (m, l, acc) meet
    // through lane permutes, each weighted by 2^(m - M_wave). A 32-lane swap of two
    // different units followed by an add leaves one unit's sum in the lower half of the
    // wave and the other's in the upper half, so each halving of the lanes also halves the
    // registers: after the 32- and 16-lane steps lane L holds unit (L >> 4) & 3 of its
    // lane slot (16 dims per lane; with 8, two components of unit L >> 5), and the row
    // rotations finish the lane groups that share a 16-lane row.
    // The kWaves wave states then meet in LDS, combined per output with one weight each.
    static_assert(kWaves == 4, "the wave states are read as one f32x4");
    constexpr int WS = S::WS;
    extern __shared__ float smem[];
    float *s_acc = smem;                // [kWaves][WS]: wave, then head gi, then dim
    float *s_m = s_acc + kWaves * WS;   // [G][kWaves]
    float *s_l = s_m + G * kWaves;      // [G][kWaves]
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        const float mw = eb::class_reduce<S::LPK2, true>(m[gi]);
        const float w = eb::fast_exp2(m[gi] - (mw == -INFINITY ? 0.0f : mw));
        const float lw = eb::class_reduce<S::LPK2, false>(l[gi] * w);
        if (lane == 0) {
            s_m[gi * kWaves + wave] = mw;
            s_l[gi * kWaves + wave] = lw;
        }
        float *dst = s_acc + wave * WS + gi * HD;
        if constexpr (NV4 == 4) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 t = acc[gi][i] * w;
                v[4 * i + 0] = t.x;
                v[4 * i + 1] = t.y;
                v[4 * i + 2] = t.z;
                v[4 * i + 3] = t.w;
            }
            float v2[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)  // lower half: v[k] summed; upper: v[k + 8]
                v2[k] = eb::swap_sum32(v[k], v[k + 8]);
            f32x4 out;
#pragma unroll
            for (int k = 0; k < 4; ++k)  // even rows: v2[k] summed; odd rows: v2[k + 4]
                out[k] = eb::row_class_reduce<S::LPK2, false>(eb::swap_sum16(v2[k], v2[k + 4]));
            if ((lane & 15) < S::LPK)
                *reinterpret_cast<f32x4 *>(dst + dim_of<S::LPK, EB>((lane >> 4) & 3, ls)) = out;
        } else if constexpr (NV4 == 2 && S::LPK2 == 16) {
            // 8 dims per lane, the 4 lane groups in the 4 rows of 16 lanes: the same
            // halving swaps leave lane L with 2 of the 8 sums, unit (L >> 5) and components
            // 2 ((L >> 4) & 1) + 0, 1 (6 swaps and adds against 16 lane exchanges).
            float v[8];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const f32x4 t = acc[gi][i] * w;
                v[4 * i + 0] = t.x;
                v[4 * i + 1] = t.y;
                v[4 * i + 2] = t.z;
                v[4 * i + 3] = t.w;
            }
            float v2[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)  // lower half: v[k] summed; upper: v[k + 4]
                v2[k] = eb::swap_sum32(v[k], v[k + 4]);
            const float o0 = eb::swap_sum16(v2[0], v2[2]);  // even rows: v2[0]; odd: v2[2]
            const float o1 = eb::swap_sum16(v2[1], v2[3]);
            if (dims_on)
                *reinterpret_cast<float2 *>(dst + dim_of<S::LPK, EB>(lane >> 5, ls) +
                                            2 * ((lane >> 4) & 1)) = make_float2(o0, o1);
        } else {
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                const f32x4 t = acc[gi][i] * w;
                f32x4 out;
                out.x = eb::class_reduce<S::LPK2, false>(t.x);
                out.y = eb::class_reduce<S::LPK2, false>(t.y);
                out.z = eb::class_reduce<S::LPK2, false>(t.z);
                out.w = eb::class_reduce<S::LPK2, false>(t.w);
                if (kg == 0 && dims_on)
                    *reinterpret_cast<f32x4 *>(dst + dim_of<S::LPK, EB>(i, ls)) = out;
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
        const int gi = idx / HD;
        const int d = idx % HD;
        const f32x4 m4 = *reinterpret_cast<const f32x4 *>(s_m + gi * kWaves);
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(s_l + gi * kWaves);
        const float M = fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w));
        const float mref = (M == -INFINITY) ? 0.0f : M;
        const float w0 = eb::fast_exp2(m4.x - mref), w1 = eb::fast_exp2(m4.y - mref);
        const float w2 = eb::fast_exp2(m4.z - mref), w3 = eb::fast_exp2(m4.w - mref);
        const float A = (w0 * s_acc[idx] + w1 * s_acc[WS + idx]) +
                        (w2 * s_acc[2 * WS + idx] + w3 * s_acc[3 * WS + idx]);
        const float L = (w0 * l4.x + w1 * l4.y) + (w2 * l4.z + w3 * l4.w);
        const int hh = head0 + gi;
        if (a.nsplit == 1) {
            a.o[(size_t)hh * HD + d] = A / L;
        } else {
            a.part_acc[((size_t)split * a.h + hh) * HD + d] = A;
            if (d == 0) {
                a.part_ml[((size_t)split * a.h + hh) * 2 + 0] = M;
                a.part_ml[((size_t)split * a.h + hh) * 2 + 1] = L;
            }
        }
    }
}

// ---- E4M3 caches on the matrix cores ----------------------------------------------------
//
// decode_mx_kernel<HD, G>: OCP FP8 E4M3 caches at head dims 64, 128 and 256. Same grid, split
// plan, partial layout and merge as decode_kernel. Per byte an E4M3 cache carries four times
// the f32 elements, and the lane-wise kernel's multiply-add per element and head bounds it
// (67 % of wave cycles issuing VALU at Mistral 32k keys); here both products run on the
// matrix cores. A wave step is a tile of 16 keys; lane (n, g) is lane n + 16 g.
//  - Scores S[key][head] = K q^T on v_mfma_f32_16x16x32_f16. A = the tile's 16 key rows:
//    lane (n, g) holds 8 dims of key n per 32-dim chunk (a 16-byte load holds 16 dims, two
//    chunks' worth), converted to f16 (exact: every E4M3 value is an f16). B = q: column n
//    is head n % G (heads repeated across the 16 columns), as the f16 high and low halves of
//    q * scale * log2(e) * 2^e_h (two products per chunk; each f16 x f16 product is exact in
//    f32). e_h is a power of two per head that puts its largest |q| in [2^13, 2^14), so that
//    the halves neither overflow nor lose bits to subnormals. Lane (n, g) then holds the
//    scores of keys 4g .. 4g + 3 for head n % G.
//  - Online softmax with a lazily moved reference max per head (wave-uniform), weights
//    p = 2^(s - m) * 2^7: below 2^15 (s exceeds m by at most the slack of 8), so their f16
//    halves keep terms down to 2^-31 of the reference term. The reference is a score
//    itself, so a lone key's weight is exactly 2^7 and its output exactly its V row.
//  - O[head][dim] += P V on v_mfma_f32_16x16x16_f16. A = P: lane (n, g) supplies head
//    n % G at keys 4g .. 4g + 3, which are exactly its score registers (as f16 high and
//    low halves: two products). B = V: lane (n, g) loads dims DV n .. DV n + DV - 1
//    (DV = HD / 16) of keys 4g + t, t = 0..3, and product e (0 .. DV - 1) takes element e
//    of each load, so output column n of accumulator e is dim DV n + e. No lane exchange
//    and no LDS between the two products.
//  - Lane (n, g) register r of accumulator e holds head (4g + r) % G: every lane group
//    holds every head, so the epilogue reads lanes 0..15.
// The new key (knew / vnew, after the optional norm and RoPE) is rounded to E4M3 in LDS and
// folded in by the owning split's wave 0 as one more tile with a single valid key, through
// the same code as the cache rows.
// Measured against decode_kernel (HIP events, decode steps from graphs): Mistral 32k keys
// 25.0 -> 20.0 us, Qwen L=8191 12.8 -> 10.7 us, Gemma-4 16k keys 20.6 -> 18.9 us. The same
// scheme over IEEE-half caches measured 3-5 % slower than decode_kernel.
// 0 runs decode_kernel over E4M3 caches too (the comparison above).
#ifndef EB_DECODE_MX
#define EB_DECODE_MX 1
#endif

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr bool mx_head_dim(int hd) { return hd == 64 || hd == 128 || hd == 256; }

template <int HD, int G>
struct MxShape {
    static constexpr int EB = 1;
    static_assert(mx_head_dim(HD), "head dim 64, 128 or 256");
    static constexpr int KPW = 16;                 // keys per wave step (one tile)
    static constexpr int NC = HD / 32;             // 32-dim chunks of a key row
    static constexpr int KL = NC / 2;              // K loads per tile and lane (16 bytes)
    static constexpr int DV = HD / 16;             // V dims per lane per row
    static constexpr int VW = DV * EB / 4;         // words per lane per V row
    // Tiles per iteration: each of the two register buffers holds U tiles' loads. One at
    // every head dim: at head_dim 256 two measured 8 % slower (its tiles' loads,
    // accumulators and q halves fill the registers); at head_dim 128 two against one, A/B
    // on one box, two rounds, us per step: Mistral 2048 / 8192 / 32768 / 65536 keys 10.62
    // -> 8.81, 11.25 -> 10.57, 20.21 -> 19.51, 31.69 -> 30.24; Qwen 2048 / 8192 / 32768
    // keys 9.60 -> 7.85, 10.31 -> 9.58, 19.62 -> 18.41 (half the keys per iteration also
    // lets the planner give short caches more splits).
    static constexpr int U = 1;
    static constexpr int KEYS_PER_ITER = kWaves * KPW * U;
    static constexpr int RW = HD * EB / 4;         // words of one cache row (one KV head)
    static constexpr int WS = G * HD + 4;          // epilogue state per wave (floats)
    // LDS (floats): q [G][HD] | 2^-e_h [4] | knew, vnew [HD] each | their cache-type rows
    // [RW] each | epilogue: acc [kWaves][WS], m [G][kWaves], l [G][kWaves].
    static constexpr int OFF_QINV = G * HD;
    static constexpr int OFF_KN = OFF_QINV + 4;
    static constexpr int OFF_VN = OFF_KN + HD;
    static constexpr int OFF_KR = OFF_VN + HD;
    static constexpr int OFF_VR = OFF_KR + RW;
    static constexpr int OFF_ACC = OFF_VR + RW;
    static constexpr int OFF_M = OFF_ACC + kWaves * WS;
    static constexpr int OFF_L = OFF_M + G * kWaves;
    static constexpr size_t LDS_BYTES = sizeof(float) * (size_t)(OFF_L + G * kWaves);
};

// Cache policy of the E4M3 matrix-core kernel's loads. Non-temporal loads measured faster
// at head_dim 256 (Gemma-4 16383 keys 19.34 -> 18.68 us per step, 8191 keys unchanged). At
// head_dim 128 they follow the bytes a step reads (A/B on one box, two rounds, us per step,
// default -> non-temporal, one tile per iteration): Mistral 2048 / 4096 / 8192 keys 9.14 ->
// 8.63, 9.75 -> 8.84, 11.13 -> 10.48; Qwen 2048 / 4096 / 8192 keys 8.55 -> 7.96, 9.04 ->
// 8.15, 10.43 -> 9.65; 16384 keys a tie or better (Mistral 13.69 -> 13.63, Qwen 13.15 ->
// 12.92); beyond, slower (Mistral 32768 / 65536 keys 19.25 -> 20.26, 30.18 -> 32.92, Qwen
// 32768 keys 18.73 -> 19.48). So head_dim 128 streams them while a step reads at most
// kMxNtBytes of K and V (16384 keys of 8 KV heads).
constexpr size_t kMxNtBytes = (size_t)32 << 20;

template <int HD>
bool mx_streams_nt(const DecodeArgs &a) {
    if constexpr (HD == 256) return true;
    else if constexpr (HD == 128) return (size_t)a.keys * a.hkv * HD * 2 <= kMxNtBytes;
    else return false;
}

// W words of a row slice from a raw buffer (range-checked by the resource), with cache
// policy AUX.
template <int W, int AUX>
__device__ __forceinline__ void load_words(unsigned *dst, __amdgpu_buffer_rsrc_t r, int voff,
                                           int soff) {
    if constexpr (W % 4 == 0) {
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const u32x4 v = __builtin_bit_cast(
                u32x4,
                __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff + 16 * i, AUX));
            dst[4 * i + 0] = v[0];
            dst[4 * i + 1] = v[1];
            dst[4 * i + 2] = v[2];
            dst[4 * i + 3] = v[3];
        }
    } else if constexpr (W == 2) {
        const u32x2 v = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX));
        dst[0] = v[0];
        dst[1] = v[1];
    } else {
        static_assert(W == 1, "1, 2 or a multiple of 4 words");
        dst[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, AUX);
    }
}

// Two f32 as packed f16, rounded toward zero (the weights' high halves; the low halves
// take the remainders).
__device__ __forceinline__ unsigned pk_f16(float a, float b) {
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ float f16_lo(unsigned w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(unsigned w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}

// First dim of lane group g's 8 dims in 32-dim chunk c: a lane's 16-byte load holds 16
// consecutive dims, the first 8 in chunk 2C and the rest in chunk 2C + 1 (64 bytes of each
// row per load instruction). The products sum over a chunk's dims in any order; q's operand
// follows the same map.
__device__ __forceinline__ int chunk_dim(int c, int g) {
    return 64 * (c / 2) + 16 * g + 8 * (c % 2);
}

// Two E4M3 values (bytes 0, 1 or 2, 3 of w) as packed f16, exact (gfx950's scaled FP8
// conversion, scale 1).
__device__ __forceinline__ unsigned f8x2_f16(unsigned w, bool hi) {
    return __builtin_bit_cast(unsigned, hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true)
                                           : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}

// A operand of chunk c (8 dims of the lane's key) from the lane's raw K words [KL][4].
__device__ __forceinline__ f16x8 k_operand(const unsigned (*kr)[4], int c) {
    const unsigned w0 = kr[c / 2][2 * (c % 2)], w1 = kr[c / 2][2 * (c % 2) + 1];
    return __builtin_bit_cast(f16x8, u32x4{f8x2_f16(w0, false), f8x2_f16(w0, true),
                                           f8x2_f16(w1, false), f8x2_f16(w1, true)});
}

template <int HD, int G, bool STREAM_NT>
__global__ __launch_bounds__(kThreads, 1) void decode_mx_kernel(DecodeArgs a) {
    constexpr int AUX = STREAM_NT ? kStreamPolicy : 0;
    using S = MxShape<HD, G>;
    constexpr int EB = S::EB;
    constexpr int U = S::U, NC = S::NC, KL = S::KL, DV = S::DV, VW = S::VW;
    constexpr int KPW = S::KPW;
    static_assert(G == 1 || G == 2 || G == 4, "heads per workgroup");
    extern __shared__ float smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int col = blockIdx.x;
    const int kvh = col % a.hkv;
    const int sub = col / a.hkv;
    const int head0 = kvh * a.g + sub * G;
    const int split = blockIdx.y;
    const int pos = a.keys - 1;
    const int ce = a.knew != nullptr ? pos : a.keys;
    const bool tail_new = a.knew != nullptr && split == (pos / KPW) % a.nsplit;
    const int nblk = (ce + KPW - 1) / KPW;
    const int my_blk = nblk > split ? (nblk - split + a.nsplit - 1) / a.nsplit : 0;
    const int row_bytes = a.hkv * HD * EB;

    // ---- main-loop addressing (as decode_kernel's, with tiles of 16 keys) -------------------
    // Iteration `it` covers the split's local blocks it*U*kWaves .. +U*kWaves; tile (u, wave)
    // is local block it*U*kWaves + u*kWaves + wave, at rows tb[u] + rows_from(it) .. +15.
    const int blk_stride = U * kWaves * a.nsplit;
    int tb[U], kvo[U], vvo[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        tb[u] = ((u * kWaves + wave) * a.nsplit + split) * KPW;
        kvo[u] = (tb[u] + n) * row_bytes + 16 * g;           // K: key n, its 16 bytes
        vvo[u] = (tb[u] + 4 * g) * row_bytes + DV * n * EB;  // V: key 4g (+t), dims DV n
    }
    const char *kbase = static_cast<const char *>(a.kc) + (size_t)kvh * HD * EB;
    const char *vbase = static_cast<const char *>(a.vc) + (size_t)kvh * HD * EB;
    auto rows_from = [&](int it) { return it * blk_stride * KPW; };
    using KRaw = unsigned[U][KL][4];
    using VRaw = unsigned[U][4][VW];
    auto load_iter = [&](int it, KRaw &kr, VRaw &vr) {
        const int r0 = rows_from(it);
        const int left = min(ce - r0, blk_stride * KPW);
        const int nbytes = left > 0 ? (left - 1) * row_bytes + HD * EB : 0;
        const size_t off = (size_t)r0 * row_bytes;
        const __amdgpu_buffer_rsrc_t kres = make_rsrc(kbase + off, nbytes);
        const __amdgpu_buffer_rsrc_t vres = make_rsrc(vbase + off, nbytes);
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int c = 0; c < KL; ++c) load_words<4, AUX>(kr[u][c], kres, kvo[u], 64 * c);
#pragma unroll
            for (int t = 0; t < 4; ++t) load_words<VW, AUX>(vr[u][t], vres, vvo[u] + t * row_bytes, 0);
        }
    };

    // ---- q and the new rows: their loads first, then the first two iterations' ----------
    static_assert(G * HD / 4 <= kThreads, "one 16-byte q load per thread");
    const f32x4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 q4 = threadIdx.x < G * HD / 4
                         ? reinterpret_cast<const f32x4 *>(a.q + (size_t)head0 * HD)[threadIdx.x]
                         : z4;
    const bool new4 = tail_new && threadIdx.x < HD / 4;
    const f32x4 kn4 = new4 ? reinterpret_cast<const f32x4 *>(a.knew + (size_t)kvh * HD)[threadIdx.x] : z4;
    const f32x4 vn4 = new4 ? reinterpret_cast<const f32x4 *>(a.vnew + (size_t)kvh * HD)[threadIdx.x] : z4;
    __builtin_amdgcn_sched_barrier(0);
    // (an iteration past the split's blocks reads zeros; a split without blocks ignores them)
    KRaw kA, kB;
    VRaw vA, vB;
    load_iter(0, kA, vA);
    load_iter(1, kB, vB);
    __builtin_amdgcn_sched_barrier(0);

    // ---- q (and the new row) in LDS, after the optional norm and RoPE --------------------
    float *s_q = smem;
    float *s_qinv = smem + S::OFF_QINV;
    float *s_kn = smem + S::OFF_KN;
    float *s_vn = smem + S::OFF_VN;
    unsigned *s_kr = reinterpret_cast<unsigned *>(smem + S::OFF_KR);
    unsigned *s_vr = reinterpret_cast<unsigned *>(smem + S::OFF_VR);
    if (threadIdx.x < G * HD / 4) reinterpret_cast<f32x4 *>(s_q)[threadIdx.x] = q4;
    if (new4) {
        reinterpret_cast<f32x4 *>(s_kn)[threadIdx.x] = kn4;
        reinterpret_cast<f32x4 *>(s_vn)[threadIdx.x] = vn4;
    }
    __syncthreads();
    {
        // Row jobs: 0..G-1 the query heads, G the new key, G + 1 the new value. Each lane
        // owns the dim pairs (p, p + HD/2), p = lane, lane + 64, ..., so that RMSNorm and
        // RoPE never read another lane's dims.
        constexpr int NP = (HD / 2 + 63) / 64;
        const float *cs = (a.prologue && a.rcos) ? a.rcos + (size_t)a.rope_row * (HD / 2) : nullptr;
        const float *sn = (a.prologue && a.rsin) ? a.rsin + (size_t)a.rope_row * (HD / 2) : nullptr;
        const int njobs = tail_new ? G + 2 : G;
        for (int job = wave; job < njobs; job += kWaves) {
            float *x = job < G ? s_q + job * HD : (job == G ? s_kn : s_vn);
            const float *nw = !a.prologue ? nullptr : job < G ? a.qn_w : job == G ? a.kn_w : a.vn_w;
            const bool rope = cs != nullptr && job <= G;
            float x1[NP], x2[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = lane + 64 * i;
                x1[i] = p < HD / 2 ? x[p] : 0.0f;
                x2[i] = p < HD / 2 ? x[p + HD / 2] : 0.0f;
            }
            if (nw) {  // RMSNorm (kernels/src/rmsnorm.rs:6-38): x * (1/sqrt(mean x^2 + eps)) * w
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < NP; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
                ss = eb::class_reduce<1, false>(ss);
                const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = lane + 64 * i;
                    if (p < HD / 2) {
                        x1[i] = x1[i] * inv * nw[p];
                        x2[i] = x2[i] * inv * nw[p + HD / 2];
                    }
                }
            }
            if (rope) {  // RoPE (kernels/src/rope.rs:6-32): pairs (p, p + HD/2), angle p
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = lane + 64 * i;
                    if (p < HD / 2) {
                        const float c = cs[p], s = sn[p];
                        const float y1 = x1[i] * c - x2[i] * s;
                        const float y2 = x2[i] * c + x1[i] * s;
                        x1[i] = y1;
                        x2[i] = y2;
                    }
                }
            }
            if (job < G) {
                // q * scale * log2(e), then the head's power of two
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    x1[i] *= a.scale_log2;
                    x2[i] *= a.scale_log2;
                    amax = fmaxf(amax, fmaxf(fabsf(x1[i]), fabsf(x2[i])));
                }
                amax = eb::class_reduce<1, true>(amax);
                int ex = 0;
                if (amax > 0.0f && amax <= 3.0e38f) {
                    frexpf(amax, &ex);
                    ex = 14 - ex;  // amax * 2^ex in [2^13, 2^14)
                    // (2^ex and 2^-ex stay normal floats; below 2^-112 a head's q ends in
                    // f16 subnormals, scores of that size being nothing next to 0)
                    ex = ex < -126 ? -126 : ex > 126 ? 126 : ex;
                }
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = lane + 64 * i;
                    if (p < HD / 2) {
                        x[p] = ldexpf(x1[i], ex);
                        x[p + HD / 2] = ldexpf(x2[i], ex);
                    }
                }
                if (lane == 0) s_qinv[job] = ldexpf(1.0f, -ex);
            } else {
                // the new row as the cache holds it: in LDS (for the fold) and, by the first
                // head subgroup, in cache row `pos` (no workgroup reads that row here)
                unsigned *raw = job == G ? s_kr : s_vr;
                void *dst = job == G ? a.kc_w : a.vc_w;
                const size_t drow = (size_t)pos * a.hkv * HD + (size_t)kvh * HD;
#pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int p = lane + 64 * i;
                    if (p < HD / 2) {
#pragma unroll
                        for (int side = 0; side < 2; ++side) {
                            const int d = p + side * (HD / 2);
                            const float v = side ? x2[i] : x1[i];
                            const uint8_t bv = (uint8_t)(eb::f8e4m3_bits(v) & 0xFFu);
                            reinterpret_cast<uint8_t *>(raw)[d] = bv;
                            if (sub == 0) static_cast<uint8_t *>(dst)[drow + d] = bv;
                        }
                    }
                }
            }
        }
    }
    __syncthreads();

    // B operands of the score products: head n % G, the lane's dims of chunk c, high and
    // low halves.
    f16x8 qh[NC], ql[NC];
    const int own = n % G;
    const float c_own = s_qinv[own];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const float *src = s_q + own * HD + chunk_dim(c, g);
        const f32x4 v0 = *reinterpret_cast<const f32x4 *>(src);
        const f32x4 v1 = *reinterpret_cast<const f32x4 *>(src + 4);
        const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const _Float16 hi = (_Float16)v[j];
            qh[c][j] = hi;
            ql[c][j] = (_Float16)(v[j] - (float)hi);
        }
    }

    // ---- the online softmax state --------------------------------------------------------
    floatx4 acc[DV];
#pragma unroll
    for (int e = 0; e < DV; ++e) acc[e] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float mh[G];  // reference max per head (log2 units), the same in every lane
#pragma unroll
    for (int h = 0; h < G; ++h) mh[h] = -INFINITY;
    float l_own = 0.0f;           // this lane's share of the weight sum of head `own`
    float m_own = -INFINITY;      // m of head `own`
    float mref = 0.0f;            // m_own, 0 while -inf
    float gthr = -INFINITY;       // a score x = s - mref above this moves the reference

    // NT tiles at once: raw K words [NT][KL][4], raw V words [NT][4][VW]; in tile t the
    // keys 4g + r < lim[t] are valid (wave-uniform). All score products first, then one
    // softmax update for the NT tiles, then the P V products.
    auto consume = [&](auto nt, const unsigned (*kr)[KL][4], const unsigned (*vr)[4][VW],
                       const int *lim) {
        constexpr int NT = decltype(nt)::value;
        floatx4 sc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            // two accumulators (high and low halves of q): no product waits for its neighbour
            floatx4 s = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f16x8 kk = k_operand(kr[t], c);
                s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qh[c], s, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, ql[c], s2, 0, 0, 0);
            }
            sc[t] = s + s2;
        }
        float x[NT][4];
        auto weigh = [&] {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) x[t][r] = fmaf(sc[t][r], c_own, -mref);
                if (lim[t] < KPW) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (4 * g + r >= lim[t]) x[t][r] = -INFINITY;
                }
            }
        };
        weigh();
        bool grow = false;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) grow = grow || x[t][r] > gthr;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            // New reference per head: the tiles' max where it exceeds m by more than the
            // slack, taken from the scores themselves (times the power of two, exact), so
            // that the max key's x is exactly 0.
            float sm = -INFINITY;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (4 * g + r < lim[t]) sm = fmaxf(sm, sc[t][r]);
            sm *= c_own;
            sm = fmaxf(sm, eb::lane_xor16(sm));
            sm = fmaxf(sm, eb::lane_xor32(sm));
            // every lane of head h holds lane h's sm: the same scores, the same reduction
            float corr[G];
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float mt = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm), h));
                const float mn = mt > mh[h] + kSlack ? mt : mh[h];
                corr[h] = mn == mh[h] ? 1.0f : eb::fast_exp2(mh[h] - mn);
                mh[h] = mn;
            }
#pragma unroll
            for (int e = 0; e < DV; ++e)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[e][r] *= corr[r % G];
            // the same update for the lane's own head, from its own sm
            const float mn = sm > m_own + kSlack ? sm : m_own;
            l_own *= mn == m_own ? 1.0f : eb::fast_exp2(m_own - mn);
            m_own = mn;
            mref = m_own == -INFINITY ? 0.0f : m_own;
            gthr = m_own == -INFINITY ? -INFINITY : kSlack;
            weigh();
        }
        f16x4 ph[NT], pl[NT];
        f16x4 vb[NT][DV];  // B operands: element e of the lane's four rows
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = eb::fast_exp2(x[t][r]) * 128.0f;
            l_own += (p[0] + p[1]) + (p[2] + p[3]);
            // A operands: the weights' f16 high halves and their remainders
            const unsigned h01 = pk_f16(p[0], p[1]), h23 = pk_f16(p[2], p[3]);
            const unsigned l01 = pk_f16(p[0] - f16_lo(h01), p[1] - f16_hi(h01));
            const unsigned l23 = pk_f16(p[2] - f16_lo(h23), p[3] - f16_hi(h23));
            ph[t] = __builtin_bit_cast(f16x4, u32x2{h01, h23});
            pl[t] = __builtin_bit_cast(f16x4, u32x2{l01, l23});
#pragma unroll
                for (int e = 0; e < DV; e += 2) {
                    // bytes e, e + 1 of rows 0, 1 (and 2, 3) as [r0.e, r1.e, r0.e+1, r1.e+1]
                    // (v_perm byte selectors: 0-3 the second operand's bytes, 4-7 the first's)
                    const unsigned k = (unsigned)(e % 4);
                    const unsigned sel = k | (4u + k) << 8 | (k + 1u) << 16 | (5u + k) << 24;
                    const unsigned b01 = __builtin_amdgcn_perm(vr[t][1][e / 4], vr[t][0][e / 4], sel);
                    const unsigned b23 = __builtin_amdgcn_perm(vr[t][3][e / 4], vr[t][2][e / 4], sel);
                    vb[t][e] = __builtin_bit_cast(f16x4, u32x2{f8x2_f16(b01, false), f8x2_f16(b23, false)});
                    vb[t][e + 1] = __builtin_bit_cast(f16x4, u32x2{f8x2_f16(b01, true), f8x2_f16(b23, true)});
                }
        }
        // high halves into every accumulator, then the low halves (independent neighbours)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < DV; ++e)
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[t], vb[t][e], acc[e], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < DV; ++e)
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl[t], vb[t][e], acc[e], 0, 0, 0);
    };
    auto consume_iter = [&](int it, const KRaw &kr, const VRaw &vr) {
        const int r0 = rows_from(it);
        int lim[U];
#pragma unroll
        for (int u = 0; u < U; ++u) lim[u] = ce - r0 - tb[u];
        consume(std::integral_constant<int, U>{}, kr, vr, lim);
    };

    // ---- the main loop: iterations in pairs (A, B), each buffer refilled once consumed ----
    const int n_iter = (my_blk + U * kWaves - 1) / (U * kWaves);
    const int n_pairs = (n_iter + 1) / 2;
    if (n_pairs > 0) {
        for (int pr = 1; pr < n_pairs; ++pr) {
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(2 * pr - 2, kA, vA);
            load_iter(2 * pr, kA, vA);
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(2 * pr - 1, kB, vB);
            load_iter(2 * pr + 1, kB, vB);
        }
        __builtin_amdgcn_sched_barrier(0);
        consume_iter(2 * n_pairs - 2, kA, vA);
        consume_iter(2 * n_pairs - 1, kB, vB);
    }

    // The new key: one more tile whose only valid key (index 0: lanes n = 0 for K, lane
    // group 0's first row for V) is the row in LDS.
    if (tail_new && wave == 0) {
        unsigned kr[1][KL][4], vr[1][4][VW];
#pragma unroll
        for (int c = 0; c < KL; ++c)
#pragma unroll
            for (int w = 0; w < 4; ++w)
                kr[0][c][w] = n == 0 ? s_kr[(64 * c + 16 * g) / 4 + w] : 0u;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int w = 0; w < VW; ++w)
                vr[0][t][w] = (g == 0 && t == 0) ? s_vr[DV * n * EB / 4 + w] : 0u;
        const int lim1[1] = {1};
        consume(std::integral_constant<int, 1>{}, kr, vr, lim1);
    }

    // ---- epilogue: the waves' states meet in LDS (as decode_kernel's) -------------------
    constexpr int WS = S::WS;
    float *s_acc = smem + S::OFF_ACC;
    float *s_m = smem + S::OFF_M;
    float *s_l = smem + S::OFF_L;
    float lt = l_own + eb::lane_xor16(l_own);
    lt += eb::lane_xor32(lt);
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float lh =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lt), h));
        if (lane == 0) {
            s_m[h * kWaves + wave] = mh[h];
            s_l[h * kWaves + wave] = lh;
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int r = 0; r < G; ++r)
#pragma unroll
            for (int e4 = 0; e4 < DV; e4 += 4)
                *reinterpret_cast<f32x4 *>(s_acc + wave * WS + r * HD + DV * n + e4) =
                    f32x4{acc[e4][r], acc[e4 + 1][r], acc[e4 + 2][r], acc[e4 + 3][r]};
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
        const int gi = idx / HD;
        const int d = idx % HD;
        const f32x4 m4 = *reinterpret_cast<const f32x4 *>(s_m + gi * kWaves);
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(s_l + gi * kWaves);
        const float M = fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w));
        const float mref = (M == -INFINITY) ? 0.0f : M;
        const float w0 = eb::fast_exp2(m4.x - mref), w1 = eb::fast_exp2(m4.y - mref);
        const float w2 = eb::fast_exp2(m4.z - mref), w3 = eb::fast_exp2(m4.w - mref);
        const float A = (w0 * s_acc[idx] + w1 * s_acc[WS + idx]) +
                        (w2 * s_acc[2 * WS + idx] + w3 * s_acc[3 * WS + idx]);
        const float L = (w0 * l4.x + w1 * l4.y) + (w2 * l4.z + w3 * l4.w);
        const int hh = head0 + gi;
        if (a.nsplit == 1) {
            a.o[(size_t)hh * HD + d] = A / L;
        } else {
            a.part_acc[((size_t)split * a.h + hh) * HD + d] = A;
            if (d == 0) {
                a.part_ml[((size_t)split * a.h + hh) * 2 + 0] = M;
                a.part_ml[((size_t)split * a.h + hh) * 2 + 1] = L;
            }
        }
    }
}

// Log-sum-exp merge of the split partials (a second launch, so the partials written by
// every XCD are visible without in-kernel fences). Grid (h, ceil(HD / DS)): a workgroup owns
// DS dims of one head (dims past HD in the last block are read as anything and not stored); thread (grp, d) of GROUPS = 256/DS groups folds splits grp,
// grp + GROUPS, ... into a running (M, L, A), issuing a batch of kBatch splits' loads
// before using any, so up to GROUPS*kBatch splits merge in one memory round trip. The
// groups then combine through LDS: o[h][d] = A / L.
constexpr int merge_dims_per_block(int hd) {
    return hd >= 64 ? 64 : hd >= 32 ? 32 : hd >= 16 ? 16 : hd;
}

template <int HD>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(const float *__restrict__ part_acc,
                                                                const float *__restrict__ part_ml,
                                                                float *__restrict__ o, int h,
                                                                int hkv, int nsplit) {
    constexpr int DS = merge_dims_per_block(HD);
    constexpr int GROUPS = kThreads / DS;
    constexpr int kBatch = 16;
    __shared__ float s_m[GROUPS][DS];
    __shared__ float s_l[GROUPS][DS];
    __shared__ float s_a[GROUPS][DS];
    // Workgroup x merges head (x % hkv) * (h / hkv) + x / hkv: with hkv a multiple of the 8
    // XCDs (workgroup ids dealt round robin) it runs on the XCD whose workgroups wrote that
    // head's partials (KV head x % hkv). A/B on one box against head x, two rounds: Qwen
    // L=8191 4661 -> 4690 GB/s, 2048 keys 2187 -> 2209, Gemma-4 16k keys 6190 -> 6237, the
    // half Qwen L=8191 step 10.66 -> 10.58 us.
    const int hh = (int)(blockIdx.x % hkv) * (h / hkv) + (int)(blockIdx.x / hkv);
    const int dl = threadIdx.x % DS;
    const int grp = threadIdx.x / DS;
    const int d = blockIdx.y * DS + dl;
    // Buffer resources over the partials: a split past nsplit is out of range and reads
    // zeros (masked below), so the batch needs no clamping and its offsets are affine.
    const __amdgpu_buffer_rsrc_t racc = make_rsrc(part_acc, nsplit * h * HD * 4);
    const __amdgpu_buffer_rsrc_t rml = make_rsrc(part_ml, nsplit * h * 2 * 4);
    const int acc_step = GROUPS * h * HD * 4, ml_step = GROUPS * h * 2 * 4;
    float M = -INFINITY, L = 0.0f, A = 0.0f;
    for (int s0 = grp; s0 < nsplit; s0 += GROUPS * kBatch) {
        float2 bml[kBatch];
        float ba[kBatch];
        const int acc0 = ((s0 * h + hh) * HD + d) * 4, ml0 = (s0 * h + hh) * 2 * 4;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            bml[j] = __builtin_bit_cast(
                float2, __builtin_amdgcn_raw_buffer_load_b64(rml, ml0 + j * ml_step, 0, 0));
            ba[j] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(racc, acc0 + j * acc_step, 0, 0));
        }
        // Every load of the batch is issued before the first result is used (otherwise the
        // running max below is scheduled between the loads, one round trip each); splits
        // past nsplit are masked here, after the loads.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (s0 + j * GROUPS >= nsplit) bml[j].x = -INFINITY;
        float bM = bml[0].x;
#pragma unroll
        for (int j = 1; j < kBatch; ++j) bM = fmaxf(bM, bml[j].x);
        const float Mn = fmaxf(M, bM);
        const float mref = (Mn == -INFINITY) ? 0.0f : Mn;
        const float c = eb::fast_exp2(M - mref);
        L *= c;
        A *= c;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const float w = eb::fast_exp2(bml[j].x - mref);
            L += w * bml[j].y;
            A += w * ba[j];
        }
        M = Mn;
    }
    s_m[grp][dl] = M;
    s_l[grp][dl] = L;
    s_a[grp][dl] = A;
    __syncthreads();
    if (grp == 0) {
        float Mt = s_m[0][dl];
#pragma unroll
        for (int g2 = 1; g2 < GROUPS; ++g2) Mt = fmaxf(Mt, s_m[g2][dl]);
        const float mref = (Mt == -INFINITY) ? 0.0f : Mt;
        float Lt = 0.0f, At = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < GROUPS; ++g2) {
            const float w = eb::fast_exp2(s_m[g2][dl] - mref);
            Lt += w * s_l[g2][dl];
            At += w * s_a[g2][dl];
        }
        if (HD % DS == 0 || d < HD) o[(size_t)hh * HD + d] = At / Lt;
    }
}

struct DecodePlan {
    int G = 1;       // query heads per workgroup (1, 2 or 4, dividing h/hkv)
    int nsub = 1;    // workgroups per KV head along the head axis
    int nsplit = 1;  // splits along the key axis
    bool short_iter = false;  // the SHORT shape (f32 head_dim 256, short caches)
};

// Caches of at most this many keys take the SHORT shape where it exists.
constexpr size_t kShortKeys = 4096;
static_assert(DecodeShapeOf<256, 2, 4, false>::U == 2 && DecodeShapeOf<256, 2, 4, true>::U == 1,
              "the SHORT shape halves the keys per iteration");

// E4M3 caches at head dims 64, 128 and 256 run decode_mx_kernel.
template <int HD, int EB>
constexpr bool use_mx() {
    return EB_DECODE_MX != 0 && EB == 1 && mx_head_dim(HD);
}

template <int HD, int G, int EB>
constexpr int keys_per_iter_of() {
    if constexpr (use_mx<HD, EB>())
        return MxShape<HD, G>::KEYS_PER_ITER;
    else
        return DecodeShapeOf<HD, G, EB>::KEYS_PER_ITER;
}

template <int G, int EB>
int keys_per_iter_g(size_t hd) {
#define EB_KPI(D) \
    case D: return keys_per_iter_of<D, G, EB>();
    switch (hd) {
        EB_HEAD_DIMS(EB_KPI)
        default: return keys_per_iter_of<256, G, EB>();
    }
#undef EB_KPI
}

template <int EB>
int keys_per_iter_e(size_t hd, int G) {
    switch (G) {
        case 4: return keys_per_iter_g<4, EB>(hd);
        case 2: return keys_per_iter_g<2, EB>(hd);
        default: return keys_per_iter_g<1, EB>(hd);
    }
}

int keys_per_iter(size_t hd, int G, eb::CacheElem ce) {
    switch (ce) {
        case eb::CacheElem::F16: return keys_per_iter_e<2>(hd, G);
        case eb::CacheElem::E4M3: return keys_per_iter_e<1>(hd, G);
        default: return keys_per_iter_e<4>(hd, G);
    }
}

constexpr size_t kMinSplitKeys = 128;

// Workgroups to aim for per CU.
int wgs_per_cu() {
    static int v = [] {
        const char *e = std::getenv("EB_DECODE_WGS_PER_CU");
        int x = e ? std::atoi(e) : 1;
        return (x >= 1 && x <= 64) ? x : 1;
    }();
    return v;
}

DecodePlan plan_decode(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count,
                       eb::CacheElem ce) {
    DecodePlan p;
    const size_t g = h / hkv;
    // At most 4 query heads per workgroup: their q fragments and accumulators, plus two
    // K/V register buffers, must fit the register file without spilling.
    p.G = (g % 4 == 0) ? 4 : (g % 2 == 0) ? 2 : 1;
    p.nsub = (int)(g / p.G);
    const size_t keys = pos + 1;
    const size_t cols = hkv * (size_t)p.nsub;
    p.short_iter = ce == eb::CacheElem::F32 && hd == 256 && keys <= kShortKeys;
    const size_t iter_rows = (size_t)keys_per_iter(hd, p.G, ce) / (p.short_iter ? 2 : 1);
    // Enough workgroups to cover the CUs, but at least one pair of iterations per split;
    // one iteration in the E4M3 matrix-core kernel. There, against a pair (A/B on one box,
    // two rounds, us per step): Qwen 512 / 1024 / 2048 keys 7.90 -> 7.64, 7.92 -> 7.68,
    // 7.99 -> 7.74, Gemma-4 2048 keys 10.77 -> 10.17; elsewhere it measured mixed (half
    // Mistral 1024 keys 8.55 -> 8.65, f32 Gemma-4 1024 keys 8.59 -> 8.47).
    const bool mx = EB_DECODE_MX != 0 && ce == eb::CacheElem::E4M3 && mx_head_dim((int)hd);
    const size_t target = (size_t)cu_count * (size_t)wgs_per_cu();
    size_t nsplit = std::max<size_t>(1, target / cols);
    nsplit = std::min(nsplit, std::max<size_t>(1, keys / ((mx ? 1 : 2) * iter_rows)));
    nsplit = std::min(nsplit, (size_t)kMaxSplits);
    // Fewer than kMinSplitKeys keys stay in one split: the merge launch then costs more
    // than the split saves (Qwen3 width at 101 keys: one split 6.5 us; three 5.5 us plus
    // a 3 us merge in the kernel trace).
    if (keys < kMinSplitKeys) nsplit = 1;
    // An iteration's loads address a window of iter_rows * nsplit cache rows from one
    // base with 32-bit offsets: keep the window under 2^30 bytes.
    const size_t row_bytes = hkv * hd * sizeof(float);
    while (nsplit > 1 && iter_rows * nsplit * row_bytes > ((size_t)1 << 30)) nsplit /= 2;
    p.nsplit = (int)nsplit;
    return p;
}

template <int HD, int G, int EB, bool SHORT>
hipError_t launch_lanes(hipStream_t st, const DecodePlan &p, const DecodeArgs &a) {
    using S = DecodeShapeOf<HD, G, EB, SHORT>;
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    if (S::LDS_BYTES > 64 * 1024)
        std::call_once(once, [&] {
            attr_err = hipFuncSetAttribute(
                reinterpret_cast<const void *>(&decode_kernel<HD, G, EB, SHORT>),
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::LDS_BYTES);
        });
    if (attr_err != hipSuccess) return attr_err;
    dim3 grid((unsigned)(a.hkv * p.nsub), (unsigned)p.nsplit);
    decode_kernel<HD, G, EB, SHORT><<<grid, kThreads, S::LDS_BYTES, st>>>(a);
    return hipSuccess;
}

template <int HD, int G, int EB>
hipError_t launch_g(hipStream_t st, const DecodePlan &p, const DecodeArgs &a) {
    if constexpr (use_mx<HD, EB>()) {
        using M = MxShape<HD, G>;
        static_assert(M::LDS_BYTES <= 64 * 1024, "decode_mx_kernel LDS");
        dim3 grid((unsigned)(a.hkv * p.nsub), (unsigned)p.nsplit);
        if constexpr (HD == 128) {
            if (mx_streams_nt<HD>(a))
                decode_mx_kernel<HD, G, true><<<grid, kThreads, M::LDS_BYTES, st>>>(a);
            else
                decode_mx_kernel<HD, G, false><<<grid, kThreads, M::LDS_BYTES, st>>>(a);
        } else {
            decode_mx_kernel<HD, G, HD == 256><<<grid, kThreads, M::LDS_BYTES, st>>>(a);
        }
        return hipSuccess;
    }
    if constexpr (EB == 4 && HD == 256) {
        if (p.short_iter) return launch_lanes<HD, G, EB, true>(st, p, a);
    }
    return launch_lanes<HD, G, EB, false>(st, p, a);
}

template <int HD, int EB>
hipError_t launch_hd(hipStream_t st, const DecodePlan &p, const DecodeArgs &a) {
    hipError_t e;
    switch (p.G) {
        case 4: e = launch_g<HD, 4, EB>(st, p, a); break;
        case 2: e = launch_g<HD, 2, EB>(st, p, a); break;
        default: e = launch_g<HD, 1, EB>(st, p, a); break;
    }
    if (e != hipSuccess) return e;
    if (p.nsplit > 1) {
        constexpr int DS = merge_dims_per_block(HD);
        dim3 grid((unsigned)a.h, (unsigned)((HD + DS - 1) / DS));
        decode_merge_kernel<HD><<<grid, kThreads, 0, st>>>(a.part_acc, a.part_ml, a.o, a.h,
                                                          a.hkv, p.nsplit);
    }
    return hipSuccess;
}

template <int EB>
hipError_t launch_elem(hipStream_t st, size_t hd, const DecodePlan &p, const DecodeArgs &a) {
    if (hd == 4) {
        if constexpr (EB == 4) return launch_hd<4, 4>(st, p, a);  // f32 caches only
        return hipErrorInvalidValue;
    }
#define EB_LAUNCH_HD(D) \
    case D:             \
        if constexpr (D != 4) return launch_hd<D, EB>(st, p, a);
    switch (hd) {
        EB_HEAD_DIMS(EB_LAUNCH_HD)
        default: return hipErrorInvalidValue;
    }
#undef EB_LAUNCH_HD
    return hipErrorInvalidValue;
}

}  // namespace

namespace eb {

// Workspace layout (floats): part_acc [nsplit*h*hd] | part_ml [nsplit*h*2]. Every split
// writes its whole partial before the merge reads it, so no initialisation is needed.
// The figure is the cache type's own plan: the f32, IEEE-half and E4M3 plans hold
// different rows per iteration, and the narrow plans can take more splits (head_dim 256),
// so sizes handed to callers come from decode_workspace_floats_any, the largest.
size_t decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count,
                               CacheElem ce) {
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count, ce);
    if (p.nsplit <= 1) return 0;
    return (size_t)p.nsplit * h * (hd + 2);
}

size_t decode_workspace_floats_any(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count) {
    size_t n = decode_workspace_floats(h, hkv, pos, hd, cu_count, CacheElem::F32);
    if (hd >= 8) {
        n = std::max(n, decode_workspace_floats(h, hkv, pos, hd, cu_count, CacheElem::F16));
        n = std::max(n, decode_workspace_floats(h, hkv, pos, hd, cu_count, CacheElem::E4M3));
    }
    return n;
}

eb_status launch_attn_decode_any(hipStream_t st, const float *q, const void *kc, const void *vc,
                                 void *kc_w, void *vc_w, const float *knew, const float *vnew,
                                 float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                                 float scale, float *ws, size_t ws_floats, int cu_count,
                                 size_t window, CacheElem ce, const DecodePrologue *pro) {
    if (ce != CacheElem::F32 && hd < 8)
        return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: f16 and e4m3 caches need head_dim >= 8");
    if (pro && !knew) return fail(EB_OTHER, "attn_decode: the prologue needs the new rows");
    const size_t rope_row = pos;  // absolute position, before any window shift
    // A window is a shift of the cache view: keys first..=pos become keys 0..=pos-first of
    // caches based at row `first` (the fused write then lands on the same absolute row).
    if (window > 0 && pos + 1 > window) {
        const size_t first = pos + 1 - window;
        const size_t shift = first * hkv * hd * (size_t)ce;  // bytes
        kc = static_cast<const char *>(kc) + shift;
        vc = static_cast<const char *>(vc) + shift;
        if (kc_w) kc_w = static_cast<char *>(kc_w) + shift;
        if (vc_w) vc_w = static_cast<char *>(vc_w) + shift;
        pos -= first;
    }
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) |
         reinterpret_cast<uintptr_t>(vc) | reinterpret_cast<uintptr_t>(knew) |
         reinterpret_cast<uintptr_t>(vnew) | reinterpret_cast<uintptr_t>(o) |
         reinterpret_cast<uintptr_t>(ws)) & 15)
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_decode: q/caches/new rows/o/workspace must be 16-byte aligned");
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count, ce);
    const size_t need = decode_workspace_floats(h, hkv, pos, hd, cu_count, ce);
    if (need > 0 && (ws == nullptr || ws_floats < need))
        return fail(EB_SHAPE_MISMATCH, "attn_decode: workspace too small");
    DecodeArgs a{};
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.kc_w = kc_w;
    a.vc_w = vc_w;
    a.knew = knew;
    a.vnew = vnew;
    a.o = o;
    if (ws) {
        a.part_acc = ws;
        a.part_ml = ws + (size_t)p.nsplit * h * hd;
    }
    a.h = (int)h;
    a.hkv = (int)hkv;
    a.g = (int)(h / hkv);
    a.keys = (int)(pos + 1);
    a.nsplit = p.nsplit;
    a.scale_log2 = scale * kLog2e;
    if (pro) {
        a.prologue = true;
        a.qn_w = pro->q_norm;
        a.kn_w = pro->k_norm;
        a.vn_w = pro->v_norm;
        a.eps = pro->eps;
        a.rcos = pro->rope_cos;
        a.rsin = pro->rope_sin;
        a.rope_row = (int)rope_row;
        const float *ptrs[5] = {pro->q_norm, pro->k_norm, pro->v_norm, pro->rope_cos,
                                pro->rope_sin};
        for (const float *pp : ptrs)
            if (reinterpret_cast<uintptr_t>(pp) & 15)
                return fail(EB_UNSUPPORTED_CONFIG,
                            "attn_decode: norm gains and RoPE tables must be 16-byte aligned");
        if ((pro->rope_cos == nullptr) != (pro->rope_sin == nullptr))
            return fail(EB_OTHER, "attn_decode: RoPE needs both tables");
        if (pro->rope_cos && !decode_fuses_rope(hd, ce))
            return fail(EB_UNSUPPORTED_CONFIG,
                        "attn_decode: RoPE cannot be fused into the step at head_dim %zu over "
                        "a narrow cache (apply it with the pre-attention pass)", hd);
    }
    if (!attn_head_dim_supported(hd))
        return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: head_dim %zu", hd);
    const hipError_t e = ce == CacheElem::F16    ? launch_elem<2>(st, hd, p, a)
                         : ce == CacheElem::E4M3 ? launch_elem<1>(st, hd, p, a)
                                                 : launch_elem<4>(st, hd, p, a);
    if (e != hipSuccess) return eb::hip_fail(e, "attn_decode launch set-up");
    return check_launch("attn_decode");
}

eb_status launch_attn_decode(hipStream_t st, const float *q, const float *kc, const float *vc,
                             float *kc_w, float *vc_w, const float *knew, const float *vnew,
                             float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                             float scale, float *ws, size_t ws_floats, int cu_count,
                             size_t window) {
    return launch_attn_decode_any(st, q, kc, vc, kc_w, vc_w, knew, vnew, o, h, hkv, pos, hd,
                                  scale, ws, ws_floats, cu_count, window, CacheElem::F32,
                                  nullptr);
}

}  // namespace eb
