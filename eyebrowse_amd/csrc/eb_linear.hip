// linear_f16w for gfx950: y[m, o] = sum_k x[m, k] * w[o, k], x and y f32, w IEEE half.
//
// Replaces linear_f16w (crates/eyebrowse-kernels/src/matmul.rs:84-144), a 16x16-tiled
// scalar GEMM that unpacks two halves per u32 word. The weight layout is the reference's:
// the logical [out, in] matrix flattened row-major, two halves per 32-bit word, low half
// first (crates/eyebrowse-gpu/src/tensor.rs:6-23); read as little-endian 16-bit units it
// is a plain half array, which is how the kernels address it.
//
// Two regimes:
//  - Few rows (decode, m <= kLinearGemvRows): HBM-bound on the weight (2*in*out bytes per
//    launch). One wave per kRowsPerWave output features (one per wave below 16384
//    features); lanes stride the contraction in 16-byte chunks (8 halves), each chunk
//    reused for every x row; the multiply-adds read the halves directly (v_fma_mix_f32)
//    and accumulate in f32. A wave reduction ends it.
//  - Many rows (prefill): matrix cores. The weight is exactly representable in f16, so
//    only x needs care: each x row is scaled by a power of two 2^-e (its largest
//    magnitude lands in [2^14, 2^15)) and split into x_hi = f16(x') and
//    x_lo = f16(x' - x_hi). Then x' = x_hi + x_lo to about 2^-22 relative, every product
//    x_hi*w and x_lo*w is exact in f32, and two v_mfma_f32_32x32x16_f16 per 32x32x16
//    block accumulate them in f32. The output is multiplied back by 2^e (ldexp). This
//    runs on the f16 matrix cores (2.5 PFLOP/s dense) at about f32 accuracy, where an
//    FP32-MFMA GEMM would be capped at 157 TFLOP/s. A pre-pass writes the row exponents.
//    Rows whose largest magnitude is not finite keep e = 0 and so give a non-finite
//    result, as the f32 product would.
// A scalar kernel covers shapes the vector paths do not (in % 8 != 0, unaligned
// pointers), like the reference's odd-width test (matmul.rs:255-272).
//
// Up to three (weight, output) pairs that share x run in one launch: q/k/v projections
// of one layer read the normalised hidden state once per tile instead of three times.
#include "eb_common.h"
#include "eb_internal.h"

#include <algorithm>
#include <cstdint>
#include <climits>
#include <mutex>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct LinearSegs {
    const _Float16 *w[eb::kLinearMaxSegs];
    float *y[eb::kLinearMaxSegs];
    int n[eb::kLinearMaxSegs];      // output features of each pair
    int first[eb::kLinearMaxSegs + 1];  // first work unit of each pair; first[nseg] = total
    int nseg;
};

// The pair that owns work unit u (units are numbered pair by pair).
__device__ __forceinline__ int seg_of(const LinearSegs &s, int u) {
    int i = 0;
#pragma unroll
    for (int j = 1; j < eb::kLinearMaxSegs; ++j) i += (j < s.nseg && u >= s.first[j]) ? 1 : 0;
    return i;
}

__device__ __forceinline__ float wave_sum(float v) {
    v = eb::group_sum<16>(v);
    v += eb::lane_xor16(v);
    v += eb::lane_xor32(v);
    return v;
}

// ---------------------------------------------------------------- few rows ------------
constexpr int kRowsPerWave = 4;   // output features per wave
// Fewer output features than this many waves' worth (at kRowsPerWave each, i.e. below
// 16384 features) run one feature per wave, so that the launch still spreads over the
// chip: the Qwen o_proj (1024 features, in 2048) is 64 workgroups at four features per
// wave and 256 at one. A feature's sum is the same either way (the same lanes, chunks and
// reduction), so the results are bit-identical. Measured (us per launch, 64 launches per
// graph, one box; four -> one feature per wave): Qwen o_proj 3.45 -> 2.53, q_proj 2.85 ->
// 2.28, k/v_proj 2.82 -> 2.19, o_proj at 4 rows 6.63 -> 4.50, Mistral k_proj 4.66 -> 3.22,
// o_proj 8.42 -> 8.14, fused q/k/v (6144 features) 10.9 -> 10.5, a 4096-row head 3.08 ->
// 2.86. The Qwen LM head (151936 features) keeps four: one measured 44.1 -> 72.0, and
// two / eight 50.6 / 47.9 against four's 43.5 (the Mistral head, 32768 x 4096: 41.0 / 60.8
// against 39.6).
#ifndef EB_GEMV_ONE_ROW_UNITS
#define EB_GEMV_ONE_ROW_UNITS 4096
#endif
constexpr int kGemvOneRowUnits = EB_GEMV_ONE_ROW_UNITS;
// 16-byte weight chunks per lane in flight per feature. Rows of up to 1024 halves take one
// per pass: the Qwen LM head (in 1024) read at 5.0 TB/s with 4 (half of them clamped
// repeats of the row's last chunk), 6.3 TB/s with 2 and 6.9 TB/s with 1; 8 features per
// wave at 1 or 2 chunks measured 6.1-6.3. Longer rows keep 4: at in 4096 (the Mistral LM
// head) 4 chunks read 6.39 TB/s, 2 chunks 5.93 and 1 chunk 6.22.
constexpr int gemv_unroll(int k) { return k <= 1024 ? 1 : 4; }

// MR: capacity in x rows (the launch passes m <= MR). Requires in % 8 == 0 and 16-byte
// aligned x, w and rows (in % 8 == 0 keeps every row start aligned).
template <int MR, int kChunkUnroll, int RPW = kRowsPerWave>
__global__ __launch_bounds__(kThreads) void linear_gemv_kernel(const float *__restrict__ x,
                                                               LinearSegs s, int m, int K) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int unit = blockIdx.x * kWaves + wave;  // a group of RPW features
    if (unit >= s.first[s.nseg]) return;          // whole waves only; no barriers below
    const int sg = seg_of(s, unit);
    const int N = s.n[sg];
    const int o0 = (unit - s.first[sg]) * RPW;
    const _Float16 *w = s.w[sg];
    const int k8 = K / 8;

    float acc[RPW][MR];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int i = 0; i < MR; ++i) acc[r][i] = 0.0f;

    for (int c0 = 0; c0 < k8; c0 += 64 * kChunkUnroll) {
        // All weight loads of the step first (clamped addresses, masked values), non-temporal:
        // each weight is read once per launch (the Qwen LM head, 311 MB: 4.78 -> 5.07 TB/s).
        f16x8 wv[kChunkUnroll][RPW];
#pragma unroll
        for (int u = 0; u < kChunkUnroll; ++u) {
            const int c = c0 + u * 64 + lane;
            const int cc = c < k8 ? c : k8 - 1;
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int o = min(o0 + r, N - 1);
                wv[u][r] = __builtin_nontemporal_load(
                    reinterpret_cast<const f16x8 *>(w + (size_t)o * K + (size_t)cc * 8));
            }
        }
#pragma unroll
        for (int u = 0; u < kChunkUnroll; ++u) {
            const int c = c0 + u * 64 + lane;
            if (c >= k8) break;
#pragma unroll
            for (int i = 0; i < MR; ++i) {
                if (i >= m) break;
                const f32x4 xa = *reinterpret_cast<const f32x4 *>(x + (size_t)i * K + c * 8);
                const f32x4 xb = *reinterpret_cast<const f32x4 *>(x + (size_t)i * K + c * 8 + 4);
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const f16x8 h = wv[u][r];
                    float t = acc[r][i];
                    t += xa.x * (float)h[0];
                    t += xa.y * (float)h[1];
                    t += xa.z * (float)h[2];
                    t += xa.w * (float)h[3];
                    t += xb.x * (float)h[4];
                    t += xb.y * (float)h[5];
                    t += xb.z * (float)h[6];
                    t += xb.w * (float)h[7];
                    acc[r][i] = t;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            const float v = wave_sum(acc[r][i]);
            if (lane == 0 && i < m && o0 + r < N) s.y[sg][(size_t)i * N + o0 + r] = v;
        }
}

template <int U, int RPW>
void launch_gemv(unsigned blocks, hipStream_t st, const float *x, const LinearSegs &s, int m,
                 int K) {
    if (m <= 1)
        linear_gemv_kernel<1, U, RPW><<<blocks, kThreads, 0, st>>>(x, s, m, K);
    else if (m <= 2)
        linear_gemv_kernel<2, U, RPW><<<blocks, kThreads, 0, st>>>(x, s, m, K);
    else if (m <= 4)
        linear_gemv_kernel<4, U, RPW><<<blocks, kThreads, 0, st>>>(x, s, m, K);
    else
        linear_gemv_kernel<(int)eb::kLinearGemvRows, U, RPW><<<blocks, kThreads, 0, st>>>(x, s, m, K);
}

// ---------------------------------------------------------------- any shape -----------
// One thread per output element, k ascending: the reference's order of summation.
__global__ __launch_bounds__(kThreads) void linear_scalar_kernel(const float *__restrict__ x,
                                                                 LinearSegs s, int m, int K) {
    const size_t idx = (size_t)blockIdx.x * kThreads + threadIdx.x;
    int sg = 0;
    size_t base = 0;
    for (; sg < s.nseg; ++sg) {
        const size_t cnt = (size_t)m * s.n[sg];
        if (idx < base + cnt) break;
        base += cnt;
    }
    if (sg >= s.nseg) return;
    const int N = s.n[sg];
    const size_t e = idx - base;
    const int i = (int)(e / N);
    const int o = (int)(e % N);
    const _Float16 *wr = s.w[sg] + (size_t)o * K;
    const float *xr = x + (size_t)i * K;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc += xr[k] * (float)wr[k];
    s.y[sg][(size_t)i * N + o] = acc;
}

// ---------------------------------------------------------------- many rows -----------
// Row exponents: ex[i] = e_i (as a float), e_i such that the row's largest magnitude
// times 2^-e_i lies in [2^14, 2^15) (e_i = 0 for zero or non-finite rows). One wave per
// row. Scaling uses ldexp (one rounding, no intermediate overflow), so e_i may exceed the
// exponent range of a single f32 scale factor (rows of subnormals need 2^163).
// With zero_out, the wave also zeroes its row of every output (for the split-contraction
// GEMM, whose halves add into y).
__global__ __launch_bounds__(kThreads) void linear_row_scale_kernel(const float *__restrict__ x,
                                                                    float *__restrict__ ex,
                                                                    int M, int K, LinearSegs s,
                                                                    bool zero_out) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= M) return;
    if (zero_out) {
        for (int g = 0; g < s.nseg; ++g) {
            float *yr = s.y[g] + (size_t)row * s.n[g];
            for (int c = lane; c < s.n[g]; c += 64) yr[c] = 0.0f;
        }
    }
    const float *xr = x + (size_t)row * K;
    float mx = 0.0f;
    float bad = 0.0f;  // becomes NaN (and stays NaN) once a NaN or inf is seen
    for (int c = lane; c < K / 4; c += 64) {  // K % 8 == 0 on this path
        const f32x4 v = *reinterpret_cast<const f32x4 *>(xr + 4 * c);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        bad += 0.0f * ((v.x + v.y) + (v.z + v.w));
    }
    mx = eb::class_reduce<1, true>(mx);
    bad = eb::class_reduce<1, false>(bad);
    int e = 0;
    if (bad == 0.0f && mx > 0.0f) e = ilogbf(mx) - 14;
    if (lane == 0) ex[row] = (float)e;
}

constexpr int kBM = 128;  // x rows per workgroup tile
#ifndef EB_LINEAR_BK
#define EB_LINEAR_BK 32
#endif
constexpr int kBK = EB_LINEAR_BK;  // contraction per LDS stage
// Shortest contraction cut in two halves when the 128 x 128 tiles alone leave CUs idle.
#ifndef EB_LINEAR_KSPLIT_MIN
#define EB_LINEAR_KSPLIT_MIN 1024
#endif
constexpr int kLdsRow = kBK + 8;  // halves per LDS row (16-byte pad against bank conflicts)
constexpr int kXcds = 8;  // MI355X: workgroup ids are dealt round-robin to 8 XCDs

template <int WNB>
struct GemmShape {
    static constexpr int BN = 64 * WNB;  // features per workgroup tile
    static constexpr int BUF = (2 * kBM + BN) * kLdsRow;  // halves: x_hi, x_lo, w
};
template <int WNB, int NBUF>
constexpr size_t gemm_lds_bytes() {
    return (size_t)NBUF * GemmShape<WNB>::BUF * 2;
}

__device__ __forceinline__ floatx16 mfma16(f16x8 a, f16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Requires in % 8 == 0 and 16-byte aligned x and w. Tile t: m-tile t / ntn, n-unit
// t % ntn (n-units numbered pair by pair). Workgroup ids are remapped so that each XCD
// works on a contiguous range of tiles (the same x rows), which its own L2 then keeps.
// WNB: 32-feature blocks per wave (the workgroup tile is 128 rows x 64*WNB features);
// NBUF: LDS buffers per stage (2: double buffered, one barrier per stage; 1: two
// barriers, half the LDS); MINB: workgroups per CU the registers must allow.
// ksplit 2: the contraction is cut in two halves, workgroups ids [tiles, 2*tiles) taking
// the second; each half adds its (scaled) partial into y, which the row-scale pre-pass
// zeroes first.
// Two addends onto zero give the same bits in either order (0 + a + b = a + b = b + a).
template <int WNB, int NBUF, int MINB>
__global__ __launch_bounds__(kThreads, MINB) void linear_gemm_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ ex,
                                                               LinearSegs s, int M, int K,
                                                               int ksplit) {
    using Sh = GemmShape<WNB>;
    constexpr int BN = Sh::BN;
    extern __shared__ _Float16 lds[];
    __shared__ int s_ex[kBM];  // row exponents of the tile (read by the epilogue)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nt = gridDim.x / ksplit;
    const int bid = blockIdx.x % nt;
    const int half = blockIdx.x / nt;
    const int full = (nt / kXcds) * kXcds;
    const int t = bid < full ? (bid % kXcds) * (nt / kXcds) + bid / kXcds : bid;
    const int ntn = s.first[s.nseg];
    const int mt = t / ntn;
    const int nu = t % ntn;
    const int sg = seg_of(s, nu);
    const int N = s.n[sg];
    const int m0 = mt * kBM;
    const int n0 = (nu - s.first[sg]) * BN;
    const _Float16 *w = s.w[sg];
    if (tid < kBM) s_ex[tid] = (int)ex[min(m0 + tid, M - 1)];

    // Staging assignment: x tile kBM x kBK f32 (NX f32x4 per thread); w tile BN x kBK
    // halves (NW f16x8 per thread).
    constexpr int X4 = kBK / 4, W8 = kBK / 8;  // vectors per tile row
    constexpr int NX = kBM * X4 / kThreads, NW = BN * W8 / kThreads;
    f32x4 rx[NX];
    f16x8 rw[NW];
    int rs[NX];  // -e of the row each staged f32x4 belongs to
#pragma unroll
    for (int j = 0; j < NX; ++j) {
        const int idx = tid + j * kThreads;
        const int row = min(m0 + idx / X4, M - 1);
        rs[j] = -(int)ex[row];
    }
    // Whole contraction stages and buffers below 2 GiB (every model's projections): raw
    // buffer loads, the lane's byte offset computed once and the stage's as a scalar; rows
    // past M (x) or N (w) lie past the buffer's end and read as zeros. Otherwise clamped,
    // selected loads.
    const bool fast = K % kBK == 0 && (size_t)M * K * 4 <= (size_t)INT_MAX &&
                      (size_t)N * K * 2 <= (size_t)INT_MAX;
    const __amdgpu_buffer_rsrc_t xres = eb::make_rsrc(x, fast ? M * K * 4 : 0);
    const __amdgpu_buffer_rsrc_t wres = eb::make_rsrc(w, fast ? N * K * 2 : 0);
    unsigned xoff[NX], woff[NW];
#pragma unroll
    for (int j = 0; j < NX; ++j) {
        const int idx = tid + j * kThreads;
        xoff[j] = ((unsigned)(m0 + idx / X4) * (unsigned)K + (unsigned)(idx % X4) * 4u) * 4u;
    }
#pragma unroll
    for (int j = 0; j < NW; ++j) {
        const int idx = tid + j * kThreads;
        woff[j] = ((unsigned)(n0 + idx / W8) * (unsigned)K + (unsigned)(idx % W8) * 8u) * 2u;
    }
    auto load_stage = [&](int k0) {
        if (fast) {
            const int kx = __builtin_amdgcn_readfirstlane(4 * k0);  // (uniform: scalar)
            const int kw = __builtin_amdgcn_readfirstlane(2 * k0);
#pragma unroll
            for (int j = 0; j < NX; ++j)
                rx[j] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, (int)xoff[j], kx, 0));
#pragma unroll
            for (int j = 0; j < NW; ++j)
                rw[j] = __builtin_bit_cast(
                    f16x8, __builtin_amdgcn_raw_buffer_load_b128(wres, (int)woff[j], kw, 0));
            return;
        }
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int idx = tid + j * kThreads;
            const int r = idx / X4, c4 = idx % X4;
            const int row = m0 + r, k = k0 + c4 * 4;
            const bool ok = row < M && k < K;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(
                x + (size_t)min(row, M - 1) * K + (ok ? k : 0));
            rx[j] = ok ? v : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int idx = tid + j * kThreads;
            const int r = idx / W8, c8 = idx % W8;
            const int o = n0 + r, k = k0 + c8 * 8;
            const bool ok = o < N && k < K;
            const f16x8 v = *reinterpret_cast<const f16x8 *>(
                w + (size_t)min(o, N - 1) * K + (ok ? k : 0));
            rw[j] = ok ? v : f16x8{};
        }
    };
    auto store_stage = [&](int buf) {
        _Float16 *hi = lds + buf * Sh::BUF;
        _Float16 *lo = hi + kBM * kLdsRow;
        _Float16 *wt = lo + kBM * kLdsRow;
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int idx = tid + j * kThreads;
            const int r = idx / X4, c4 = idx % X4;
            const f32x4 v = {ldexpf(rx[j].x, rs[j]), ldexpf(rx[j].y, rs[j]),
                             ldexpf(rx[j].z, rs[j]), ldexpf(rx[j].w, rs[j])};
            const f16x4 h = __builtin_convertvector(v, f16x4);
            const f16x4 l = __builtin_convertvector(v - __builtin_convertvector(h, f32x4), f16x4);
            *reinterpret_cast<f16x4 *>(hi + r * kLdsRow + c4 * 4) = h;
            *reinterpret_cast<f16x4 *>(lo + r * kLdsRow + c4 * 4) = l;
        }
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            const int idx = tid + j * kThreads;
            const int r = idx / W8, c8 = idx % W8;
            *reinterpret_cast<f16x8 *>(wt + r * kLdsRow + c8 * 8) = rw[j];
        }
    };

    // Wave (wm, wn) computes rows wm*64..+64 and features wn*32*WNB..+32*WNB of the tile:
    // 2 x WNB blocks of 32 x 32.
    const int wm = wave >> 1, wn = wave & 1;
    floatx16 acc[2][WNB];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < WNB; ++b) acc[a][b] = floatx16{};

    auto compute = [&](int buf) {
        const _Float16 *hi = lds + buf * Sh::BUF;
        const _Float16 *lo = hi + kBM * kLdsRow;
        const _Float16 *wt = lo + kBM * kLdsRow;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int kof = kk * 16 + (lane >> 5) * 8;
            f16x8 ah[2], al[2], bw[WNB];
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                const int r = wm * 64 + a * 32 + (lane & 31);
                ah[a] = *reinterpret_cast<const f16x8 *>(hi + r * kLdsRow + kof);
                al[a] = *reinterpret_cast<const f16x8 *>(lo + r * kLdsRow + kof);
            }
#pragma unroll
            for (int b = 0; b < WNB; ++b) {
                const int r = wn * 32 * WNB + b * 32 + (lane & 31);
                bw[b] = *reinterpret_cast<const f16x8 *>(wt + r * kLdsRow + kof);
            }
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < WNB; ++b) {
                    acc[a][b] = mfma16(ah[a], bw[b], acc[a][b]);
                    acc[a][b] = mfma16(al[a], bw[b], acc[a][b]);
                }
        }
    };

    // This workgroup's stages: all of them, or one half of the contraction.
    const int nst_all = (K + kBK - 1) / kBK;
    const int per = (nst_all + ksplit - 1) / ksplit;
    const int st0 = half * per;
    const int nst = min(nst_all - st0, per);
    load_stage(st0 * kBK);
    store_stage(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        if (st + 1 < nst) load_stage((st0 + st + 1) * kBK);
        if constexpr (NBUF == 2) {
            compute(st & 1);
            if (st + 1 < nst) store_stage((st & 1) ^ 1);
            __syncthreads();
        } else {
            compute(0);
            if (st + 1 < nst) {
                __syncthreads();  // every wave is done reading the buffer
                store_stage(0);
                __syncthreads();
            }
        }
    }

    // Epilogue: lane holds feature j = lane % 32 of each block, rows
    // 8*(r/4) + 4*(lane/32) + r%4; scale back and store (32 consecutive features per row).
    float *y = s.y[sg];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < WNB; ++b) {
            const int o = n0 + wn * 32 * WNB + b * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rt = wm * 64 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int row = m0 + rt;
                if (row < M && o < N) {
                    const float v = ldexpf(acc[a][b][r], s_ex[rt]);
                    if (ksplit == 1)
                        y[(size_t)row * N + o] = v;
                    else
                        atomicAdd(y + (size_t)row * N + o, v);
                }
            }
        }
}

// CUs of the current device (cached per device ordinal).
int current_cu_count() {
    static std::mutex mu;
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if (cache[dev] == 0) {
        int n = 0;
        cache[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                          hipSuccess && n > 0)
                         ? n
                         : 256;
    }
    return cache[dev];
}

// ksplit 2 expects the outputs zeroed (linear_row_scale_kernel's zero_out).
template <int WNB, int NBUF, int MINB>
eb_status launch_gemm(hipStream_t st, const float *x, const float *ex, LinearSegs s,
                      const size_t *out_f, int nseg, size_t m, size_t in_f, int ksplit = 1) {
    constexpr int BN = GemmShape<WNB>::BN;
    constexpr size_t lds_bytes = gemm_lds_bytes<WNB, NBUF>();
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
        attr_err = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&linear_gemm_kernel<WNB, NBUF, MINB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
    });
    if (attr_err != hipSuccess) return eb::hip_fail(attr_err, "hipFuncSetAttribute(linear)");
    s.first[0] = 0;
    for (int i = 0; i < nseg; ++i)
        s.first[i + 1] = s.first[i] + (int)((out_f[i] + BN - 1) / BN);
    const size_t tiles = (size_t)((m + kBM - 1) / kBM) * (size_t)s.first[nseg];
    linear_gemm_kernel<WNB, NBUF, MINB><<<(unsigned)(tiles * ksplit), kThreads, lds_bytes, st>>>(
        x, ex, s, (int)m, (int)in_f, ksplit);
    return eb::check_launch("linear_f16w");
}

__global__ __launch_bounds__(kThreads) void zero_fill_kernel(float *__restrict__ y, size_t n) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = 0.0f;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

namespace eb {

size_t linear_workspace_floats(size_t m, size_t in_f) {
    return (m > kLinearGemvRows && in_f % 8 == 0) ? m : 0;
}

eb_status launch_linear_f16w_multi(hipStream_t st, const float *x, const uint16_t *const *w,
                                   float *const *y, const size_t *out_f, int nseg, size_t m,
                                   size_t in_f, float *ws, size_t ws_floats) {
    if (nseg < 1 || nseg > kLinearMaxSegs) return fail(EB_OTHER, "linear: 1..3 weights");
    if (m == 0) return ok();
    bool vec = in_f % 8 == 0 && aligned16(x);
    size_t total_out = 0;
    for (int i = 0; i < nseg; ++i) {
        vec = vec && aligned16(w[i]);
        total_out += out_f[i];
    }
    if (total_out == 0) return ok();
    if (in_f == 0) {  // empty sums: zeros (a kernel, not a memset, so graphs may hold it)
        for (int i = 0; i < nseg; ++i) {
            const size_t n = m * out_f[i];
            if (n == 0) continue;
            zero_fill_kernel<<<(unsigned)std::min<size_t>((n + kThreads - 1) / kThreads, 4096),
                               kThreads, 0, st>>>(y[i], n);
        }
        return check_launch("linear_f16w");
    }
    LinearSegs s{};
    s.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        s.w[i] = reinterpret_cast<const _Float16 *>(w[i]);
        s.y[i] = y[i];
        s.n[i] = (int)out_f[i];
    }
    if (!vec) {
        const size_t elems = m * total_out;
        linear_scalar_kernel<<<(unsigned)((elems + kThreads - 1) / kThreads), kThreads, 0, st>>>(
            x, s, (int)m, (int)in_f);
        return check_launch("linear_f16w");
    }
    if (m <= kLinearGemvRows) {
        size_t units4 = 0;
        for (int i = 0; i < nseg; ++i) units4 += (out_f[i] + kRowsPerWave - 1) / kRowsPerWave;
        const int rpw = units4 < (size_t)kGemvOneRowUnits ? 1 : kRowsPerWave;
        s.first[0] = 0;
        for (int i = 0; i < nseg; ++i)
            s.first[i + 1] = s.first[i] + (int)((out_f[i] + rpw - 1) / rpw);
        const unsigned blocks = (unsigned)((s.first[nseg] + kWaves - 1) / kWaves);
        const int mi = (int)m;
        const bool one = gemv_unroll((int)in_f) == 1;
        if (rpw == 1) {
            if (one) launch_gemv<1, 1>(blocks, st, x, s, mi, (int)in_f);
            else launch_gemv<4, 1>(blocks, st, x, s, mi, (int)in_f);
        } else {
            if (one) launch_gemv<1, kRowsPerWave>(blocks, st, x, s, mi, (int)in_f);
            else launch_gemv<4, kRowsPerWave>(blocks, st, x, s, mi, (int)in_f);
        }
        return check_launch("linear_f16w");
    }
    if (ws == nullptr || ws_floats < m) return fail(EB_SHAPE_MISMATCH, "linear: workspace too small");
    // Wide tiles (64 x 128 per wave: 0.5 LDS fragment reads per MFMA instead of 0.75) when
    // they still give every CU two workgroups; otherwise 128 x 128 tiles, whose twice as
    // many workgroups keep more of the chip busy. With at most one 128 x 128 tile per CU
    // (o_proj-like shapes: many rows, few features), long contractions are cut in two
    // halves, doubling the workgroups; the pre-pass then zeroes the outputs they add into.
    const size_t mtiles = (m + kBM - 1) / kBM;
    size_t wide_units = 0, units = 0;
    for (int i = 0; i < nseg; ++i) {
        wide_units += (out_f[i] + GemmShape<4>::BN - 1) / GemmShape<4>::BN;
        units += (out_f[i] + GemmShape<2>::BN - 1) / GemmShape<2>::BN;
    }
    const size_t cus = (size_t)current_cu_count();
    const bool wide = mtiles * wide_units >= 2 * cus;
    const int ksplit =
        (!wide && mtiles * units <= cus && in_f >= (size_t)EB_LINEAR_KSPLIT_MIN) ? 2 : 1;
    linear_row_scale_kernel<<<(unsigned)((m + kWaves - 1) / kWaves), kThreads, 0, st>>>(
        x, ws, (int)m, (int)in_f, s, ksplit > 1);
    if (wide) return launch_gemm<4, 1, 2>(st, x, ws, s, out_f, nseg, m, in_f);
    return launch_gemm<2, 2, 1>(st, x, ws, s, out_f, nseg, m, in_f, ksplit);
}

}  // namespace eb
