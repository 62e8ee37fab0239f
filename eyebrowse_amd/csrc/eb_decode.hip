// Batch-1 decode attention for gfx950: split-KV ("flash-decoding") over the seq-major
// cache [max_seq, Hkv, HD], then a log-sum-exp merge.
//
// Replaces attn_decode (crates/eyebrowse-kernels/src/attention.rs:52-90,124-162), which
// runs one thread per query head and streams the whole cache serially, and optionally
// folds in the two kv_write calls that precede it in Attention::decode
// (crates/eyebrowse-nn/src/attention.rs:149-183).
//
// Pass 1, grid (Hkv * nsub) x nsplit, 256 threads per workgroup. Workgroup (col, split)
// reduces keys [split*chunk, min((split+1)*chunk, pos+1)) for KV head col/nsub and the G
// query heads that share it (GQA: every K/V row is read once for all of them):
//  - a key row of HD floats is spread over LPK = HD/DPL lanes (DPL = 16 dims per lane),
//    so a wave covers KPW = 64/LPK keys per step; loads are 128-bit and each instruction's
//    lanes cover contiguous spans of the row;
//  - scores are lane-partial dot products summed across the LPK lanes with DPP;
//  - each lane group keeps an online softmax (running max m, sum l, acc[DPL]) in the log2
//    domain (scores times scale*log2(e), exponentials on v_exp_f32), updated once per U
//    keys;
//  - the wave's lane groups merge with shuffles, the 4 waves merge through LDS;
//  - with one split the workgroup writes o directly; otherwise it writes its partial
//    (m, l, acc[HD]) per head and pass 2 (decode_merge_kernel) computes
//    o = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M). A second launch is cheaper here
//    than merging in the last-arriving workgroup: on the 8-XCD part that needs an L2
//    write-back fence in every workgroup.
// Fused new-token write: when knew/vnew are given, key `pos` is read from them instead of
// the cache, and the workgroup whose chunk holds `pos` (first head-subgroup) copies them
// into cache row `pos`; nothing else touches that row in the launch, so the copy is exact
// and race free.
//
// The result is softmax(scale * q K^T) V over keys 0..=pos; it differs from the
// reference's 3-pass f32 softmax only by rounding (summation order, exp2 vs expf).
#include "eb_common.h"
#include "eb_internal.h"

#include <algorithm>
#include <cstdlib>

// Wave steps per softmax update: 4 when at most 2 query heads share a workgroup, else 2
// (register budget: the q fragment and accumulators grow with the head count). A
// positive EB_DECODE_U forces one value for all shapes.
#ifndef EB_DECODE_U
#define EB_DECODE_U 0
#endif
// 1: two register buffers per wave (next iteration's loads issued before the current one
// is consumed); 0: one buffer, latency hidden by other waves.
#ifndef EB_DECODE_PIPELINE
#define EB_DECODE_PIPELINE 1
#endif
// Workgroups per CU the register allocation must allow (launch-bounds minimum).
#ifndef EB_DECODE_MINB
#define EB_DECODE_MINB 1
#endif

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplits = 256;  // per column; bounds the merge's LDS weights

template <int HD, int G>
struct DecodeShape {
    static constexpr int DPL = HD >= 16 ? 16 : HD;  // dims per lane
    static constexpr int LPK = HD / DPL;            // lanes per key row
    static constexpr int KPW = 64 / LPK;            // keys per wave step
    static constexpr int NV4 = DPL / 4;             // float4 loads per lane per row
    static constexpr int U = EB_DECODE_U > 0 ? EB_DECODE_U : (G <= 2 ? 4 : 2);
    static constexpr int KEYS_PER_ITER = kWaves * KPW * U;
    static_assert(DPL % 4 == 0 && LPK <= 16, "head_dim must be a multiple of 4, at most 256");
};

// Element offset (within a row) of float4 number i held by dim slice `ls`.
template <int HD>
__device__ __forceinline__ int dim_of(int i, int ls) {
    return (i * DecodeShape<HD, 1>::LPK + ls) * 4;
}

struct DecodeArgs {
    const float *q;
    const float *kc;   // cache rows read (and row `pos` written when knew != null)
    const float *vc;
    float *kc_w;       // same as kc, writable
    float *vc_w;
    const float *knew; // [Hkv, HD] new token K (or null)
    const float *vnew;
    float *o;
    float *part_acc;   // [nsplit, h, HD]
    float *part_ml;    // [nsplit, h, 2]
    int h, hkv, g, keys, chunk, nsplit;
    float scale_log2;
};

template <int HD, int G>
__global__ __launch_bounds__(kThreads, EB_DECODE_MINB) void decode_kernel(DecodeArgs a) {
    using S = DecodeShape<HD, G>;
    constexpr int U = S::U;
    constexpr int NV4 = S::NV4;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nsub = a.g / G;
    const int col = blockIdx.x;
    const int kvh = col / nsub;
    const int head0 = kvh * a.g + (col % nsub) * G;
    const int split = blockIdx.y;
    const int c0 = split * a.chunk;
    const int c1 = min(c0 + a.chunk, a.keys);
    const int kg = lane / S::LPK;
    const int ls = lane % S::LPK;
    const int pos = a.keys - 1;
    const bool has_new = a.knew != nullptr;
    const size_t row_stride = (size_t)a.hkv * HD;

    // New-token write: one workgroup per KV head copies the row into the cache.
    if (has_new && (col % nsub) == 0 && pos >= c0 && pos < c1) {
        for (int i = threadIdx.x; i < HD / 4; i += kThreads) {
            const size_t dst = (size_t)pos * row_stride + (size_t)kvh * HD + 4 * i;
            *reinterpret_cast<float4 *>(a.kc_w + dst) =
                *reinterpret_cast<const float4 *>(a.knew + (size_t)kvh * HD + 4 * i);
            *reinterpret_cast<float4 *>(a.vc_w + dst) =
                *reinterpret_cast<const float4 *>(a.vnew + (size_t)kvh * HD + 4 * i);
        }
    }

    float qr[G][S::DPL];
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            float4 t = *reinterpret_cast<const float4 *>(a.q + (size_t)(head0 + gi) * HD +
                                                         dim_of<HD>(i, ls));
            qr[gi][4 * i + 0] = t.x;
            qr[gi][4 * i + 1] = t.y;
            qr[gi][4 * i + 2] = t.z;
            qr[gi][4 * i + 3] = t.w;
        }

    float m[G], l[G], acc[G][S::DPL];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
#pragma unroll
        for (int d = 0; d < S::DPL; ++d) acc[gi][d] = 0.0f;
    }

    const float *kbase = a.kc + (size_t)kvh * HD;
    const float *vbase = a.vc + (size_t)kvh * HD;

    // One iteration = U wave steps of KPW keys. Two register buffers: the next
    // iteration's K/V loads are issued before the current one is consumed, so the wave
    // keeps a full iteration of loads in flight while it computes.
    auto load_iter = [&](int base, float4 (&kv)[U][NV4], float4 (&vv)[U][NV4],
                         bool (&valid)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = base + (u * kWaves + wave) * S::KPW + kg;
            valid[u] = key < c1;
            const int kk = valid[u] ? key : c1 - 1;
            const float *kp = kbase + (size_t)kk * row_stride;
            const float *vp = vbase + (size_t)kk * row_stride;
            if (has_new && kk == pos) {
                kp = a.knew + (size_t)kvh * HD;
                vp = a.vnew + (size_t)kvh * HD;
            }
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                kv[u][i] = *reinterpret_cast<const float4 *>(kp + dim_of<HD>(i, ls));
                vv[u][i] = *reinterpret_cast<const float4 *>(vp + dim_of<HD>(i, ls));
            }
        }
    };
    auto consume_iter = [&](const float4 (&kv)[U][NV4], const float4 (&vv)[U][NV4],
                            const bool (&valid)[U]) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float sc[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < NV4; ++i) {
                    s += qr[gi][4 * i + 0] * kv[u][i].x;
                    s += qr[gi][4 * i + 1] * kv[u][i].y;
                    s += qr[gi][4 * i + 2] * kv[u][i].z;
                    s += qr[gi][4 * i + 3] * kv[u][i].w;
                }
                s = eb::group_sum<S::LPK>(s);
                sc[u] = valid[u] ? s * a.scale_log2 : -INFINITY;
            }
            float mloc = sc[0];
#pragma unroll
            for (int u = 1; u < U; ++u) mloc = fmaxf(mloc, sc[u]);
            const float mnew = fmaxf(m[gi], mloc);
            const float mref = (mnew == -INFINITY) ? 0.0f : mnew;
            const float corr = eb::fast_exp2(m[gi] - mref);
            float p[U];
            float psum = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                p[u] = eb::fast_exp2(sc[u] - mref);
                psum += p[u];
            }
            l[gi] = l[gi] * corr + psum;
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                float a0 = acc[gi][4 * i + 0] * corr, a1 = acc[gi][4 * i + 1] * corr;
                float a2 = acc[gi][4 * i + 2] * corr, a3 = acc[gi][4 * i + 3] * corr;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    a0 += p[u] * vv[u][i].x;
                    a1 += p[u] * vv[u][i].y;
                    a2 += p[u] * vv[u][i].z;
                    a3 += p[u] * vv[u][i].w;
                }
                acc[gi][4 * i + 0] = a0;
                acc[gi][4 * i + 1] = a1;
                acc[gi][4 * i + 2] = a2;
                acc[gi][4 * i + 3] = a3;
            }
            m[gi] = mnew;
        }
    };

    if constexpr (!EB_DECODE_PIPELINE) {
        for (int base = c0; base < c1; base += S::KEYS_PER_ITER) {
            float4 kv[U][NV4], vv[U][NV4];
            bool ok[U];
            load_iter(base, kv, vv, ok);
            consume_iter(kv, vv, ok);
        }
    } else {
        float4 kA[U][NV4], vA[U][NV4], kB[U][NV4], vB[U][NV4];
        bool okA[U], okB[U];
        // Counted loop over pairs of iterations with unconditional loads: a load issued
        // under a branch would be sunk by the compiler next to its use, draining the queue.
        // Iterations past c1 load clamped rows and are fully masked (valid = false), which
        // leaves the softmax state unchanged.
        const int n_iter = (c1 - c0 + S::KEYS_PER_ITER - 1) / S::KEYS_PER_ITER;
        load_iter(c0, kA, vA, okA);
        for (int it = 0; it < n_iter; it += 2) {
            load_iter(c0 + (it + 1) * S::KEYS_PER_ITER, kB, vB, okB);
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(kA, vA, okA);
            load_iter(c0 + (it + 2) * S::KEYS_PER_ITER, kA, vA, okA);
            __builtin_amdgcn_sched_barrier(0);
            consume_iter(kB, vB, okB);
        }
    }

    // Merge the KPW lane groups of this wave (lanes with equal `ls`).
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        float M = m[gi];
#pragma unroll
        for (int off = S::LPK; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float mref = (M == -INFINITY) ? 0.0f : M;
        const float sc = eb::fast_exp2(m[gi] - mref);
        float L = l[gi] * sc;
#pragma unroll
        for (int off = S::LPK; off < 64; off <<= 1) L += __shfl_xor(L, off);
        l[gi] = L;
        m[gi] = M;
#pragma unroll
        for (int d = 0; d < S::DPL; ++d) {
            float x = acc[gi][d] * sc;
#pragma unroll
            for (int off = S::LPK; off < 64; off <<= 1) x += __shfl_xor(x, off);
            acc[gi][d] = x;
        }
    }

    __shared__ float s_acc[kWaves][G][HD];
    __shared__ float s_m[kWaves][G];
    __shared__ float s_l[kWaves][G];
    if (kg == 0) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
#pragma unroll
            for (int i = 0; i < NV4; ++i)
#pragma unroll
                for (int c = 0; c < 4; ++c) s_acc[wave][gi][dim_of<HD>(i, ls) + c] = acc[gi][4 * i + c];
            if (ls == 0) {
                s_m[wave][gi] = m[gi];
                s_l[wave][gi] = l[gi];
            }
        }
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < G * HD; idx += kThreads) {
        const int gi = idx / HD;
        const int d = idx % HD;
        float M = s_m[0][gi];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][gi]);
        const float mref = (M == -INFINITY) ? 0.0f : M;
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float sc = eb::fast_exp2(s_m[w][gi] - mref);
            L += s_l[w][gi] * sc;
            A += s_acc[w][gi][d] * sc;
        }
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
// every XCD are visible without in-kernel fences): one 256-thread block per query head.
// Thread (grp, d), GROUPS = 256/HD groups, folds splits s = grp, grp + GROUPS, ... into a
// running (M, L, A) in batches of kBatch splits whose loads are all issued before any is
// used, so a merge costs about ceil(nsplit / (GROUPS * kBatch)) memory round trips. The
// groups then combine through LDS: o[h][d] = A / L.
template <int HD>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(const float *__restrict__ part_acc,
                                                                const float *__restrict__ part_ml,
                                                                float *__restrict__ o, int h,
                                                                int nsplit) {
    constexpr int GROUPS = HD >= kThreads ? 1 : kThreads / HD;
    constexpr int kBatch = 16;  // 32 splits (one workgroup per CU) merge in one round trip
    __shared__ float s_m[GROUPS][HD < kThreads ? HD : kThreads];
    __shared__ float s_l[GROUPS][HD < kThreads ? HD : kThreads];
    __shared__ float s_a[GROUPS][HD < kThreads ? HD : kThreads];
    const int hh = blockIdx.x;
    const int tid = threadIdx.x;
    const size_t stride_acc = (size_t)h * HD;
    const size_t stride_ml = (size_t)h * 2;

    for (int d0 = 0; d0 < HD; d0 += kThreads) {
        const int dl = tid % (HD < kThreads ? HD : kThreads);
        const int d = d0 + dl;
        const int grp = tid / (HD < kThreads ? HD : kThreads);
        float M = -INFINITY, L = 0.0f, A = 0.0f;
        if (grp < GROUPS && d < HD) {
            const float *pa = part_acc + (size_t)hh * HD + d;
            const float *pm = part_ml + (size_t)hh * 2;
            for (int s0 = grp; s0 < nsplit; s0 += GROUPS * kBatch) {
                float bm[kBatch], bl[kBatch], ba[kBatch];
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const int s = s0 + j * GROUPS;
                    const bool ok = s < nsplit;
                    bm[j] = ok ? pm[(size_t)s * stride_ml] : -INFINITY;
                    bl[j] = ok ? pm[(size_t)s * stride_ml + 1] : 0.0f;
                    ba[j] = ok ? pa[(size_t)s * stride_acc] : 0.0f;
                }
                float bM = bm[0];
#pragma unroll
                for (int j = 1; j < kBatch; ++j) bM = fmaxf(bM, bm[j]);
                const float Mn = fmaxf(M, bM);
                const float mref = (Mn == -INFINITY) ? 0.0f : Mn;
                const float c = eb::fast_exp2(M - mref);
                L *= c;
                A *= c;
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const float w = eb::fast_exp2(bm[j] - mref);
                    L += w * bl[j];
                    A += w * ba[j];
                }
                M = Mn;
            }
            s_m[grp][dl] = M;
            s_l[grp][dl] = L;
            s_a[grp][dl] = A;
        }
        __syncthreads();
        if (tid < (HD < kThreads ? HD : kThreads) && d < HD) {
            float Mt = s_m[0][tid];
#pragma unroll
            for (int g2 = 1; g2 < GROUPS; ++g2) Mt = fmaxf(Mt, s_m[g2][tid]);
            const float mref = (Mt == -INFINITY) ? 0.0f : Mt;
            float Lt = 0.0f, At = 0.0f;
#pragma unroll
            for (int g2 = 0; g2 < GROUPS; ++g2) {
                const float w = eb::fast_exp2(s_m[g2][tid] - mref);
                Lt += w * s_l[g2][tid];
                At += w * s_a[g2][tid];
            }
            o[(size_t)hh * HD + d] = At / Lt;
        }
        __syncthreads();
    }
}

struct DecodePlan {
    int G = 1;       // query heads per workgroup (a power of two dividing h/hkv, <= 8)
    int nsub = 1;    // workgroups per KV head along the head axis
    int chunk = 0;   // keys per split
    int nsplit = 1;  // splits along the key axis
};

template <int G>
int keys_per_iter_g(size_t hd) {
    switch (hd) {
        case 4: return DecodeShape<4, G>::KEYS_PER_ITER;
        case 8: return DecodeShape<8, G>::KEYS_PER_ITER;
        case 16: return DecodeShape<16, G>::KEYS_PER_ITER;
        case 32: return DecodeShape<32, G>::KEYS_PER_ITER;
        case 64: return DecodeShape<64, G>::KEYS_PER_ITER;
        case 128: return DecodeShape<128, G>::KEYS_PER_ITER;
        default: return DecodeShape<256, G>::KEYS_PER_ITER;
    }
}

int keys_per_iter(size_t hd, int G) {
    switch (G) {
        case 8: return keys_per_iter_g<8>(hd);
        case 4: return keys_per_iter_g<4>(hd);
        case 2: return keys_per_iter_g<2>(hd);
        default: return keys_per_iter_g<1>(hd);
    }
}

// Workgroups to aim for per CU: enough waves in flight to cover HBM latency.
int wgs_per_cu() {
    static int v = [] {
        const char *e = std::getenv("EB_DECODE_WGS_PER_CU");
        int x = e ? std::atoi(e) : 1;
        return (x >= 1 && x <= 64) ? x : 1;
    }();
    return v;
}

DecodePlan plan_decode(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count) {
    DecodePlan p;
    const size_t g = h / hkv;
    p.G = (g % 8 == 0) ? 8 : (g % 4 == 0) ? 4 : (g % 2 == 0) ? 2 : 1;
    p.nsub = (int)(g / p.G);
    const size_t keys = pos + 1;
    const size_t cols = hkv * (size_t)p.nsub;
    const size_t kpi = (size_t)keys_per_iter(hd, p.G);
    const size_t target = (size_t)cu_count * (size_t)wgs_per_cu();
    const size_t want = std::max<size_t>(1, target / cols);
    size_t chunk = (keys + want - 1) / want;
    chunk = std::max(kpi, (chunk + kpi - 1) / kpi * kpi);
    size_t nsplit = (keys + chunk - 1) / chunk;
    if (nsplit > (size_t)kMaxSplits) {
        chunk = (keys + kMaxSplits - 1) / kMaxSplits;
        chunk = (chunk + kpi - 1) / kpi * kpi;
        nsplit = (keys + chunk - 1) / chunk;
    }
    p.chunk = (int)chunk;
    p.nsplit = (int)nsplit;
    return p;
}

template <int HD, int G>
void launch_g(hipStream_t st, const DecodePlan &p, const DecodeArgs &a) {
    dim3 grid((unsigned)(a.hkv * p.nsub), (unsigned)p.nsplit);
    decode_kernel<HD, G><<<grid, kThreads, 0, st>>>(a);
}

template <int HD>
void launch_hd(hipStream_t st, const DecodePlan &p, const DecodeArgs &a) {
    switch (p.G) {
        case 8: launch_g<HD, 8>(st, p, a); break;
        case 4: launch_g<HD, 4>(st, p, a); break;
        case 2: launch_g<HD, 2>(st, p, a); break;
        default: launch_g<HD, 1>(st, p, a); break;
    }
    if (p.nsplit > 1)
        decode_merge_kernel<HD><<<(unsigned)a.h, kThreads, 0, st>>>(a.part_acc, a.part_ml, a.o,
                                                                    a.h, p.nsplit);
}

}  // namespace

namespace eb {

// Workspace layout (floats): part_acc [nsplit*h*hd] | part_ml [nsplit*h*2]. Every split
// writes its whole partial before the merge reads it, so no initialisation is needed.
size_t decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count) {
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count);
    if (p.nsplit <= 1) return 0;
    return (size_t)p.nsplit * h * (hd + 2);
}

eb_status launch_attn_decode(hipStream_t st, const float *q, const float *kc, const float *vc,
                             float *kc_w, float *vc_w, const float *knew, const float *vnew,
                             float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                             float scale, float *ws, size_t ws_floats, int cu_count) {
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) |
         reinterpret_cast<uintptr_t>(vc) | reinterpret_cast<uintptr_t>(knew) |
         reinterpret_cast<uintptr_t>(vnew)) & 15)
        return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: q/caches/new rows must be 16-byte aligned");
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count);
    const size_t need = decode_workspace_floats(h, hkv, pos, hd, cu_count);
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
    a.chunk = p.chunk;
    a.nsplit = p.nsplit;
    a.scale_log2 = scale * kLog2e;
    switch (hd) {
        case 4: launch_hd<4>(st, p, a); break;
        case 8: launch_hd<8>(st, p, a); break;
        case 16: launch_hd<16>(st, p, a); break;
        case 32: launch_hd<32>(st, p, a); break;
        case 64: launch_hd<64>(st, p, a); break;
        case 128: launch_hd<128>(st, p, a); break;
        case 256: launch_hd<256>(st, p, a); break;
        default: return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: head_dim %zu", hd);
    }
    return check_launch("attn_decode");
}

}  // namespace eb
