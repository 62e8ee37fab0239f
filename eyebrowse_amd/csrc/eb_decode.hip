// Batch-1 decode attention for gfx950: split-KV ("flash-decoding") over the seq-major
// cache [max_seq, Hkv, HD], then a log-sum-exp merge.
//
// Replaces attn_decode (crates/eyebrowse-kernels/src/attention.rs:52-90,124-162), which
// runs one thread per query head and streams the whole cache serially. Here the keys
// 0..=pos are cut into chunks; one 256-thread workgroup reduces one chunk for one KV head
// and the G query heads that share it (GQA: every K/V row is read once for all of them).
//
// Pass 1 (decode_split_kernel), per workgroup:
//  - a key row of HD floats is spread over LPK = HD/DPL lanes (DPL = 16 dims per lane),
//    so a wave covers KPW = 64/LPK keys per step; the loads are 128-bit and each
//    instruction's lanes cover contiguous 64-byte..1-KiB spans of the row;
//  - scores are lane-partial dot products summed across the LPK lanes with DPP;
//  - every lane group keeps an online softmax (running max m, sum l, acc[DPL]) in the
//    log2 domain (scores pre-multiplied by scale*log2(e), exponentials via v_exp_f32),
//    updating once per U keys;
//  - at the end the groups of a wave merge with lane shuffles, the 4 waves merge through
//    LDS, and the workgroup writes either the final row (one split) or its partial
//    (m, l, acc[HD]) per query head to the workspace.
// Pass 2 (decode_merge_kernel): o[h] = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M).
//
// The result equals softmax(scale * q K^T) V over keys 0..=pos; it differs from the
// reference's 3-pass f32 softmax only by rounding (summation order, exp2 vs expf).
#include "eb_common.h"
#include "eb_internal.h"

#include <algorithm>
#include <cstdlib>

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplits = 1024;

template <int HD>
struct DecodeShape {
    static constexpr int DPL = HD >= 16 ? 16 : HD;  // dims per lane
    static constexpr int LPK = HD / DPL;            // lanes per key row
    static constexpr int KPW = 64 / LPK;            // keys per wave step
    static constexpr int NV4 = DPL / 4;             // float4 loads per lane per row
    static constexpr int U = 2;                     // wave steps per softmax update
    static constexpr int KEYS_PER_ITER = kWaves * KPW * U;
    static_assert(DPL % 4 == 0 && LPK <= 16, "head_dim must be a multiple of 4, at most 256");
};

// Element offset (within a row) of float4 number i held by dim slice `ls`.
template <int HD>
__device__ __forceinline__ int dim_of(int i, int ls) {
    return (i * DecodeShape<HD>::LPK + ls) * 4;
}

template <int HD, int G>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    float *__restrict__ o, float *__restrict__ part_acc, float *__restrict__ part_ml, int h,
    int hkv, int g, int keys, int chunk, int nsplit, float scale_log2) {
    using S = DecodeShape<HD>;
    constexpr int U = S::U;
    constexpr int NV4 = S::NV4;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nsub = g / G;
    const int kvh = blockIdx.x / nsub;
    const int head0 = kvh * g + (blockIdx.x % nsub) * G;
    const int split = blockIdx.y;
    const int c0 = split * chunk;
    const int c1 = min(c0 + chunk, keys);
    const int kg = lane / S::LPK;
    const int ls = lane % S::LPK;

    float qr[G][S::DPL];
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            float4 t = *reinterpret_cast<const float4 *>(q + (size_t)(head0 + gi) * HD +
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

    const size_t row_stride = (size_t)hkv * HD;
    const float *kbase = kc + (size_t)kvh * HD;
    const float *vbase = vc + (size_t)kvh * HD;

    for (int base = c0; base < c1; base += S::KEYS_PER_ITER) {
        float4 kv[U][NV4], vv[U][NV4];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int key = base + (u * kWaves + wave) * S::KPW + kg;
            valid[u] = key < c1;
            int kk = valid[u] ? key : c1 - 1;
            const float *kp = kbase + (size_t)kk * row_stride;
            const float *vp = vbase + (size_t)kk * row_stride;
#pragma unroll
            for (int i = 0; i < NV4; ++i) {
                kv[u][i] = *reinterpret_cast<const float4 *>(kp + dim_of<HD>(i, ls));
                vv[u][i] = *reinterpret_cast<const float4 *>(vp + dim_of<HD>(i, ls));
            }
        }
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
                sc[u] = valid[u] ? s * scale_log2 : -INFINITY;
            }
            float mloc = sc[0];
#pragma unroll
            for (int u = 1; u < U; ++u) mloc = fmaxf(mloc, sc[u]);
            float mnew = fmaxf(m[gi], mloc);
            float mref = (mnew == -INFINITY) ? 0.0f : mnew;
            float corr = eb::fast_exp2(m[gi] - mref);
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
    }

    // Merge the KPW lane groups of this wave (lanes with equal `ls`).
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        float M = m[gi];
#pragma unroll
        for (int off = S::LPK; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
        float mref = (M == -INFINITY) ? 0.0f : M;
        float sc = eb::fast_exp2(m[gi] - mref);
        float L = l[gi] * sc;
#pragma unroll
        for (int off = S::LPK; off < 64; off <<= 1) L += __shfl_xor(L, off);
        l[gi] = L;
        m[gi] = M;
#pragma unroll
        for (int d = 0; d < S::DPL; ++d) {
            float a = acc[gi][d] * sc;
#pragma unroll
            for (int off = S::LPK; off < 64; off <<= 1) a += __shfl_xor(a, off);
            acc[gi][d] = a;
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
        float mref = (M == -INFINITY) ? 0.0f : M;
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            float sc = eb::fast_exp2(s_m[w][gi] - mref);
            L += s_l[w][gi] * sc;
            A += s_acc[w][gi][d] * sc;
        }
        const int hh = head0 + gi;
        if (nsplit == 1) {
            o[(size_t)hh * HD + d] = A / L;
        } else {
            part_acc[((size_t)split * h + hh) * HD + d] = A;
            if (d == 0) {
                part_ml[((size_t)split * h + hh) * 2 + 0] = M;
                part_ml[((size_t)split * h + hh) * 2 + 1] = L;
            }
        }
    }
}

// One block per query head: log-sum-exp merge of the split partials.
template <int HD>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float *__restrict__ part_acc,
                                                           const float *__restrict__ part_ml,
                                                           float *__restrict__ o, int h,
                                                           int nsplit) {
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_red[256];
    const int hh = blockIdx.x;
    const int tid = threadIdx.x;

    float M = -INFINITY;
    for (int s = tid; s < nsplit; s += 256) M = fmaxf(M, part_ml[((size_t)s * h + hh) * 2]);
    s_red[tid] = M;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (tid < stride) s_red[tid] = fmaxf(s_red[tid], s_red[tid + stride]);
        __syncthreads();
    }
    M = s_red[0];
    __syncthreads();
    float mref = (M == -INFINITY) ? 0.0f : M;
    float L = 0.0f;
    for (int s = tid; s < nsplit; s += 256) {
        float w = eb::fast_exp2(part_ml[((size_t)s * h + hh) * 2] - mref);
        s_w[s] = w;
        L += w * part_ml[((size_t)s * h + hh) * 2 + 1];
    }
    s_red[tid] = L;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (tid < stride) s_red[tid] += s_red[tid + stride];
        __syncthreads();
    }
    L = s_red[0];
    for (int d = tid; d < HD; d += 256) {
        float A = 0.0f;
        for (int s = 0; s < nsplit; ++s) A += part_acc[((size_t)s * h + hh) * HD + d] * s_w[s];
        o[(size_t)hh * HD + d] = A / L;
    }
}

struct DecodePlan {
    int G = 1;       // query heads per workgroup (a power of two dividing h/hkv)
    int nsub = 1;    // workgroups per KV head along the head axis
    int chunk = 0;   // keys per split
    int nsplit = 1;  // splits along the key axis
};

int keys_per_iter(size_t hd) {
    switch (hd) {
        case 4: return DecodeShape<4>::KEYS_PER_ITER;
        case 8: return DecodeShape<8>::KEYS_PER_ITER;
        case 16: return DecodeShape<16>::KEYS_PER_ITER;
        case 32: return DecodeShape<32>::KEYS_PER_ITER;
        case 64: return DecodeShape<64>::KEYS_PER_ITER;
        case 128: return DecodeShape<128>::KEYS_PER_ITER;
        default: return DecodeShape<256>::KEYS_PER_ITER;
    }
}

// Workgroups to aim for per CU: enough waves in flight to cover HBM latency.
int wgs_per_cu() {
    static int v = [] {
        const char *e = std::getenv("EB_DECODE_WGS_PER_CU");
        int x = e ? std::atoi(e) : 2;
        return (x >= 1 && x <= 64) ? x : 2;
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
    const size_t kpi = (size_t)keys_per_iter(hd);
    size_t target = (size_t)cu_count * (size_t)wgs_per_cu();
    size_t want = std::max<size_t>(1, target / cols);
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
void launch_split(hipStream_t st, const DecodePlan &p, const float *q, const float *kc,
                  const float *vc, float *o, float *pacc, float *pml, int h, int hkv, int g,
                  int keys, float scale_log2) {
    dim3 grid((unsigned)(hkv * p.nsub), (unsigned)p.nsplit);
    decode_split_kernel<HD, G><<<grid, kThreads, 0, st>>>(q, kc, vc, o, pacc, pml, h, hkv, g, keys,
                                                          p.chunk, p.nsplit, scale_log2);
}

template <int HD>
void launch_hd(hipStream_t st, const DecodePlan &p, const float *q, const float *kc,
               const float *vc, float *o, float *ws, int h, int hkv, int keys, float scale_log2) {
    const int g = h / hkv;
    float *pacc = ws;
    float *pml = ws ? ws + (size_t)p.nsplit * h * HD : nullptr;
    switch (p.G) {
        case 8: launch_split<HD, 8>(st, p, q, kc, vc, o, pacc, pml, h, hkv, g, keys, scale_log2); break;
        case 4: launch_split<HD, 4>(st, p, q, kc, vc, o, pacc, pml, h, hkv, g, keys, scale_log2); break;
        case 2: launch_split<HD, 2>(st, p, q, kc, vc, o, pacc, pml, h, hkv, g, keys, scale_log2); break;
        default: launch_split<HD, 1>(st, p, q, kc, vc, o, pacc, pml, h, hkv, g, keys, scale_log2); break;
    }
    if (p.nsplit > 1)
        decode_merge_kernel<HD><<<(unsigned)h, 256, 0, st>>>(pacc, pml, o, h, p.nsplit);
}

}  // namespace

namespace eb {

size_t decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count) {
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count);
    if (p.nsplit <= 1) return 0;
    return (size_t)p.nsplit * h * (hd + 2);
}

eb_status launch_attn_decode(hipStream_t st, const float *q, const float *kc, const float *vc,
                             float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                             float scale, float *ws, size_t ws_floats, int cu_count) {
    DecodePlan p = plan_decode(h, hkv, pos, hd, cu_count);
    if (p.nsplit > 1 && (ws == nullptr || ws_floats < (size_t)p.nsplit * h * (hd + 2)))
        return fail(EB_SHAPE_MISMATCH, "attn_decode: workspace too small");
    const float sl2 = scale * kLog2e;
    const int hi = (int)h, hk = (int)hkv, keys = (int)(pos + 1);
    switch (hd) {
        case 4: launch_hd<4>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 8: launch_hd<8>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 16: launch_hd<16>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 32: launch_hd<32>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 64: launch_hd<64>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 128: launch_hd<128>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        case 256: launch_hd<256>(st, p, q, kc, vc, o, ws, hi, hk, keys, sl2); break;
        default: return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: head_dim %zu", hd);
    }
    return check_launch("attn_decode");
}

}  // namespace eb
