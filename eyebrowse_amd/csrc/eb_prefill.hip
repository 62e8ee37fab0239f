// Causal GQA flash-attention prefill for gfx950 on FP32 matrix cores.
//
// Replaces attn_prefill (crates/eyebrowse-kernels/src/attention.rs:10-50,94-120), which
// runs one thread per (query row, head) and re-reads K/V from memory for every row.
//
// Layout of the work
//  - A workgroup is 4 waves; each wave owns 32 query rows of one head. The workgroup covers
//    HPW heads of one KV group (GQA: the K/V tiles it stages are shared by all of them)
//    and 32 * 4/HPW consecutive query rows.
//  - K and V tiles of 32 keys are staged in LDS (double buffered: the next tile is
//    fetched into registers while the current one is in use).
//  - Everything is computed transposed so that the query index sits on the lane:
//      S^T[key][query] = K Q^T         (v_mfma_f32_32x32x2_f32, contraction over head_dim)
//      O^T[d][query]  += V^T P^T       (same instruction, contraction over the 32 keys)
//    The S^T accumulator holds, per lane, 16 keys of one query, which is exactly the B
//    operand layout the PV product needs, so P never leaves registers, and the online
//    softmax state (running max m, partial sum l) is a per-lane scalar.
//  - The contraction indices are permuted freely (a sum does not care about order): lane
//    half hf reads head dims [hf*HD/2, (hf+1)*HD/2) for QK^T, and the PV step t pairs keys
//    8*(t/4) + 4*hf + t%4 with the S^T registers that hold them.
//  - Softmax runs in the log2 domain: scores are multiplied by scale*log2(e) and
//    exponentiated with v_exp_f32. Only the diagonal tile of each wave is masked; tiles
//    past the wave's last query are skipped.
//  - Workgroups are numbered so the longest query blocks start first and so consecutive
//    workgroup ids (which the dispatcher spreads over the 8 XCDs) walk across KV groups:
//    with 8 groups each XCD keeps one group's K/V in its own L2.
//
// FLOPs per launch: 2*H*HD*T*(T+1) algorithmic (QK^T and PV over the causal pairs); the
// kernel issues MFMA work for whole 32x32 tiles, i.e. slightly more on the diagonal.
#include "eb_common.h"
#include "eb_internal.h"

#include <cstdlib>
#include <mutex>
#include <string>

// Workgroups the compiler must fit per CU for head_dim <= 128 (bounds registers per wave:
// 2 four-wave workgroups = 2 waves per SIMD). head_dim 256 keeps one: its Q fragment and
// O^T accumulators alone take 256 registers per lane.
#ifndef EB_PREFILL_MIN_BLOCKS
#define EB_PREFILL_MIN_BLOCKS 2
#endif

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTile = 32;  // keys per tile, queries per wave

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int HD>
struct PrefillShape {
    static constexpr int KS = HD + 4;          // K row stride in LDS (floats), bank spread
    static constexpr int HALF = HD / 2;        // QK^T contraction steps per lane half
    static constexpr int NB = HD >= 32 ? HD / 32 : 1;  // 32-row blocks of O^T
    static constexpr int TILE_F4 = kTile * HD / 4;     // float4 per K (or V) tile
    static constexpr int NLD = (TILE_F4 + kThreads - 1) / kThreads;
    static constexpr size_t LDS_BYTES = (size_t)(2 * kTile * KS + 2 * kTile * HD) * sizeof(float);
};

// Query block processed by workgroup `flat`. Rank r = flat / ngroups runs over the query
// blocks of every KV group; ranks are dealt in passes of `pass` ranks (one workgroup per
// CU per pass). Even passes go heaviest first; odd passes run in reverse, so the two
// workgroups a CU holds at once (from passes 0 and 1) add up to the same causal work.
__device__ __forceinline__ int prefill_block_of(int flat, int ngroups, int nqb, int pass) {
    const int rank = flat / ngroups;
    if (pass <= 0) return nqb - 1 - rank;
    const int round = rank / pass;
    const int first = round * pass;
    const int count = min(pass, nqb - first);
    const int order = (round & 1) ? first + (count - 1 - (rank - first)) : rank;
    return nqb - 1 - order;
}

template <int HD, int HPW>
__global__ __launch_bounds__(kThreads, (HD <= 128 ? EB_PREFILL_MIN_BLOCKS : 1)) void prefill_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ o, int H, int Hkv, int T, float scale_log2, int nqb, int ngroups,
    int pass) {
    using S = PrefillShape<HD>;
    constexpr int WPH = 4 / HPW;    // waves per head
    constexpr int QB = kTile * WPH; // query rows per workgroup
    constexpr int HALF = S::HALF;
    constexpr int NB = S::NB;
    constexpr int KS = S::KS;

    extern __shared__ float smem[];
    float *Ks = smem;                    // [2][32][KS]
    float *Vs = smem + 2 * kTile * KS;   // [2][32][HD]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hf = lane >> 5;
    const int col = lane & 31;
    const int g = H / Hkv;
    const int gsub = g / HPW;
    const int flat = blockIdx.x;
    const int grp = flat % ngroups;
    const int qb = prefill_block_of(flat, ngroups, nqb, pass);
    const int kvh = grp / gsub;
    const int head = kvh * g + (grp % gsub) * HPW + wave / WPH;
    const int q0 = qb * QB + (wave % WPH) * kTile;
    const int wg_last = min(qb * QB + QB, T) - 1;
    const int ntiles = wg_last / kTile + 1;
    const int my_tiles = q0 < T ? q0 / kTile + 1 : 0;
    const int qi = q0 + col;

    // Q fragment: query qi, head dims [HALF*hf, HALF*hf + HALF).
    float qreg[HALF];
    {
        const bool qv = qi < T;
        const float *qp = q + ((size_t)(qv ? qi : 0) * H + head) * HD + HALF * hf;
        if constexpr (HALF % 4 == 0) {
#pragma unroll
            for (int i = 0; i < HALF / 4; ++i) {
                float4 t = qv ? *reinterpret_cast<const float4 *>(qp + 4 * i)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
                qreg[4 * i + 0] = t.x;
                qreg[4 * i + 1] = t.y;
                qreg[4 * i + 2] = t.z;
                qreg[4 * i + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int s = 0; s < HALF; ++s) qreg[s] = qv ? qp[s] : 0.0f;
        }
    }

    floatx16 oacc[NB];
#pragma unroll
    for (int mb = 0; mb < NB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[mb][r] = 0.0f;
    float m = -INFINITY;
    float l = 0.0f;

    float4 rk[S::NLD], rv[S::NLD];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int r = 0; r < S::NLD; ++r) {
            const int idx = tid + r * kThreads;
            if (idx < S::TILE_F4) {
                const int row = idx / (HD / 4);
                const int c4 = idx % (HD / 4);
                const int key = kb + row;
                if (key < T) {
                    const size_t off = ((size_t)key * Hkv + kvh) * HD + c4 * 4;
                    rk[r] = *reinterpret_cast<const float4 *>(k + off);
                    rv[r] = *reinterpret_cast<const float4 *>(v + off);
                } else {
                    rk[r] = make_float4(0.f, 0.f, 0.f, 0.f);
                    rv[r] = rk[r];
                }
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int r = 0; r < S::NLD; ++r) {
            const int idx = tid + r * kThreads;
            if (idx < S::TILE_F4) {
                const int row = idx / (HD / 4);
                const int c4 = idx % (HD / 4);
                *reinterpret_cast<float4 *>(Ks + (buf * kTile + row) * KS + c4 * 4) = rk[r];
                *reinterpret_cast<float4 *>(Vs + (buf * kTile + row) * HD + c4 * 4) = rv[r];
            }
        }
    };

    load_tile(0);
    store_tile(0);
    __syncthreads();

    for (int it = 0; it < ntiles; ++it) {
        const int buf = it & 1;
        const int kb = it * kTile;
        if (it + 1 < ntiles) load_tile(kb + kTile);

        if (it < my_tiles) {
            // S^T = K Q^T for this tile: 16 keys x 1 query per lane.
            floatx16 sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
            const float *kr = Ks + (buf * kTile + col) * KS + HALF * hf;
            if constexpr (HALF % 4 == 0) {
#pragma unroll
                for (int i = 0; i < HALF / 4; ++i) {
                    float4 a = *reinterpret_cast<const float4 *>(kr + 4 * i);
                    sacc = mfma32(a.x, qreg[4 * i + 0], sacc);
                    sacc = mfma32(a.y, qreg[4 * i + 1], sacc);
                    sacc = mfma32(a.z, qreg[4 * i + 2], sacc);
                    sacc = mfma32(a.w, qreg[4 * i + 3], sacc);
                }
            } else {
#pragma unroll
                for (int s = 0; s < HALF; ++s) sacc = mfma32(kr[s], qreg[s], sacc);
            }

            // Online softmax over this tile's keys (log2 domain).
            const bool diag = (kb == q0);
            float p[16];
            float mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kb + 8 * (r >> 2) + 4 * hf + (r & 3);
                float x = sacc[r] * scale_log2;
                if (diag && key > qi) x = -INFINITY;
                p[r] = x;
                mt = fmaxf(mt, x);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mnew = fmaxf(m, mt);
            const float corr = eb::fast_exp2(m - mnew);
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = eb::fast_exp2(p[r] - mnew);
                ps += p[r];
            }
            l = l * corr + ps;
            m = mnew;
#pragma unroll
            for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[mb][r] *= corr;

            // O^T += V^T P^T: step t pairs key 8*(t/4) + 4*hf + t%4 with p[t].
            const float *vt = Vs + buf * kTile * HD;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int kl = 8 * (t >> 2) + 4 * hf + (t & 3);
                const float *vp = vt + kl * HD;
                if constexpr (NB == 8) {
                    float4 a0 = *reinterpret_cast<const float4 *>(vp + 8 * col);
                    float4 a1 = *reinterpret_cast<const float4 *>(vp + 8 * col + 4);
                    oacc[0] = mfma32(a0.x, p[t], oacc[0]);
                    oacc[1] = mfma32(a0.y, p[t], oacc[1]);
                    oacc[2] = mfma32(a0.z, p[t], oacc[2]);
                    oacc[3] = mfma32(a0.w, p[t], oacc[3]);
                    oacc[4] = mfma32(a1.x, p[t], oacc[4]);
                    oacc[5] = mfma32(a1.y, p[t], oacc[5]);
                    oacc[6] = mfma32(a1.z, p[t], oacc[6]);
                    oacc[7] = mfma32(a1.w, p[t], oacc[7]);
                } else if constexpr (NB == 4) {
                    float4 a = *reinterpret_cast<const float4 *>(vp + 4 * col);
                    oacc[0] = mfma32(a.x, p[t], oacc[0]);
                    oacc[1] = mfma32(a.y, p[t], oacc[1]);
                    oacc[2] = mfma32(a.z, p[t], oacc[2]);
                    oacc[3] = mfma32(a.w, p[t], oacc[3]);
                } else if constexpr (NB == 2) {
                    float2 a = *reinterpret_cast<const float2 *>(vp + 2 * col);
                    oacc[0] = mfma32(a.x, p[t], oacc[0]);
                    oacc[1] = mfma32(a.y, p[t], oacc[1]);
                } else if constexpr (HD >= 32) {
                    oacc[0] = mfma32(vp[col], p[t], oacc[0]);
                } else {
                    const float a = col < HD ? vp[col] : 0.0f;
                    oacc[0] = mfma32(a, p[t], oacc[0]);
                }
            }
        }

        if (it + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Normalise and store: lane holds O[qi][NB*c + mb] for c = 8*(r/4) + 4*hf + r%4.
    const float lt = l + __shfl_xor(l, 32);
    if (my_tiles > 0 && qi < T) {
        const float inv = 1.0f / lt;
        float *op = o + ((size_t)qi * H + head) * HD;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 8 * (r >> 2) + 4 * hf + (r & 3);
            if constexpr (NB == 8) {
                *reinterpret_cast<float4 *>(op + 8 * c) =
                    make_float4(oacc[0][r] * inv, oacc[1][r] * inv, oacc[2][r] * inv, oacc[3][r] * inv);
                *reinterpret_cast<float4 *>(op + 8 * c + 4) =
                    make_float4(oacc[4][r] * inv, oacc[5][r] * inv, oacc[6][r] * inv, oacc[7][r] * inv);
            } else if constexpr (NB == 4) {
                *reinterpret_cast<float4 *>(op + 4 * c) =
                    make_float4(oacc[0][r] * inv, oacc[1][r] * inv, oacc[2][r] * inv, oacc[3][r] * inv);
            } else if constexpr (NB == 2) {
                *reinterpret_cast<float2 *>(op + 2 * c) = make_float2(oacc[0][r] * inv, oacc[1][r] * inv);
            } else if constexpr (HD >= 32) {
                op[c] = oacc[0][r] * inv;
            } else {
                if (c < HD) op[c] = oacc[0][r] * inv;
            }
        }
    }
}

// Ranks per pass of the snake order: one workgroup per CU per pass. EB_PREFILL_ORDER=heavy
// turns the snake off (plain heaviest-first order).
int prefill_pass(int ngroups) {
    static const bool snake = [] {
        const char *e = std::getenv("EB_PREFILL_ORDER");
        return !(e && std::string(e) == "heavy");
    }();
    if (!snake) return 0;
    const int cus = eb::current_cu_count();
    return cus >= ngroups ? cus / ngroups : 1;
}

template <int HD, int HPW>
eb_status launch_prefill_t(hipStream_t st, const float *q, const float *k, const float *v,
                           float *o, int H, int Hkv, int T, float scale_log2) {
    constexpr int QB = kTile * (4 / HPW);
    const size_t lds = PrefillShape<HD>::LDS_BYTES;
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void *>(&prefill_kernel<HD, HPW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    });
    if (attr_err != hipSuccess) return eb::hip_fail(attr_err, "hipFuncSetAttribute(prefill)");
    const int g = H / Hkv;
    const int ngroups = Hkv * (g / HPW);
    const int nqb = (T + QB - 1) / QB;
    const unsigned blocks = (unsigned)(nqb * ngroups);
    prefill_kernel<HD, HPW><<<blocks, kThreads, lds, st>>>(q, k, v, o, H, Hkv, T, scale_log2, nqb,
                                                          ngroups, prefill_pass(ngroups));
    return eb::check_launch("attn_prefill");
}

template <int HD>
eb_status launch_prefill_hd(hipStream_t st, const float *q, const float *k, const float *v,
                            float *o, int H, int Hkv, int T, float scale_log2) {
    const int g = H / Hkv;
    if (g % 4 == 0) return launch_prefill_t<HD, 4>(st, q, k, v, o, H, Hkv, T, scale_log2);
    if (g % 2 == 0) return launch_prefill_t<HD, 2>(st, q, k, v, o, H, Hkv, T, scale_log2);
    return launch_prefill_t<HD, 1>(st, q, k, v, o, H, Hkv, T, scale_log2);
}

}  // namespace

namespace eb {

eb_status launch_attn_prefill(hipStream_t st, const float *q, const float *k, const float *v,
                              float *o, size_t h, size_t hkv, size_t s, size_t hd,
                              float scale) {
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o)) & 15)
        return fail(EB_UNSUPPORTED_CONFIG, "attn_prefill: q/k/v/o must be 16-byte aligned");
    const float sl2 = scale * kLog2e;
    const int H = (int)h, Hk = (int)hkv, T = (int)s;
    switch (hd) {
        case 4: return launch_prefill_hd<4>(st, q, k, v, o, H, Hk, T, sl2);
        case 8: return launch_prefill_hd<8>(st, q, k, v, o, H, Hk, T, sl2);
        case 16: return launch_prefill_hd<16>(st, q, k, v, o, H, Hk, T, sl2);
        case 32: return launch_prefill_hd<32>(st, q, k, v, o, H, Hk, T, sl2);
        case 64: return launch_prefill_hd<64>(st, q, k, v, o, H, Hk, T, sl2);
        case 128: return launch_prefill_hd<128>(st, q, k, v, o, H, Hk, T, sl2);
        case 256: return launch_prefill_hd<256>(st, q, k, v, o, H, Hk, T, sl2);
        default: return fail(EB_UNSUPPORTED_CONFIG, "attn_prefill: head_dim %zu", hd);
    }
}

}  // namespace eb
