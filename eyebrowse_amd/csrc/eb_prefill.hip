// Causal GQA flash-attention prefill for gfx950 on the matrix cores.
//
// Replaces attn_prefill (crates/eyebrowse-kernels/src/attention.rs:10-50,94-120), which
// runs one thread per (query row, head) and re-reads K/V from memory for every row.
//
// Layout of the work
//  - Every wave owns 32 query rows of one head. A workgroup covers HPW heads of one KV
//    group (GQA: the K/V tiles it stages serve all of them), WPH consecutive 32-row query
//    sub-blocks per head (QB = 32*WPH rows), and splits the key range KSPLIT ways: wave
//    set ks takes key tiles t with t % KSPLIT == ks, and the KSPLIT partial softmax states
//    are merged through LDS at the end. Splitting the keys halves the longest per-wave
//    chain, so the causal triangle's big query blocks no longer set the kernel's length.
//  - Each step stages KSPLIT tiles of 32 keys (K and V) in LDS, double buffered: the next
//    step is fetched into registers while the current one is in use.
//  - Everything is computed transposed so that the query index sits on the lane:
//      S^T[key][query] = K Q^T         (contraction over head_dim)
//      O^T[d][query]  += V^T P^T       (contraction over the 32 keys of a tile)
//  - For head_dim >= 32 both run on the f16 matrix cores (v_mfma_f32_32x32x16_f16) at
//    about f32 accuracy (head_dim < 32 uses v_mfma_f32_32x32x2_f32 for both; at head_dim
//    256 the split fills 256 VGPRs and about 200 AGPRs, one wave per SIMD):
//      - every K, Q and V row is scaled by a power of two (its largest magnitude lands in
//        [2^14, 2^15)) and split exactly into hi = f16(x') and lo = f16(x' - hi), so
//        x' = hi + lo to about 2^-22; all-zero rows get an exponent below every real one;
//        rows holding inf or NaN keep exponent 0 and pass them on;
//      - K Q^T = hi*hi + hi*lo + lo*hi (lo*lo is below 2^-22 of the product), in f32;
//        each score is scaled back with ldexp by its key's and query's exponents;
//      - V is staged transposed ([head_dim][keys] halves) so that each lane's 8 keys of an
//        MFMA step are contiguous; P is scaled per key by 2^(ev_key - E) and split, where
//        E, per query, is the exponent of its largest term p * 2^ev_key: O^T accumulates
//        in units of 2^E (rescaled when E moves, with the softmax correction), so p' <= 1
//        and the largest terms keep the split's full precision;
//      - the reference max of the online softmax moves only when a score exceeds it by
//        more than kSlack, and the rescale of l and O^T is skipped for the whole wave
//        when no lane needs it.
//    The S^T accumulator holds, per lane, 16 keys of one query, which is exactly the B
//    operand layout the PV product needs, so P never leaves registers, and the online
//    softmax state (running max m, partial sum l) is a per-lane scalar.
//  - The contraction indices are permuted freely (a sum does not care about order): lane
//    half hf reads head dims [hf*HD/2, (hf+1)*HD/2) for QK^T, and the PV step t pairs keys
//    8*(t/4) + 4*hf + t%4 with the S^T registers that hold them.
//  - Softmax runs in the log2 domain: scores are multiplied by scale*log2(e) and
//    exponentiated with v_exp_f32. Only the diagonal tile of each wave is masked; tiles
//    past the wave's last query are skipped.
//  - Workgroups are numbered heaviest query block first, and consecutive workgroup ids
//    (which the dispatcher spreads over the 8 XCDs) walk across KV groups: with 8 groups
//    each XCD keeps one group's K/V in its own L2.
//
// FLOPs per launch: 2*H*HD*T*(T+1) algorithmic (QK^T and PV over the causal pairs); the
// kernel issues MFMA work for whole 32x32 tiles, i.e. slightly more on the diagonal.
#include "eb_common.h"
#include "eb_internal.h"

#include <algorithm>
#include <climits>
#include <mutex>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native 4-wide vector for staged K/V values. HIP's float4 is a class type: a conditional
// on it is lowered through a stack copy (scratch memory); this one stays in registers.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// x - f32(h), h the low (sub_f16_lo) or high (sub_f16_hi) half of a packed pair, in one
// mixed-precision fma (exact here: x - h fits f32 when h = f16(x)).
__device__ __forceinline__ float sub_f16_lo(unsigned h2, float x) {
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(x));
    return d;
}
__device__ __forceinline__ float sub_f16_hi(unsigned h2, float x) {
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(x));
    return d;
}

// 1: the f16 mode without key splits stores its output from registers and runs three
// waves per SIMD (FAST3, below); 0: the output goes through an LDS tile, two waves per SIMD.
#ifndef EB_PREFILL_FAST_OCC
#define EB_PREFILL_FAST_OCC 1
#endif
// 1: FAST3 over records keeps three LDS buffers, each step's copy issued two steps ahead.
#ifndef EB_PREFILL_FAST_TB
#define EB_PREFILL_FAST_TB 1
#endif

constexpr int kTile = 32;  // keys per tile, queries per wave
constexpr size_t kLdsBytesPerCu = 160 * 1024;  // gfx950 LDS per CU
constexpr float kSlack = 8.0f;  // log2 units the reference max may lag a score (SPV)
constexpr int kUnitSlack = 8;   // bits a P V term may exceed its query's O^T unit (SPV)

__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 mfma16(f16x8 a, f16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int HD, int HPW, int WPH, int KSPLIT>
struct PrefillCfg {
    static constexpr int HD_ = HD;
    static constexpr int NW = HPW * WPH * KSPLIT;  // waves per workgroup
    static constexpr int THREADS = NW * 64;
    static constexpr int QB = kTile * WPH;         // query rows per workgroup
    static constexpr int KS = HD + 4;              // K row stride in LDS (floats), bank spread
    static constexpr int HALF = HD / 2;            // QK^T contraction steps per lane half
    static constexpr int NB = HD >= 32 ? HD / 32 : 1;  // 32-row blocks of O^T
    static constexpr int STEP_KEYS = kTile * KSPLIT;   // keys staged per step
    static constexpr int STEP_F4 = STEP_KEYS * HD / 4;  // float4 per K (or V) step
    static constexpr int NLD = (STEP_F4 + THREADS - 1) / THREADS;
    // head_dim >= 32: Q K^T on the f16 matrix cores with an exact hi/lo split (K rows and
    // Q rows scaled by powers of two first); smaller head dims keep FP32 MFMA throughout.
    static constexpr bool SQK = HD >= 32;
    // V^T P^T the same way (V rows scaled and split at staging, stored transposed, hi
    // then lo halves; P scaled per key and split in registers).
    static constexpr bool SPV = HD >= 32;
    // Split tile images (SPV): 16-byte chunks laid out chunk-major (sk_chunk, sv_chunk): K
    // hi chunk c (dims 8c .. 8c + 7) of key r at c * KCS + r, the K lo chunks KC on; V^T hi
    // chunk c (keys 8c .. 8c + 7 in the permuted key order) of V^T row p at 2 KC + c * HD +
    // p, the V^T lo chunks 4 HD on; then the K exponents [32] and V exponents [32] at float
    // EXPO; whole KiB. An MFMA operand read then takes 256 contiguous bytes per 16 lanes (no
    // bank conflict) at immediate offsets. The K chunk columns are KCS = 33 chunks apart, so
    // that the staging writes of one key's chunks (16 consecutive lanes) also meet 16
    // different bank groups. A buffer holds KSPLIT images; a pre-split record is one image,
    // copied into LDS with memory-to-LDS loads.
    static constexpr int KCS = kTile + 1;
    static constexpr int KC = HD / 8 * KCS;               // chunks of the K hi (or lo) part
    static constexpr int EXPO = 4 * (2 * KC + 8 * HD);
    static constexpr int IMG = SPV ? (EXPO + 64 + 255) / 256 * 256 : 0;
    // head_dim < 32: K rows [STEP_KEYS][KS] and V rows [STEP_KEYS][HD], f32; whole KiB
    static constexpr int BUF =
        SPV ? KSPLIT * IMG : (STEP_KEYS * KS + STEP_KEYS * HD + 255) / 256 * 256;
    static constexpr int PS_FLOATS = IMG;  // floats per pre-split record
    // f16 mode (hi halves only): a buffer holds KSPLIT tile images of FIMG floats, each a
    // K part and a V^T part of 16-byte chunks (8 halves) laid out chunk-major: K chunk c
    // (dims 8c .. 8c + 7) of key r at chunk c * 32 + r, V^T chunk c (keys 8c .. 8c + 7 in
    // the permuted key order) of V^T row p at 4 HD + c * HD + p (fk_chunk, fv_chunk). An
    // MFMA operand read then takes 256 contiguous bytes per 16 lanes (no bank conflict,
    // no padding) at offsets that are immediates. The f16-mode records (head_dim <= 128)
    // are these images, copied into LDS with memory-to-LDS loads.
    static constexpr int FIMG = 32 * HD;
    static constexpr int FBUF = (STEP_KEYS / kTile) * FIMG;
    static constexpr int FPS_CH = FIMG / 4;              // chunks per record
    static constexpr int FPS_FLOATS = FIMG;
    static constexpr int REC = 3 + 16 * NB;  // merged fields per lane: m, l, V unit, O^T
    static constexpr int MERGE = (KSPLIT - 1) * HPW * WPH * REC * 64;  // floats
    static constexpr int OS = HD + 4;                  // output staging row stride (floats)
    static constexpr int OUT = HPW * WPH * kTile * OS; // output staging, one tile per slot
    static constexpr int LDS_FLOATS =
        (2 * BUF > MERGE ? 2 * BUF : MERGE) > OUT ? (2 * BUF > MERGE ? 2 * BUF : MERGE) : OUT;
    static constexpr size_t LDS_BYTES = (size_t)LDS_FLOATS * sizeof(float);
};

// Buffer size (floats) of the mode's LDS layout (FAST: tile images of hi halves).
template <class C, bool FAST>
constexpr int bufsize() { return FAST ? C::FBUF : C::BUF; }

// f16-mode tile images: the 16-byte chunk index of chunk c of K row r (key r, dims 8c ..
// 8c + 7), and of chunk c of V^T row p (keys 8c .. 8c + 7).
template <int HD>
__device__ __forceinline__ int fk_chunk(int r, int c) { return c * kTile + r; }
template <int HD>
__device__ __forceinline__ int fv_chunk(int p, int c) { return 4 * HD + c * HD + p; }
// Split tile images: the same for the hi (lo = 0) or lo (lo = 1) halves.
template <class C>
__device__ __forceinline__ int sk_chunk(int r, int c, int lo) { return lo * C::KC + c * C::KCS + r; }
template <class C>
__device__ __forceinline__ int sv_chunk(int p, int c, int lo) {
    return 2 * C::KC + lo * 4 * C::HD_ + c * C::HD_ + p;
}
// Image size of the mode (floats).
template <class C, bool FAST>
constexpr int imgsize() { return FAST ? C::FIMG : C::IMG; }

// Fetch the K and V rows [kb, kb + STEP_KEYS) of KV head kvh into registers; rows past
// T read as zero. Every element is assigned on every call (clamped addresses, selected
// values): conditionally written register arrays end up in scratch memory.
// EB: bytes per k/v element: 4 (f32), 2 (IEEE half) or 1 (OCP FP8 E4M3), converted to f32
// here (exactly).
template <class C, int EB, bool NT = false>
__device__ __forceinline__ void prefill_load_step(const void *__restrict__ k,
                                                  const void *__restrict__ v,
                                                  f32x4 (&rk)[C::NLD], f32x4 (&rv)[C::NLD],
                                                  int kb, int T, int Hkv, int kvh, int tid,
                                                  int hdr) {
    constexpr int HD = C::HD_;
#pragma unroll
    for (int r = 0; r < C::NLD; ++r) {
        const int idx = min(tid + r * C::THREADS, C::STEP_F4 - 1);
        const int row = idx / (HD / 4);
        const int c4 = idx % (HD / 4);
        const int key = kb + row;
        // rows of hdr <= HD dims (head dims padded up to the instantiation read as zeros)
        const bool in = key < T && (HD == 4 || c4 * 4 < hdr);
        const size_t off = ((size_t)min(key, T - 1) * Hkv + kvh) * hdr + min(c4 * 4, hdr - 4);
        f32x4 kx, vx;
        if constexpr (EB == 2) {
            kx = __builtin_convertvector(
                *reinterpret_cast<const f16x4 *>(static_cast<const _Float16 *>(k) + off), f32x4);
            vx = __builtin_convertvector(
                *reinterpret_cast<const f16x4 *>(static_cast<const _Float16 *>(v) + off), f32x4);
        } else if constexpr (EB == 1) {
            kx = eb::f8x4_to_f32(
                *reinterpret_cast<const unsigned *>(static_cast<const uint8_t *>(k) + off));
            vx = eb::f8x4_to_f32(
                *reinterpret_cast<const unsigned *>(static_cast<const uint8_t *>(v) + off));
        } else {
            const f32x4 *kp = reinterpret_cast<const f32x4 *>(static_cast<const float *>(k) + off);
            const f32x4 *vp = reinterpret_cast<const f32x4 *>(static_cast<const float *>(v) + off);
            kx = NT ? __builtin_nontemporal_load(kp) : *kp;
            vx = NT ? __builtin_nontemporal_load(vp) : *vp;
        }
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        rk[r] = in ? kx : z;
        rv[r] = in ? vx : z;
    }
}

// Write the staged rows into LDS buffer `buf`: K rows [STEP_KEYS][KS], then V rows
// [STEP_KEYS][HD].
// Largest value over aligned groups of N consecutive lanes (N a power of two, up to 64).
template <int N>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (N >= 2) x = fmaxf(x, eb::dpp<eb::kDppQuadXor1>(x));
    if constexpr (N >= 4) x = fmaxf(x, eb::dpp<eb::kDppQuadXor2>(x));
    if constexpr (N >= 8) x = fmaxf(x, eb::dpp<eb::kDppRowHalfMirror>(x));
    if constexpr (N >= 16) x = fmaxf(x, eb::dpp<eb::kDppRowMirror>(x));
    if constexpr (N >= 32) x = fmaxf(x, eb::lane_xor16(x));
    if constexpr (N >= 64) x = fmaxf(x, eb::lane_xor32(x));
    return x;
}

// The exponent e that brings a row whose largest magnitude is mx into [2^14, 2^15); 0 for
// rows holding inf (which then keep it), and kZeroRowExp for all-zero rows (masked or
// padding rows), below every real exponent so that a tile's largest exponent ignores
// them. (fmaxf drops NaN, so a NaN row gets the exponent of its other elements and still
// passes its NaN on.) frexp gives m * 2^k with m in [0.5, 1): the exponent is k - 1.
constexpr int kZeroRowExp = -200;  // (ev << 23 of every exponent fits an int)
__device__ __forceinline__ int split_exponent(float mx) {
    if (mx > 3.4028235e38f) return 0;
    return mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) - 15 : kZeroRowExp;
}

// The value held by lane i ^ N (N = 8, 16 or 32).
template <int N>
__device__ __forceinline__ unsigned lane_xor_u(unsigned x) {
    static_assert(N == 8 || N == 16 || N == 32, "8, 16 or 32");
    const float f = __builtin_bit_cast(float, x);
    if constexpr (N == 32) return __builtin_bit_cast(unsigned, eb::lane_xor32(f));
    else if constexpr (N == 16) return __builtin_bit_cast(unsigned, eb::lane_xor16(f));
    else return __builtin_bit_cast(unsigned, eb::dpp<0x128>(f));  // row_ror:8 = i ^ 8 in a row
}

// x' = x * 2^-e (exact), hi = f16(x'), lo = f16(x' - hi): x' = hi + lo to about 2^-22.
__device__ __forceinline__ void split_f16(f32x4 x, int e, f16x4 &hi, f16x4 &lo) {
    const f32x4 v = {ldexpf(x.x, -e), ldexpf(x.y, -e), ldexpf(x.z, -e), ldexpf(x.w, -e)};
    hi = __builtin_convertvector(v, f16x4);
    lo = __builtin_convertvector(v - __builtin_convertvector(hi, f32x4), f16x4);
}

// Write the staged rows into LDS buffer `buf`. SQK (head_dim >= 32): the split tile images
// (K rows scaled by their exponents and split into f16 hi and lo halves, V rows likewise
// and transposed, then both exponent arrays); otherwise f32 K rows [STEP_KEYS][KS], then
// V rows [STEP_KEYS][HD].
// FAST: rows are rounded to f16 as they are (no exponent, no lo halves, no exponent
// arrays) and written as the f16 mode's tile images (fk_chunk, fv_chunk).
// V16 (with FAST false): K split as above, V rows rounded to f16 as they are, as FAST does
// (the scores-accurate mode; its V^T lo halves and V exponents are not written).
template <class C, bool FAST = false, bool V16 = false>
__device__ __forceinline__ void prefill_store_step(float *smem, const f32x4 (&rk)[C::NLD],
                                                   const f32x4 (&rv)[C::NLD], int buf,
                                                   int tid) {
    constexpr int HD = C::HD_;
    constexpr int IMGX = imgsize<C, FAST>();
    float *Kb = smem + buf * bufsize<C, FAST>();
#pragma unroll
    for (int r = 0; r < C::NLD; ++r) {
        const int idx = tid + r * C::THREADS;
        const int row = idx / (HD / 4);
        const int c4 = idx % (HD / 4);
        if constexpr (C::SQK) {
            // HD/4 consecutive lanes hold one K row (every lane is in range for HD >= 32):
            // its tile's image is row / 32, its row there row % 32; halves 4 c4 .. 4 c4 + 3
            // are half of chunk c4 / 2.
            const f32x4 x = rk[r];
            float *img = Kb + (row / kTile) * IMGX;
            _Float16 *imh = reinterpret_cast<_Float16 *>(img);
            const int kr = row % kTile;
            if constexpr (FAST) {
                *reinterpret_cast<f16x4 *>(imh + 8 * fk_chunk<HD>(kr, c4 / 2) + (c4 & 1) * 4) =
                    __builtin_convertvector(x, f16x4);
            } else {
                const float m4 =
                    fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
                const float mx = group_max<HD / 4>(m4);
                const int e = split_exponent(mx);
                f16x4 hi, lo;
                split_f16(x, e, hi, lo);
                *reinterpret_cast<f16x4 *>(imh + 8 * sk_chunk<C>(kr, c4 / 2, 0) + (c4 & 1) * 4) = hi;
                *reinterpret_cast<f16x4 *>(imh + 8 * sk_chunk<C>(kr, c4 / 2, 1) + (c4 & 1) * 4) = lo;
                if (c4 == 0) reinterpret_cast<int *>(img + C::EXPO)[kr] = e;
            }
            const f32x4 y = rv[r];
            int ev = 0;
            f16x4 vh, vl;
            if constexpr (FAST || V16) {
                vh = __builtin_convertvector(y, f16x4);
                vl = vh;
            } else {
                const float vm4 =
                    fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
                ev = split_exponent(group_max<HD / 4>(vm4));
                split_f16(y, ev, vh, vl);
            }
            // V^T row of dim d is p(d) = (d % NB) * 32 + d / NB (the MFMA reader then walks
            // consecutive rows). Keys are stored permuted within each 16: groups of four in
            // the order 0, 2, 1, 3, so that the 8 keys one lane half feeds an MFMA step
            // (keys 16u + 4hf + 0..3 and 16u + 8 + 4hf + 0..3) fill one chunk.
            if constexpr (HD / 4 > 32) {
                // A row spans the whole wave (no partner row in it): halves one by one.
                const int g4s = (row >> 2) & 3;
                const int js = (row & ~15) | (((g4s & 1) << 1 | (g4s >> 1)) << 2) | (row & 3);
                _Float16 *vimg = reinterpret_cast<_Float16 *>(Kb + (js / kTile) * IMGX);
                const int jc = (js % kTile) / 8, jw = js % 8;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = c4 * 4 + i;
                    const int pr = (d % C::NB) * 32 + d / C::NB;
                    if constexpr (FAST) {
                        vimg[8 * fv_chunk<HD>(pr, jc) + jw] = vh[i];
                    } else {
                        vimg[8 * sv_chunk<C>(pr, jc, 0) + jw] = vh[i];
                        if constexpr (!V16) vimg[8 * sv_chunk<C>(pr, jc, 1) + jw] = vl[i];
                    }
                }
            } else {
                // Rows j and j + 1 (lanes i and i ^ HD/4) pair their halves: the even row's
                // lane writes dims 0, 1 of its four, the odd row's lane dims 2, 3, each as
                // one 32-bit (key j, key j + 1) word.
                using u32x2 = __attribute__((ext_vector_type(2))) unsigned;
                const u32x2 ho = __builtin_bit_cast(u32x2, vh), lw = __builtin_bit_cast(u32x2, vl);
                const u32x2 hp = {lane_xor_u<HD / 4>(ho.x), lane_xor_u<HD / 4>(ho.y)};
                const u32x2 lp = (FAST || V16) ? lw : u32x2{lane_xor_u<HD / 4>(lw.x), lane_xor_u<HD / 4>(lw.y)};
                const f16x4 vh2 = __builtin_bit_cast(f16x4, hp), vl2 = __builtin_bit_cast(f16x4, lp);
                const bool odd = row & 1;
                const int g4 = (row >> 2) & 3;
                const int j0 = (row & ~15) | (((g4 & 1) << 1 | (g4 >> 1)) << 2) | (row & 2);
                unsigned *vimg = reinterpret_cast<unsigned *>(Kb + (j0 / kTile) * IMGX);
                const int jc = (j0 % kTile) / 8, jw = (j0 % 8) / 2;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int i = odd ? 2 + t : t;  // which of the four dims
                    const int d = c4 * 4 + i;
                    const int pr = (d % C::NB) * 32 + d / C::NB;
                    const _Float16 he = odd ? vh2[i] : vh[i], ho2 = odd ? vh[i] : vh2[i];
                    const _Float16 le = odd ? vl2[i] : vl[i], lo2 = odd ? vl[i] : vl2[i];
                    using h2 = __attribute__((ext_vector_type(2))) _Float16;
                    if constexpr (FAST) {
                        vimg[4 * fv_chunk<HD>(pr, jc) + jw] = __builtin_bit_cast(unsigned, h2{he, ho2});
                    } else {
                        vimg[4 * sv_chunk<C>(pr, jc, 0) + jw] = __builtin_bit_cast(unsigned, h2{he, ho2});
                        if constexpr (!V16)
                            vimg[4 * sv_chunk<C>(pr, jc, 1) + jw] = __builtin_bit_cast(unsigned, h2{le, lo2});
                    }
                }
            }
            if (!FAST && !V16 && c4 == 0) reinterpret_cast<int *>(img + C::EXPO)[kTile + kr] = ev;
        } else if (idx < C::STEP_F4) {
            float *Vb = Kb + C::STEP_KEYS * C::KS;
            *reinterpret_cast<f32x4 *>(Kb + row * C::KS + c4 * 4) = rk[r];
            *reinterpret_cast<f32x4 *>(Vb + row * HD + c4 * 4) = rv[r];
        }
    }
}

// Copy NIMG tile images (records tile0 .. tile0 + NIMG - 1 of one KV head, recs, each
// clamped to the last record, nt - 1: a clamped image is never read) of IMGF floats into
// LDS at lds with memory-to-LDS loads: wave w moves KiB blocks w * BPW .. w * BPW + BPW - 1
// of each image (lane i bytes 16i .. 16i + 15 of a block), a load's immediate offset
// applying to both its global and its LDS address. Issued as inline assembly, which the
// compiler's wait counting does not see (it would otherwise wait for these loads before
// every read of the other buffer); the loads are complete after wait_vm_all(). m0 is a
// reserved register, so the compiler warns that it does not preserve it around the asm:
// the generated code of these kernels keeps no value of its own in m0 (in their gfx950
// assembly every m0 write is this asm's), so nothing else sees the clobber.
template <int IMGF, int NIMG, int NW>
__device__ __forceinline__ void img_copy(const float *__restrict__ recs, float *lds, int tile0,
                                         int nt, int wave, int lane) {
    constexpr int BLK = IMGF / 256;  // KiB blocks per image
    constexpr int BPW = (BLK + NW - 1) / NW;
    static_assert(IMGF % 256 == 0, "whole KiB images");
    const int j0 = wave * BPW;
#pragma unroll
    for (int k = 0; k < NIMG; ++k) {
        const int t = min(tile0 + k, nt - 1);
        const float *src = recs + (size_t)t * IMGF + j0 * 256 + lane * 4;
        const unsigned dst = __builtin_amdgcn_readfirstlane(
            (unsigned)(uintptr_t)(__attribute__((address_space(3))) float *)(lds + k * IMGF +
                                                                              j0 * 256));
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            if (BLK % NW == 0 || j0 + i < BLK)  // (uniform)
                asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off offset:%2"
                             :
                             : "s"(dst + 4096 * (i / 4)), "v"(src + 1024 * (i / 4)),
                               "i"(1024 * (i % 4))
                             : "memory", "m0");
        }
    }
}

// The pre-split and pre-convert passes' shape: one 32-key tile per workgroup (the records'
// layout), 512 threads at head_dim >= 128 (more of the tile's loads and stores in flight
// per CU: the LDS allows two such workgroups per CU at 256, four at 128; measured 1-2 %
// faster on 512- and 1024-row prompts, long prompts unchanged), 256 below.
template <int HD>
using PresplitCfg = PrefillCfg<HD, 4, HD >= 128 ? 2 : 1, 1>;

// Pre-convert pass of the f16 mode: workgroup (t, kvh) rounds keys [(tlo + t) * 32, +32) of KV
// head kvh to f16 as the f16 mode's staging does, and writes the tile's record.
template <int HD>
__global__ __launch_bounds__(PresplitCfg<HD>::THREADS) void preconvert_kernel(
    const float *__restrict__ k, const float *__restrict__ v, float *__restrict__ ps, int nkeys,
    int Hkv, int nt, int hdr) {
    using C = PresplitCfg<HD>;
    static_assert(HD <= 128, "f16-mode records for head_dim <= 128");
    __shared__ float smem[C::FBUF];
    const int t = blockIdx.x;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    f32x4 rk[C::NLD], rv[C::NLD];
    prefill_load_step<C, 4>(k, v, rk, rv, t * kTile, nkeys, Hkv, kvh, tid, hdr);
    prefill_store_step<C, true>(smem, rk, rv, 0, tid);
    __syncthreads();
    // (the tile image is the record)
    f32x4 *rec = reinterpret_cast<f32x4 *>(ps + ((size_t)kvh * nt + t) * C::FPS_FLOATS);
    for (int c = tid; c < C::FPS_CH; c += C::THREADS)
        rec[c] = reinterpret_cast<const f32x4 *>(smem)[c];
}

// Pre-split pass: workgroup (t, kvh) splits keys [(tlo + t) * 32, +32) of KV head kvh
// (rows past nkeys as zeros) exactly as the prefill's own staging does, and writes the
// tile's record. The prefill then only copies records into LDS: the split is done once
// per key instead of once per workgroup that reads the key.

// V16: records of the scores-accurate mode (V rows rounded to f16 as they are).
template <int HD, int EB, bool NT, bool V16 = false>
__global__ __launch_bounds__(PresplitCfg<HD>::THREADS) void presplit_kernel(
    const void *__restrict__ k, const void *__restrict__ v, float *__restrict__ ps, int nkeys,
    int Hkv, int tlo, int nt, int hdr) {
    using C = PresplitCfg<HD>;
    static_assert(C::SPV, "pre-split needs the split V path");
    static_assert(C::BUF == PrefillCfg<HD, 4, 1, 1>::BUF &&
                      C::PS_FLOATS == PrefillCfg<HD, 4, 1, 1>::PS_FLOATS,
                  "the records' layout is the 32-key step's");
    __shared__ float smem[C::BUF];
    const int t = blockIdx.x;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    // (The tile image is the record. Its padding past the exponents, and with V16 its V^T lo
    // halves and V exponents, are left as they are: nothing reads them.)
    f32x4 rk[C::NLD], rv[C::NLD];
    prefill_load_step<C, EB, NT>(k, v, rk, rv, (tlo + t) * kTile, nkeys, Hkv, kvh, tid, hdr);
    prefill_store_step<C, false, V16>(smem, rk, rv, 0, tid);
    __syncthreads();
    f32x4 *rec = reinterpret_cast<f32x4 *>(ps + ((size_t)kvh * nt + t) * C::PS_FLOATS);
    for (int c = tid; c < C::IMG / 4; c += C::THREADS)
        rec[c] = reinterpret_cast<const f32x4 *>(smem)[c];
}

__device__ __forceinline__ void wait_vm_all() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// Wait until at most N vector memory loads of this wave are outstanding (they complete in
// issue order).
template <int N>
__device__ __forceinline__ void wait_vm_keep() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Four-wave head_dim <= 128 workgroups must fit two per CU (2 waves per SIMD).
// RANGE: queries start at position qbase and may have a sliding window; without it the
// kernel is specialised to a prompt from position 0 (no window), whose masks are simpler.
// EB: bytes per K/V element (4 f32, 2 IEEE half, 1 OCP FP8 E4M3: an f16 or E4M3 KV
// cache), converted to f32 as they are staged.
// PS: K/V come as pre-split records (ps: ps_nt records per KV head, record 0 = tile
// ps_tlo) instead of k/v.
// FAST (an opt-in mode, f32 K/V without pre-split records): q, K, V and P are rounded to
// f16 once and each product is one f16 MFMA (instead of three on exact hi/lo splits); the
// online softmax, its rescaling and the accumulation stay f32.
//
// Occupancy: the dynamic LDS the launch asks for (prefill_lds_bytes) bounds the waves per
// SIMD; the compiler, which does not see it, is told that bound, so that it does not trade
// the schedule for an occupancy the LDS never allows. 4-wave workgroups at head_dim <= 128
// run two per CU, so at least two waves per SIMD; the f16 mode over pre-converted records
// without key splits (FAST3) three: its LDS (two hi-half buffers, output stored from
// registers) allows four such workgroups per CU, and its registers fit 168.
template <class C, bool FAST>
constexpr bool direct_out() { return FAST && C::STEP_KEYS == kTile && EB_PREFILL_FAST_OCC; }
// FAST3 over records copies each step's images two steps ahead into three buffers.
template <class C, bool FAST, bool PS>
constexpr bool triple_buf() { return PS && direct_out<C, FAST>() && EB_PREFILL_FAST_TB; }
template <class C, bool FAST, bool PS>
constexpr size_t prefill_lds_bytes() {
    constexpr int buf2 = (triple_buf<C, FAST, PS>() ? 3 : 2) * bufsize<C, FAST>();
    constexpr int out = direct_out<C, FAST>() ? 0 : C::OUT;
    constexpr int a = buf2 > C::MERGE ? buf2 : C::MERGE;
    return (size_t)(a > out ? a : out) * sizeof(float);
}
template <int HD, int HPW, int WPH, int KSPLIT, bool FAST, bool PS>
constexpr int prefill_min_waves() {
    if (direct_out<PrefillCfg<HD, HPW, WPH, KSPLIT>, FAST>() && PS && HD <= 128) return 3;
    return (HPW * WPH * KSPLIT == 4 && HD <= 128) ? 2 : 1;
}
template <int HD, int HPW, int WPH, int KSPLIT, bool FAST, bool PS>
constexpr int prefill_max_waves() {
    constexpr size_t lds = prefill_lds_bytes<PrefillCfg<HD, HPW, WPH, KSPLIT>, FAST, PS>();
    constexpr int wgs = lds > 0 ? (int)(kLdsBytesPerCu / lds) : 8;
    constexpr int w = (wgs < 1 ? 1 : wgs) * HPW * WPH * KSPLIT / 4;
    constexpr int lo = prefill_min_waves<HD, HPW, WPH, KSPLIT, FAST, PS>();
    return w < lo ? lo : w > 8 ? 8 : w;
}
// PV1 (head_dim >= 32, with FAST false): the scores-accurate mode. The scores keep the
// three-product split; O^T += V^T P^T is one f16 product, as in FAST: V rows rounded to f16
// as they are at staging (pre-split records of the same layout, V16), the weights
// p <= 2^kSlack rounded to f16, and l summing the weights as rounded (so that they
// normalise exactly and a dominant key's rounding cancels). A third fewer products than
// the accurate mode, and no per-query unit.
template <int HD, int HPW, int WPH, int KSPLIT, bool RANGE, int EB, bool PS, bool FAST = false,
          bool PV1 = false>
__global__ __attribute__((
    amdgpu_flat_work_group_size(1, HPW * WPH * KSPLIT * 64),
    amdgpu_waves_per_eu(prefill_min_waves<HD, HPW, WPH, KSPLIT, FAST, PS>(),
                        prefill_max_waves<HD, HPW, WPH, KSPLIT, FAST, PS>()))) void prefill_kernel(
    const float *__restrict__ q, const void *__restrict__ k, const void *__restrict__ v,
    const float *__restrict__ ps, int ps_tlo, int ps_nt, float *__restrict__ o, int H,
    int Hkv, int rows, int nkeys, int qbase, int window, float scale_log2, int nqb,
    int ngroups, int ctiles, float *__restrict__ part_acc, float *__restrict__ part_ml, int hdr) {
    using C = PrefillCfg<HD, HPW, WPH, KSPLIT>;
    constexpr int QB = C::QB;
    constexpr int HALF = C::HALF;
    constexpr int NB = C::NB;
    constexpr int KS = C::KS;
    constexpr int BUFX = bufsize<C, FAST>();  // LDS buffer size of this mode

    extern __shared__ float smem[];  // [2][BUF]: K rows [STEP_KEYS][KS], V rows [STEP_KEYS][HD]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: scalar registers)
    const int hf = lane >> 5;
    const int col = lane & 31;
    const int ks = wave / (HPW * WPH);     // key split this wave takes
    const int slot = wave % (HPW * WPH);   // (head, query sub-block) of this wave
    const int g = H / Hkv;
    const int gsub = g / HPW;
    const int flat = blockIdx.x;
    // (uniform: the divisions by run-time values go through the vector unit, so their
    // results are moved to scalar registers)
    const int grp = __builtin_amdgcn_readfirstlane(flat % ngroups);
    const int qb = __builtin_amdgcn_readfirstlane(nqb - 1 - flat / ngroups);  // heaviest first
    const int kvh = __builtin_amdgcn_readfirstlane(grp / gsub);
    const int head = __builtin_amdgcn_readfirstlane(kvh * g + (grp % gsub) * HPW + slot / WPH);
    // Query rows are local (0..rows-1) and sit at positions qbase + row. Key tiles of 32
    // cover keys [32 t, 32 t + 32); a query at p sees keys max(0, p - window + 1)..p
    // (0..p without a window).
    if constexpr (!RANGE) {
        qbase = 0;
        window = 0;
    }
    const int q0 = qb * QB + (slot % WPH) * kTile;
    const int p_first = qbase + qb * QB;
    const int p_last = qbase + min(qb * QB + QB, rows) - 1;
    const int t0 = window > 0 ? max(0, p_first - window + 1) / kTile : 0;
    // Key chunk blockIdx.y of the block's tiles t0..tE (ctiles tiles each): a block with
    // more than one chunk writes partial states, which prefill_merge_kernel combines.
    const int tE = p_last / kTile;
    const int nch = (tE - t0) / ctiles + 1;
    const int chunk = blockIdx.y;
    if (chunk >= nch) return;  // (workgroup-uniform)
    const int c_lo = t0 + chunk * ctiles;
    const int c_hi = min(tE, c_lo + ctiles - 1);
    const int nsteps = (c_hi - c_lo) / KSPLIT + 1;
    const bool live = q0 < rows;
    const int wp0 = qbase + q0;                         // this wave's first position
    const int wp1 = qbase + min(q0 + kTile, rows) - 1;  // and last
    const int my_t0 = window > 0 ? max(0, wp0 - window + 1) / kTile : 0;
    const int my_t1 = wp1 / kTile;
    const int qi = q0 + col;
    const int pi = qbase + qi;

    // The first step's K/V loads (records memory-to-LDS, or K/V rows into registers) go
    // out right behind the q fragment's, so that the two latencies overlap.
    f32x4 rk[PS ? 1 : C::NLD], rv[PS ? 1 : C::NLD];
    static_assert(!(PS && FAST) || HD <= 128, "f16-mode records for head_dim <= 128");
    constexpr int IMGX = imgsize<C, FAST>();
    const float *recs = PS ? ps + (size_t)kvh * ps_nt * IMGX : nullptr;
    // TB: three buffers, the first two steps' copies issued here (a wave's copy of one step
    // is TBL loads; they complete in issue order).
    constexpr bool TB = triple_buf<C, FAST, PS>();
    constexpr int TBL = (IMGX / 256 + C::NW - 1) / C::NW * KSPLIT;
    static_assert(!TB || (IMGX / 256) % C::NW == 0, "every wave issues TBL loads per step");
    auto load_first_step = [&] {
        if constexpr (PS) {
            img_copy<IMGX, KSPLIT, C::NW>(recs, smem, c_lo - ps_tlo, ps_nt, wave, lane);
            if constexpr (TB)
                img_copy<IMGX, KSPLIT, C::NW>(recs, smem + BUFX, c_lo + KSPLIT - ps_tlo, ps_nt,
                                              wave, lane);
        } else
            prefill_load_step<C, EB>(k, v, rk, rv, c_lo * kTile, nkeys, Hkv, kvh, tid, hdr);
    };

    // Q fragment. SQK: query qi scaled by 2^-eq (its largest magnitude in [2^14, 2^15))
    // and split into f16 hi/lo, dims ks*16 + hf*8 .. +8 for every 16-dim step ks; else
    // f32, head dims [HALF*hf, HALF*hf + HALF).
    constexpr int NKS = HD / 16;
    f16x8 qh[C::SQK ? NKS : 1], ql[C::SQK ? NKS : 1];
    int eq = 0;
    if constexpr (C::SQK) {
        const bool qv = qi < rows;
        const float *qp = q + ((size_t)(qv ? qi : 0) * H + head) * hdr + 8 * hf;
        f32x4 qa[NKS], qb[NKS];
        const float qs = qv ? scale_log2 : 0.0f;
        float mx = 0.0f;
        // Every lane loads (rows past the end from the clamped row 0) and scales by qs, 0
        // past the end, so that the loads issue back to back; such a lane's query column
        // never reaches the output. Dims past hdr (a head dim padded up to this
        // instantiation) are zeros. A head dim that is an odd multiple of 8 ends halfway
        // into its last 16-dim step: there the upper half-wave (dims +8..+15) reads the
        // lower half's address (inside the row) and keeps zeros.
        if (hdr == HD) {  // (uniform) the instantiation's own head dim
#pragma unroll
            for (int k2 = 0; k2 < NKS; ++k2) {
                qa[k2] = *reinterpret_cast<const f32x4 *>(qp + 16 * k2);
                qb[k2] = *reinterpret_cast<const f32x4 *>(qp + 16 * k2 + 4);
            }
        } else {
#pragma unroll
            for (int k2 = 0; k2 < NKS; ++k2) {
                const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const bool full = 16 * k2 + 16 <= hdr;     // (uniform)
                const bool half = !full && 16 * k2 < hdr;  // (uniform) hdr = 16 k2 + 8
                // one load pair per step (a step wholly past hdr reads the row's start)
                const float *qe = full ? qp + 16 * k2 : half ? qp + 16 * k2 - 8 * hf : qp;
                const f32x4 a = *reinterpret_cast<const f32x4 *>(qe);
                const f32x4 b = *reinterpret_cast<const f32x4 *>(qe + 4);
                const bool keep = full || (half && !hf);
                qa[k2] = keep ? a : z;
                qb[k2] = keep ? b : z;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_first_step();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k2 = 0; k2 < NKS; ++k2) {
            // The softmax scale (log2 units) is applied to q before its split, so the
            // product needs no multiply per score.
            qa[k2] = qa[k2] * qs;
            qb[k2] = qb[k2] * qs;
            const float m8 = fmaxf(fmaxf(fmaxf(fabsf(qa[k2].x), fabsf(qa[k2].y)),
                                         fmaxf(fabsf(qa[k2].z), fabsf(qa[k2].w))),
                                   fmaxf(fmaxf(fabsf(qb[k2].x), fabsf(qb[k2].y)),
                                         fmaxf(fabsf(qb[k2].z), fabsf(qb[k2].w))));
            mx = fmaxf(mx, m8);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));  // the other half of the row
        eq = FAST ? 0 : split_exponent(mx);
#pragma unroll
        for (int k2 = 0; k2 < NKS; ++k2) {
            f16x4 h0, l0, h1, l1;
            if constexpr (FAST) {
                h0 = __builtin_convertvector(qa[k2], f16x4);
                h1 = __builtin_convertvector(qb[k2], f16x4);
                l0 = h0;
                l1 = h1;
            } else {
                split_f16(qa[k2], eq, h0, l0);
                split_f16(qb[k2], eq, h1, l1);
            }
            qh[k2] = f16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
            ql[k2] = f16x8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        }
    }
    float qreg[C::SQK ? 1 : HALF];
    if constexpr (!C::SQK) {
        load_first_step();
        const bool qv = qi < rows;
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
    // SPV: O^T is accumulated in units of 2^E (per query; both lane halves of a query hold
    // the same E).
    int E = (FAST || PV1) ? 0 : kZeroRowExp;

    static_assert(!PS || C::SPV, "pre-split records carry the split V layout");
    // ... and the first step's K/V into LDS.
    if constexpr (TB)
        wait_vm_keep<TBL>();
    else if constexpr (PS)
        wait_vm_all();
    else
        prefill_store_step<C, FAST, PV1>(smem, rk, rv, 0, tid);
    __syncthreads();

    // The next step's K/V: PS records straight into the other buffer (which every wave
    // finished reading before the last barrier), otherwise K/V rows into registers. Past the
    // last step this re-reads clamped rows (the buffer written from them is never read).
    auto prefetch = [&](int it1, int b1) {
        if constexpr (PS)
            img_copy<IMGX, KSPLIT, C::NW>(recs, smem + b1 * BUFX, c_lo + it1 * KSPLIT - ps_tlo,
                                          ps_nt, wave, lane);
        else
            prefill_load_step<C, EB>(k, v, rk, rv, (c_lo + it1 * KSPLIT) * kTile, nkeys, Hkv,
                                      kvh, tid, hdr);
    };
    auto stage = [&](int b1) {
        if constexpr (PS)
            wait_vm_all();
        else
            prefill_store_step<C, FAST, PV1>(smem, rk, rv, b1, tid);
    };

    if constexpr (C::SPV) {
        // Per-tile stages on the split f16 operands (head_dim >= 32):
        //  qk:      S^T = K Q^T for the wave's tile in buffer b (16 keys x 1 query per lane);
        //  softmax: the online softmax update (m, l, the O^T unit E, the rescale of O^T) and
        //           the P^T operands;
        //  pv:      O^T += V^T P^T from buffer b.
        auto tile_qk = [&](int b, floatx16 &sacc) {
            const float *img = smem + b * BUFX + ks * IMGX;  // tile ks's image
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
            // K chunk 2 k2 + hf of key col: hi (FAST: the only) halves, the lo ones 4 HD
            // chunks on
            const _Float16 *kimg = reinterpret_cast<const _Float16 *>(img) +
                                   8 * (FAST ? fk_chunk<HD>(col, hf) : sk_chunk<C>(col, hf, 0));
            if constexpr (FAST && NKS <= 8) {
                // All of the tile's K operands are read before the first product (the
                // compiler would otherwise wait out each read's latency before its product).
                f16x8 ka[NKS];
#pragma unroll
                for (int k2 = 0; k2 < NKS; ++k2)
                    ka[k2] = *reinterpret_cast<const f16x8 *>(kimg + 8 * 2 * kTile * k2);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k2 = 0; k2 < NKS; ++k2) sacc = mfma16(ka[k2], qh[k2], sacc);
            } else if constexpr (FAST) {  // (head_dim 256: no registers for that)
#pragma unroll
                for (int k2 = 0; k2 < NKS; ++k2)
                    sacc = mfma16(*reinterpret_cast<const f16x8 *>(kimg + 8 * 2 * kTile * k2),
                                  qh[k2], sacc);
            } else {
                // Three products per 16-dim step (hi*hi, hi*lo, lo*hi; lo*lo is below 2^-22).
                // (both operands read before the products with key splits, the lo operand
                // after the first product without: the orders that leave the staged
                // kernels at head_dim 128 without a register spill)
#pragma unroll
                for (int k2 = 0; k2 < NKS; ++k2) {
                    const _Float16 *kh = kimg + 8 * 2 * C::KCS * k2;
                    const f16x8 ah = *reinterpret_cast<const f16x8 *>(kh);
                    f16x8 al;
                    if constexpr (KSPLIT > 1)
                        al = *reinterpret_cast<const f16x8 *>(kh + 8 * C::KC);
                    sacc = mfma16(ah, qh[k2], sacc);
                    if constexpr (KSPLIT == 1)
                        al = *reinterpret_cast<const f16x8 *>(kh + 8 * C::KC);
                    sacc = mfma16(ah, ql[k2], sacc);
                    sacc = mfma16(al, qh[k2], sacc);
                }
            }
            // Scores back from the split's units: 2^(eq + ek), ek the exponent of each of
            // this lane's keys (read four at a time).
            if constexpr (!FAST) {
                const int *Eb = reinterpret_cast<const int *>(img + C::EXPO);
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4) {
                    const int4 e4 = *reinterpret_cast<const int4 *>(Eb + 8 * s4 + 4 * hf);
                    sacc[4 * s4 + 0] = ldexpf(sacc[4 * s4 + 0], eq + e4.x);
                    sacc[4 * s4 + 1] = ldexpf(sacc[4 * s4 + 1], eq + e4.y);
                    sacc[4 * s4 + 2] = ldexpf(sacc[4 * s4 + 2], eq + e4.z);
                    sacc[4 * s4 + 3] = ldexpf(sacc[4 * s4 + 3], eq + e4.w);
                }
            }
        };

        auto tile_softmax = [&](int b, int kb, const floatx16 &sacc, f16x8 (&ph)[2],
                                f16x8 (&pl)[2]) {
            // the scores in log2 units
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = sacc[r];
            // Online softmax over this tile's keys (log2 domain). Only tiles that reach past
            // the wave's first position, or (window) below its last position's window, need
            // the per-key mask.
            const bool edge =
                RANGE ? (kb + kTile - 1 > wp0 || (window > 0 && kb <= wp1 - window)) : kb == q0;
            if (edge) {  // wave-uniform: most tiles skip the per-key mask
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb + 8 * (r >> 2) + 4 * hf + (r & 3);
                    if (key > pi || (RANGE && window > 0 && key <= pi - window)) p[r] = -INFINITY;
                }
            }
            float mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, p[r]);
            mt = fmaxf(mt, eb::lane_xor32(mt));
            // Lazy reference max: m moves only when a score exceeds it by more than kSlack
            // (log2 units), so most tiles need no rescale of l and O^T; terms 2^(s - m) then
            // stay below 2^kSlack, which the f16 split holds exactly.
            const bool grow = mt > m + kSlack;
            const float mnew = grow ? fmaxf(m, mt) : m;
            // A query can meet a tile with all of its keys masked before its first visible
            // key (unaligned chunk starts, windows): keep exp2 away from -inf - -inf.
            const float mref = mnew == -INFINITY ? 0.0f : mnew;
            const float corr = grow ? eb::fast_exp2(m - mref) : 1.0f;
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = eb::fast_exp2(p[r] - mref);
                if constexpr (!PV1) ps += p[r];
            }
            if constexpr (!PV1) l = l * corr + ps;
            const float mold = m;
            m = mnew;
            if constexpr (FAST || PV1) {
                // One f16 product: P rounded to f16 (p <= 2^kSlack, so no unit is needed),
                // the V^T hi halves (V rounded to f16 at staging). O^T follows the softmax
                // correction when any lane's reference max moved.
                if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
                    for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) oacc[mb][r] *= corr;
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    unsigned hw[4];
#pragma unroll
                    for (int c2 = 0; c2 < 4; ++c2) {
                        const int r = 8 * u + 2 * c2;
                        hw[c2] = __builtin_bit_cast(
                            unsigned, __builtin_convertvector(f32x2{p[r], p[r + 1]}, f16x2));
                        if constexpr (PV1) {
                            // l sums the weights as rounded, so that they normalise exactly
                            // and a dominant key's rounding cancels
                            const f32x2 pr = __builtin_convertvector(
                                __builtin_bit_cast(f16x2, hw[c2]), f32x2);
                            ps += pr.x + pr.y;
                        }
                    }
                    ph[u] = __builtin_bit_cast(f16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
                    pl[u] = ph[u];
                }
                if constexpr (PV1) l = l * corr + ps;
            } else {
                // The tile's V exponents ev (V row = 2^ev * v').
                const int *Ev =
                    reinterpret_cast<const int *>(smem + b * BUFX + ks * IMGX + C::EXPO) + kTile;
                int ev[16];
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4) {
                    const int4 e4 = *reinterpret_cast<const int4 *>(Ev + 8 * s4 + 4 * hf);
                    ev[4 * s4 + 0] = e4.x;
                    ev[4 * s4 + 1] = e4.y;
                    ev[4 * s4 + 2] = e4.z;
                    ev[4 * s4 + 3] = e4.w;
                }
                // This query's unit: O^T is held in units of 2^E, E the exponent of its
                // largest term p * 2^ev, so that p' = p * 2^(ev - E) <= 1 and the largest
                // terms keep full f16 hi/lo precision (a wave-wide unit would push the p'
                // of a query's small-V keys below f16 range whenever another query, or a
                // key of negligible weight, brings a large V row). p * 2^ev has the float
                // bits of p plus ev in the exponent field (an upper bound for p = 0 or
                // subnormal), so the tile's largest term comes from an integer max.
                unsigned tb = 0x80000000u;  // the smallest int
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const unsigned t = __builtin_bit_cast(unsigned, p[r]) + ((unsigned)ev[r] << 23);
                    tb = (int)t > (int)tb ? t : tb;
                }
                int tx = ((int)tb >> 23) - 126;
                tx = max(tx, __builtin_bit_cast(int, eb::lane_xor32(__builtin_bit_cast(float, tx))));
                // The softmax correction 2^-(mref - mold) moves the accumulated terms down:
                // the unit follows by whole bits, the fraction goes into the rescale factor.
                // The unit moves up only for a term more than 2^kUnitSlack above it (then
                // to that term): p' <= 2^kUnitSlack, which f16 holds, and most tiles keep
                // the unit, so the wave skips the rescale.
                const float dm = mref - mold;
                const int Eb = !grow ? E : (dm < 1000.0f ? max(E - (int)dm, kZeroRowExp) : kZeroRowExp);
                const int En = tx > Eb + kUnitSlack ? tx : Eb;
                if (__builtin_amdgcn_ballot_w64(grow || En != E) != 0) {
                    const float f = ldexpf(corr, E - En);  // <= 1 (grow) or 2^(E - En) <= 1
#pragma unroll
                    for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) oacc[mb][r] *= f;
                }
                E = En;
                // P^T operands: k-step u takes this lane's keys r = 8u .. 8u+7.
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    unsigned hw[4], lw[4];
#pragma unroll
                    for (int c2 = 0; c2 < 4; ++c2) {
                        const int r = 8 * u + 2 * c2;
                        const f32x2 pp = {ldexpf(p[r], ev[r] - E), ldexpf(p[r + 1], ev[r + 1] - E)};
                        hw[c2] = __builtin_bit_cast(unsigned, __builtin_convertvector(pp, f16x2));
                        const f32x2 rem = {sub_f16_lo(hw[c2], pp.x), sub_f16_hi(hw[c2], pp.y)};
                        lw[c2] = __builtin_bit_cast(unsigned, __builtin_convertvector(rem, f16x2));
                    }
                    ph[u] = __builtin_bit_cast(f16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
                    pl[u] = __builtin_bit_cast(f16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
                }
            }
        };

        // O^T += V^T P^T: block mb's row col is dim NB*col + mb (the layout the output stage
        // expects), stored at V^T row 32*mb + col; keys 16u + 4hf + 0..3 and 16u + 8 + 4hf +
        // 0..3 of this wave's tile (the order of ph / pl). FAST: the hi halves only.
        auto tile_pv = [&](int b, const f16x8 (&ph)[2], const f16x8 (&pl)[2]) {
            // V^T chunk hf + 2u of row 32 mb + col in tile ks's image: hi (FAST: the only)
            // halves, the lo ones 4 HD chunks on
            const _Float16 *vimg =
                reinterpret_cast<const _Float16 *>(smem + b * BUFX + ks * IMGX) +
                8 * (FAST ? fv_chunk<HD>(col, hf) : sv_chunk<C>(col, hf, 0));
            if constexpr (FAST || PV1) {
                // One product: the NB V fragments of one 16-key half are read first and the
                // products go round the NB accumulators (measured 2-4 % faster than one
                // accumulator's products back to back; the three-product mode has no
                // registers left for it)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    f16x8 vh[NB];
#pragma unroll
                    for (int mb = 0; mb < NB; ++mb)
                        vh[mb] = *reinterpret_cast<const f16x8 *>(vimg + 8 * (2 * u * HD + 32 * mb));
#pragma unroll
                    for (int mb = 0; mb < NB; ++mb) oacc[mb] = mfma16(vh[mb], ph[u], oacc[mb]);
                }
            } else {
#pragma unroll
                for (int mb = 0; mb < NB; ++mb) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const _Float16 *vp = vimg + 8 * (2 * u * HD + 32 * mb);
                        const f16x8 vh = *reinterpret_cast<const f16x8 *>(vp);
                        const f16x8 vl = *reinterpret_cast<const f16x8 *>(vp + 8 * 4 * HD);
                        oacc[mb] = mfma16(vh, ph[u], oacc[mb]);
                        oacc[mb] = mfma16(vh, pl[u], oacc[mb]);
                        oacc[mb] = mfma16(vl, ph[u], oacc[mb]);
                    }
                }
            }
        };

        floatx16 sacc;
        f16x8 ph[2], pl[2];
        int b3 = 0;  // TB: it % 3
        for (int it = 0; it < nsteps; ++it) {
            const int buf = TB ? b3 : it & 1;
            const int tile = c_lo + it * KSPLIT + ks;
            if constexpr (TB)
                prefetch(it + 2, b3 == 0 ? 2 : b3 - 1);  // into buffer (it + 2) % 3, free
            else                                         // since the last barrier
                prefetch(it + 1, buf ^ 1);
            if (live && tile >= my_t0 && tile <= my_t1 && tile <= c_hi) {
                tile_qk(buf, sacc);
                tile_softmax(buf, tile * kTile, sacc, ph, pl);
                // The P V products at raised wave priority: with two waves on a SIMD, the one
                // that reaches them issues first, so that the other's softmax runs beside
                // them (measured +3 % at Qwen, +6 % at Mistral T=4096; the f16 mode, with a
                // third of the products, measured slower with it, and head dim 256 runs one
                // wave per SIMD).
                constexpr bool kPvPrio = !FAST && !PV1 && HD <= 128;
                if constexpr (kPvPrio) __builtin_amdgcn_s_setprio(1);
                tile_pv(buf, ph, pl);
                if constexpr (kPvPrio) __builtin_amdgcn_s_setprio(0);
            }
            if constexpr (TB) {
                wait_vm_keep<TBL>();  // step it + 1 in LDS, step it + 2 still in flight
                b3 = b3 == 2 ? 0 : b3 + 1;
            } else {
                stage(buf ^ 1);
            }
            __syncthreads();
        }
        if constexpr (TB) wait_vm_all();  // (the copies past the last step)
    } else {
    for (int it = 0; it < nsteps; ++it) {
        const int buf = it & 1;
        const int tile = c_lo + it * KSPLIT + ks;
        const int kb = tile * kTile;
        prefetch(it + 1, buf ^ 1);

        if (live && tile >= my_t0 && tile <= my_t1 && tile <= c_hi) {
            const float *Kb = smem + buf * C::BUF + ks * kTile * KS;
            const float *Vb = smem + buf * C::BUF + C::STEP_KEYS * KS + ks * kTile * HD;
            // S^T = K Q^T for this tile: 16 keys x 1 query per lane (FP32 MFMA).
            floatx16 sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
            const float *kr = Kb + col * KS + HALF * hf;
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
            const bool edge =
                RANGE ? (kb + kTile - 1 > wp0 || (window > 0 && kb <= wp1 - window)) : kb == q0;
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = sacc[r] * scale_log2;
            if (edge) {  // wave-uniform: most tiles skip the per-key mask
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb + 8 * (r >> 2) + 4 * hf + (r & 3);
                    if (key > pi || (RANGE && window > 0 && key <= pi - window)) p[r] = -INFINITY;
                }
            }
            float mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, p[r]);
            mt = fmaxf(mt, eb::lane_xor32(mt));
            const float mnew = fmaxf(m, mt);
            // A query can meet a tile with all of its keys masked before its first visible
            // key (unaligned chunk starts, windows): keep exp2 away from -inf - -inf.
            const float mref = (RANGE && mnew == -INFINITY) ? 0.0f : mnew;
            const float corr = eb::fast_exp2(m - mref);
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = eb::fast_exp2(p[r] - mref);
                ps += p[r];
            }
            l = l * corr + ps;
            m = mnew;
#pragma unroll
            for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[mb][r] *= corr;

            // O^T += V^T P^T: step t pairs key 8*(t/4) + 4*hf + t%4 with p[t].
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int kl = 8 * (t >> 2) + 4 * hf + (t & 3);
                const float *vp = Vb + kl * HD;
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

        stage(buf ^ 1);
        __syncthreads();
    }
    }

    // The lane's coordinates again, from the lane id: recomputed here, they need not stay
    // live (or spill) through the loop.
    const int elane = __lane_id();
    const int ehf = elane >> 5, ecol = elane & 31, eqi = q0 + ecol;

    // Merge the key splits: waves ks >= 1 hand (m, l, O^T) to wave ks = 0 of their slot
    // through LDS (reusing the tile buffers, free after the loop's last barrier). Fields are
    // stored [record][field][elane] so every access is a contiguous 64-elane row.
    if constexpr (KSPLIT > 1) {
        if (ks > 0) {
            float *rec = smem + ((ks - 1) * (HPW * WPH) + slot) * C::REC * 64;
            rec[0 * 64 + elane] = m;
            rec[1 * 64 + elane] = l;
            rec[2 * 64 + elane] = __int_as_float(E);
#pragma unroll
            for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) rec[(3 + mb * 16 + r) * 64 + elane] = oacc[mb][r];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int j = 1; j < KSPLIT; ++j) {
                const float *rec = smem + ((j - 1) * (HPW * WPH) + slot) * C::REC * 64;
                const float m2 = rec[elane];
                const float l2 = rec[64 + elane];
                const int E2 = __float_as_int(rec[128 + elane]);
                const float M = fmaxf(m, m2);
                const float Mr = (M == -INFINITY) ? 0.0f : M;
                const float a1 = eb::fast_exp2(m - Mr);   // 0 when this wave saw no keys
                const float a2 = eb::fast_exp2(m2 - Mr);  // 0 when split j saw no keys
                l = l * a1 + l2 * a2;
                m = M;
                // both O^T partials to the larger unit 2^En (SPV; E stays unused otherwise)
                const int En = max(E, E2);
                const float b1 = C::SPV ? ldexpf(a1, E - En) : a1;
                const float b2 = C::SPV ? ldexpf(a2, E2 - En) : a2;
                E = En;
#pragma unroll
                for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        oacc[mb][r] = oacc[mb][r] * b1 + rec[(3 + mb * 16 + r) * 64 + elane] * b2;
            }
        }
    }

    // Normalise, then store through LDS: elane (ecol, ehf) holds O[q0 + ecol][NB*c + mb] for
    // c = 8*(r/4) + 4*ehf + r%4, i.e. 16-byte pieces of 32 different output rows. Each
    // slot's 32 x HD tile is transposed through LDS so the global stores are whole rows
    // (HD contiguous floats per (query, head)).
    // A block split into key chunks writes its raw state instead: O^T (in units of 2^E for
    // SPV) and (m, l, E) per query, for prefill_merge_kernel.
    const float lt = l + __shfl_xor(l, 32);
    const bool partial = nch > 1;
    if constexpr (KSPLIT > 1) __syncthreads();  // the merge records are read; reuse LDS
    float *ot = smem + slot * kTile * C::OS;    // this slot's staging tile [32][OS]
    if (ks == 0 && live) {
        const float inv = partial ? 1.0f : 1.0f / lt;
        // SPV: O^T is in units of 2^E; ldexp each normalised value back (exact)
        if constexpr (C::SPV) {
            if (!partial) {
#pragma unroll
                for (int mb = 0; mb < NB; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[mb][r] = ldexpf(oacc[mb][r] * inv, E);
            }
        }
        if (partial && ehf == 0 && eqi < rows)
            *reinterpret_cast<float4 *>(part_ml + (((size_t)chunk * rows + eqi) * H + head) * 4) =
                make_float4(m, lt, __int_as_float(C::SPV ? E : 0), 0.0f);
        const float sc_o = C::SPV ? 1.0f : inv;
        if constexpr (direct_out<C, FAST>()) {
            // Straight from the registers: elane (ecol, ehf) stores NB consecutive dims NB*c ..
            // NB*c + NB - 1 of its query's row for each of its 16 values of c.
            if (eqi < rows) {
                float *dst = partial ? part_acc + (size_t)chunk * rows * H * HD : o;
                const int dstride = partial ? HD : hdr;
                float *orow = dst + ((size_t)eqi * H + head) * dstride;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int c = 8 * (r >> 2) + 4 * ehf + (r & 3);
                    if (NB * c >= dstride) continue;  // (dims past hdr: the padding)
                    if constexpr (NB >= 4) {
#pragma unroll
                        for (int j = 0; j < NB / 4; ++j)
                            *reinterpret_cast<float4 *>(orow + NB * c + 4 * j) =
                                make_float4(oacc[4 * j][r], oacc[4 * j + 1][r],
                                            oacc[4 * j + 2][r], oacc[4 * j + 3][r]);
                    } else if constexpr (NB == 2) {
                        *reinterpret_cast<float2 *>(orow + 2 * c) = make_float2(oacc[0][r], oacc[1][r]);
                    } else {
                        orow[c] = oacc[0][r];
                    }
                }
            }
            return;
        }
        float *orow = ot + ecol * C::OS;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = 8 * (r >> 2) + 4 * ehf + (r & 3);
            if constexpr (NB == 8) {
                *reinterpret_cast<float4 *>(orow + 8 * c) =
                    make_float4(oacc[0][r] * sc_o, oacc[1][r] * sc_o, oacc[2][r] * sc_o, oacc[3][r] * sc_o);
                *reinterpret_cast<float4 *>(orow + 8 * c + 4) =
                    make_float4(oacc[4][r] * sc_o, oacc[5][r] * sc_o, oacc[6][r] * sc_o, oacc[7][r] * sc_o);
            } else if constexpr (NB == 4) {
                *reinterpret_cast<float4 *>(orow + 4 * c) =
                    make_float4(oacc[0][r] * sc_o, oacc[1][r] * sc_o, oacc[2][r] * sc_o, oacc[3][r] * sc_o);
            } else if constexpr (NB == 2) {
                *reinterpret_cast<float2 *>(orow + 2 * c) = make_float2(oacc[0][r] * sc_o, oacc[1][r] * sc_o);
            } else if constexpr (HD >= 32) {
                orow[c] = oacc[0][r] * sc_o;
            } else {
                if (c < HD) orow[c] = oacc[0][r] * sc_o;
            }
        }
    }
    if constexpr (direct_out<C, FAST>()) return;
    __syncthreads();
    if (ks == 0 && live) {
        // o rows hold hdr dims; the partials keep the instantiation's HD
        float *dst = partial ? part_acc + (size_t)chunk * rows * H * HD : o;
        const int dstride = partial ? HD : hdr;
        constexpr int ROW4 = HD / 4;  // float4 per output row
#pragma unroll
        for (int j = 0; j < (kTile * ROW4 + 63) / 64; ++j) {
            const int idx = j * 64 + elane;
            if (kTile * ROW4 % 64 == 0 || idx < kTile * ROW4) {
                const int row = idx / ROW4;
                const int c4 = idx % ROW4;
                if (q0 + row < rows && 4 * c4 < dstride)
                    *reinterpret_cast<float4 *>(dst + ((size_t)(q0 + row) * H + head) * dstride + 4 * c4) =
                        *reinterpret_cast<const float4 *>(ot + row * C::OS + 4 * c4);
            }
        }
    }
}

// Combines the key chunks of the query blocks that were split: o = sum_c w_c O_c /
// sum_c w_c l_c with w_c = 2^(m_c - M), M the largest m_c, and O_c in units of 2^E_c
// (brought to the largest E first, so nothing overflows). A chunk that saw no key of a
// query has m = -inf and weight 0. Blocks of one chunk were written by the prefill itself.
// Thread (pair, d4): four output dims of one (row, head) pair; the chunks' states are read
// kMergeBatch at a time, all loads of a batch issued before any is used.
constexpr int kMergeBatch = 8;
// One chunk's term in the merge of key chunks: its Oᵀ partial acc is in units of 2^E
// (E = ml.z's int bits) and carries the weight w = 2^d, d = m - Mr <= 0 (ml.x = m, the
// chunk's running max in log2 units; Mr the row's largest). The term w·acc·2^E is
// acc·2^f·2^G with f = d - floor(d) in [0, 1) and G = E + floor(d): merge_exp gives G,
// and the row's reference exponent EM is the largest G, i.e. that of its largest weighted
// term, so that a chunk of negligible weight but large V rows cannot push the others
// below f32 range. d is clamped at -300: below that the term is under 2^-170 of any
// finite E and rounds away in the sum.
__device__ __forceinline__ int merge_exp(float4 ml, float Mr) {
    if (ml.x == -INFINITY) return kZeroRowExp;  // a chunk that saw no key
    return __float_as_int(ml.z) + (int)floorf(fmaxf(ml.x - Mr, -300.0f));
}
__device__ __forceinline__ void merge_add(float4 ml, float4 acc, float Mr, int EM, float4 &A,
                                          float &L) {
    if (ml.x == -INFINITY) return;
    const float d = fmaxf(ml.x - Mr, -300.0f);
    const float fl = floorf(d);
    const float wf = eb::fast_exp2(d - fl);
    const int sh = __float_as_int(ml.z) + (int)fl - EM;
    L += eb::fast_exp2(d) * ml.y;
    A.x += ldexpf(acc.x * wf, sh);
    A.y += ldexpf(acc.y * wf, sh);
    A.z += ldexpf(acc.z * wf, sh);
    A.w += ldexpf(acc.w * wf, sh);
}

template <int HD>
__global__ __launch_bounds__(256) void prefill_merge_kernel(
    const float *__restrict__ part_acc, const float *__restrict__ part_ml, float *__restrict__ o,
    int rows, int H, int QB, int qbase, int window, int ctiles, int hdr) {
    constexpr int TP = HD >= 4 ? HD / 4 : 1;  // threads per (row, head) pair
    constexpr int PER = 256 / TP;
    const int pair = blockIdx.x * PER + threadIdx.x / TP;
    const int d = 4 * (threadIdx.x % TP);
    if (pair >= rows * H || d >= hdr) return;  // (o rows hold hdr <= HD dims)
    const int row = pair / H;
    const int head = pair % H;
    const int qb = row / QB;
    const int p_first = qbase + qb * QB;
    const int p_last = qbase + min(qb * QB + QB, rows) - 1;
    const int t0 = window > 0 ? max(0, p_first - window + 1) / kTile : 0;
    const int nch = (p_last / kTile - t0) / ctiles + 1;
    if (nch <= 1) return;
    const size_t cstride = (size_t)rows * H;  // (row, head) pairs per chunk
    const size_t at0 = (size_t)row * H + head;
    if (nch <= kMergeBatch) {
        // One batch holds every chunk: one memory round trip.
        float4 ml[kMergeBatch], acc[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
            const size_t at = at0 + (size_t)min(j, nch - 1) * cstride;
            ml[j] = *reinterpret_cast<const float4 *>(part_ml + at * 4);
            acc[j] = *reinterpret_cast<const float4 *>(part_acc + at * HD + d);
        }
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) M = fmaxf(M, ml[j].x);
        const float Mr = (M == -INFINITY) ? 0.0f : M;
        int EM = kZeroRowExp;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) EM = max(EM, merge_exp(ml[j], Mr));
        float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
            if (j < nch) merge_add(ml[j], acc[j], Mr, EM, A, L);
        const float inv = 1.0f / L;
        *reinterpret_cast<float4 *>(o + at0 * hdr + d) =
            make_float4(ldexpf(A.x * inv, EM), ldexpf(A.y * inv, EM), ldexpf(A.z * inv, EM),
                        ldexpf(A.w * inv, EM));
        return;
    }
    float M = -INFINITY;
    for (int c0 = 0; c0 < nch; c0 += kMergeBatch) {
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
            M = fmaxf(M, part_ml[(at0 + (size_t)min(c0 + j, nch - 1) * cstride) * 4]);
    }
    const float Mr = (M == -INFINITY) ? 0.0f : M;
    int EM = kZeroRowExp;
    for (int c0 = 0; c0 < nch; c0 += kMergeBatch) {
        float4 ml[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
            ml[j] = *reinterpret_cast<const float4 *>(
                part_ml + (at0 + (size_t)min(c0 + j, nch - 1) * cstride) * 4);
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) EM = max(EM, merge_exp(ml[j], Mr));
    }
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += kMergeBatch) {
        float4 ml[kMergeBatch], acc[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
            const size_t at = at0 + (size_t)min(c0 + j, nch - 1) * cstride;
            ml[j] = *reinterpret_cast<const float4 *>(part_ml + at * 4);
            acc[j] = *reinterpret_cast<const float4 *>(part_acc + at * HD + d);
        }
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j)
            if (c0 + j < nch) merge_add(ml[j], acc[j], Mr, EM, A, L);
    }
    const float inv = 1.0f / L;
    *reinterpret_cast<float4 *>(o + at0 * hdr + d) =
        make_float4(ldexpf(A.x * inv, EM), ldexpf(A.y * inv, EM), ldexpf(A.z * inv, EM),
                    ldexpf(A.w * inv, EM));
}

struct PrefillRange {
    int rows;    // query rows
    int nkeys;   // key rows available in k/v
    int qbase;   // position of query row 0
    int window;  // sliding window (0: none)
    eb::CacheElem ce;  // k/v element type
    float *ws;   // workspace (null: no pre-split pass, no key chunks)
    size_t ws_floats;
    int hdr;     // the rows' head dim (at most the instantiation's; the rest reads as zeros)
};

// The instantiation a head dim runs on: the next power of two (4 .. 256). Head dims 48, 80,
// 96, ... pad their rows with zero dims, which change no score and are never stored.
size_t padded_hd(size_t hd) {
    size_t p = 4;
    while (p < hd) p *= 2;
    return p;
}

// The workgroup shape launch_prefill_hd picks for head_dim hd, H query heads, g per KV
// head, and `rows` query rows: HPW heads x WPH 32-row blocks x KSPLIT key splits. Four or
// more heads per KV head at head_dim <= 128 take 4 heads x 32 rows in 4-wave workgroups,
// two per CU, when that grid is more than one round of them (Mistral T=4096: 1024 blocks,
// 283 vs 256 TFLOP/s against two key splits); up to one round, two key splits in 8-wave
// workgroups, one per CU (Mistral T=512 37.4 -> 35.9 us, T=2048 156.4 -> 148.8, T=1024
// unchanged: the causal blocks balance over two rounds of workgroups instead of one).
struct PrefillShape {
    int hpw, wph, ksplit;
};
constexpr int kPrefillSlots = 256;  // workgroup slots of one round: one per CU
PrefillShape prefill_shape(size_t hd, int H, int g, int rows) {
    const int hpw = g % 4 == 0 ? 4 : g % 2 == 0 ? 2 : 1;
    if (hd > 128) return {hpw, 4 / hpw, 1};
    if (hpw < 4) return {hpw, 4 / hpw, 2};
    const long blocks = (long)((rows + kTile - 1) / kTile) * (H / 4);
    return {4, 1, blocks > 2 * kPrefillSlots ? 1 : 2};
}

// The pre-split pass pays one read and one write of the keys in range; it is used when at
// least this many query blocks (each of whose workgroups would re-stage every key) share
// them: 3, or 2 at head_dim 256, whose split while staging is the dearer (measured on
// chunks of 128 and 192 rows over long caches: 2 Qwen blocks -8.5 %, 3 +6 %, 4 Mistral
// blocks +4-9 %, 2 Gemma-4 blocks +10 %).
constexpr int kPresplitMinBlocks = 3;
constexpr size_t kPresplitStreamBytes = (size_t)128 << 20;
constexpr int kPresplitMinBlocks256 = 2;

// First tile and number of tiles the pre-split records cover: every key some query of the
// launch can see.
int presplit_tlo(const PrefillRange &r) {
    return r.window > 0 ? (r.qbase - r.window + 1 > 0 ? r.qbase - r.window + 1 : 0) / kTile : 0;
}
int presplit_nt(const PrefillRange &r) { return (r.nkeys + kTile - 1) / kTile - presplit_tlo(r); }

size_t presplit_floats(size_t hd, size_t h, size_t hkv, const PrefillRange &r) {
    if (hd < 32 || r.rows <= 0 || r.nkeys <= 0) return 0;
    const int qb_rows = kTile * prefill_shape(hd, (int)h, (int)(h / hkv), r.rows).wph;
    const int nqb = (r.rows + qb_rows - 1) / qb_rows;
    if (nqb < (hd > 128 ? kPresplitMinBlocks256 : kPresplitMinBlocks)) return 0;
    const size_t rec = hd == 32    ? PrefillCfg<32, 4, 1, 1>::PS_FLOATS
                       : hd == 64  ? PrefillCfg<64, 4, 1, 1>::PS_FLOATS
                       : hd == 128 ? PrefillCfg<128, 4, 1, 1>::PS_FLOATS
                                   : PrefillCfg<256, 4, 1, 1>::PS_FLOATS;
    return hkv * (size_t)presplit_nt(r) * rec;
}

// Key chunks: when the query blocks alone fill at most half of the workgroup slots
// (short prompts, a short chunk over a long cache), each block's key tiles are cut into
// chunks of ctiles tiles, one workgroup each, merged afterwards; between half and all of
// the slots, only the heaviest blocks are halved; beyond, the heaviest-first order of the
// blocks balances the causal triangle by itself. Measured against one workgroup per block
// (us per prompt): Qwen T=1024 (128 blocks) 61.8 -> 49.8, Mistral T=512 / 1024 44.0 ->
// 40.1 / 79.6 -> 69.3, Gemma-4 T=1024 148.7 -> 97.2; halving: Qwen T=2048 112.7 -> 105.8,
// Mistral 175.8 -> 161.7, Gemma-4 275.0 -> 221.8 (the planner's chunk sizes there, 640
// workgroups at Qwen T=2048, measured slower: 126); Qwen T=4096, beyond: 262 -> 319 with
// chunks. The chunk length (in steps of KSPLIT tiles) is the one among smax, smax/2,
// ... kPrefillMinSteps with the smallest estimated makespan: rounds of kPrefillSlots
// workgroups per CU slot, each costing its steps plus kPrefillFixedSteps (a prologue and
// an epilogue take about 8 us where a step takes 3.4 us).
// Each chunk pays the q fragment, one unhidden staging step and an epilogue.
constexpr int kPrefillFixedSteps = 2;
constexpr int kPrefillMinSteps = 2;
struct PrefillChunks {
    int ctiles = 1 << 30;  // tiles per chunk (one chunk per block: no merge)
    int nchmax = 1;        // most chunks of one block
};
PrefillChunks prefill_chunks(size_t hd, int H, int Hkv, const PrefillRange &r) {
    const PrefillShape sh = prefill_shape(hd, H, H / Hkv, r.rows);
    const int QB = kTile * sh.wph;
    const int ngroups = Hkv * (H / Hkv / sh.hpw);
    const int nqb = (r.rows + QB - 1) / QB;
    auto span = [&](int qb) {  // tiles t0..tE of block qb: tE - t0
        const int p_first = r.qbase + qb * QB;
        const int p_last = r.qbase + std::min(qb * QB + QB, r.rows) - 1;
        const int t0 = r.window > 0 ? std::max(0, p_first - r.window + 1) / kTile : 0;
        return p_last / kTile - t0;
    };
    int smax = 1;
    for (int qb = 0; qb < nqb; ++qb) smax = std::max(smax, span(qb) / sh.ksplit + 1);
    auto units = [&](int cs) {
        long u = 0;
        for (int qb = 0; qb < nqb; ++qb) u += span(qb) / (cs * sh.ksplit) + 1;
        return u * ngroups;
    };
    PrefillChunks ch;
    // (4-wave workgroups at head_dim <= 128 run two per CU)
    const long slots = (sh.hpw * sh.wph * sh.ksplit == 4 && hd <= 128) ? 2 * kPrefillSlots
                                                                        : kPrefillSlots;
    const long blocks = (long)nqb * ngroups;
    if (blocks > slots) return ch;
    if (2 * blocks > slots) {
        // Between half and all of the slots: the blocks of more than half the heaviest
        // one's steps are halved (the merge then reads at most two chunks).
        ch.ctiles = (smax + 1) / 2 * sh.ksplit;
        int nmax = 1;
        for (int qb = 0; qb < nqb; ++qb) nmax = std::max(nmax, span(qb) / ch.ctiles + 1);
        ch.nchmax = nmax;
        return ch;
    }
    // Halving candidates from smax down to kPrefillMinSteps steps, scored by the makespan
    // of rounds of `slots` workgroups, each costing a fixed part (prologue and epilogue,
    // about kPrefillFixedSteps steps) plus its chunk's steps.
    int cs = smax;
    long best = -1;
    for (int c = smax;; c = (c + 1) / 2) {
        const long u = units(c);
        const long cost = (u + slots - 1) / slots * (kPrefillFixedSteps + c);
        if (best < 0 || cost < best) {
            best = cost;
            cs = c;
        }
        if (c <= kPrefillMinSteps) break;
    }
    if (cs >= smax) return ch;
    ch.ctiles = cs * sh.ksplit;
    int nmax = 1;
    for (int qb = 0; qb < nqb; ++qb) nmax = std::max(nmax, span(qb) / ch.ctiles + 1);
    ch.nchmax = nmax;
    return ch;
}

// Workspace: [pre-split records | partial O^T: nchmax x rows x H x hd | partial (m, l, E):
// nchmax x rows x H x 4].
size_t chunk_floats(size_t hd, int H, const PrefillChunks &ch, const PrefillRange &r) {
    return ch.nchmax > 1 ? (size_t)ch.nchmax * r.rows * H * (hd + 4) : 0;
}
size_t workspace_floats(size_t hd, int H, int Hkv, const PrefillRange &r) {
    return presplit_floats(hd, H, Hkv, r) + chunk_floats(hd, H, prefill_chunks(hd, H, Hkv, r), r);
}

template <int HD, int HPW, int WPH, int KSPLIT, bool RANGE, int EB, bool PS, bool FAST = false,
          bool PV1 = false>
eb_status launch_prefill_r(hipStream_t st, const float *q, const void *k, const void *v,
                           const float *ps, float *o, int H, int Hkv, const PrefillRange &r,
                           float scale_log2, const PrefillChunks &ch, float *part_acc,
                           float *part_ml) {
    using C = PrefillCfg<HD, HPW, WPH, KSPLIT>;
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(
            reinterpret_cast<const void *>(
                &prefill_kernel<HD, HPW, WPH, KSPLIT, RANGE, EB, PS, FAST, PV1>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)prefill_lds_bytes<C, FAST, PS>());
    });
    if (attr_err != hipSuccess) return eb::hip_fail(attr_err, "hipFuncSetAttribute(prefill)");
    const int g = H / Hkv;
    const int ngroups = Hkv * (g / HPW);
    const int nqb = (r.rows + C::QB - 1) / C::QB;
    const dim3 grid((unsigned)(nqb * ngroups), (unsigned)ch.nchmax);
    prefill_kernel<HD, HPW, WPH, KSPLIT, RANGE, EB, PS, FAST, PV1>
        <<<grid, C::THREADS, prefill_lds_bytes<C, FAST, PS>(), st>>>(
        q, k, v, ps, presplit_tlo(r), presplit_nt(r), o, H, Hkv, r.rows, r.nkeys, r.qbase,
        r.window, scale_log2, nqb, ngroups, ch.ctiles, part_acc, part_ml, r.hdr);
    eb_status err = eb::check_launch("attn_prefill");
    if (err != EB_OK || ch.nchmax <= 1) return err;
    constexpr int PER = 256 / (HD >= 4 ? HD / 4 : 1);
    const unsigned mblocks = (unsigned)(((size_t)r.rows * H + PER - 1) / PER);
    prefill_merge_kernel<HD><<<mblocks, 256, 0, st>>>(part_acc, part_ml, o, r.rows, H, C::QB,
                                                      r.qbase, r.window, ch.ctiles, r.hdr);
    return eb::check_launch("attn_prefill (chunk merge)");
}

// PV1: the scores-accurate mode (prompts from position 0 over f32 K/V only).
template <int HD, int HPW, int WPH, int KSPLIT, bool PV1 = false>
eb_status launch_prefill_t(hipStream_t st, const float *q, const void *k, const void *v,
                           float *o, int H, int Hkv, const PrefillRange &r, float scale_log2) {
    const bool plain = r.qbase == 0 && r.window == 0;
    // r.ws non-null: sized for workspace_floats (pre-split records, then key-chunk partials)
    const size_t ps_floats = r.ws ? presplit_floats(HD, H, Hkv, r) : 0;
    const PrefillChunks ch = r.ws ? prefill_chunks(HD, H, Hkv, r) : PrefillChunks{};
    float *part_acc = ch.nchmax > 1 ? r.ws + ps_floats : nullptr;
    float *part_ml = part_acc ? part_acc + (size_t)ch.nchmax * r.rows * H * HD : nullptr;
    if constexpr (PrefillCfg<HD, HPW, WPH, KSPLIT>::SPV) {
        if (ps_floats > 0) {
            const int nt = presplit_nt(r);
            float *ps = r.ws;
            const dim3 grid((unsigned)nt, (unsigned)Hkv);
            // f32 K/V beyond half the Infinity Cache are read with non-temporal loads
            // (measured over chunks of 128-256 rows: 268 MB of cache -3 to -7 %, 67 MB
            // unchanged; prompts and caches of 33 MB, likely still cached after their
            // write, 1-5 % slower with them).
            const bool stream = (size_t)nt * kTile * Hkv * r.hdr * 4 * 2 > kPresplitStreamBytes;
            if (PV1 && stream)
                presplit_kernel<HD, 4, true, true><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            else if (PV1)
                presplit_kernel<HD, 4, false, true><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            else if (r.ce == eb::CacheElem::F16)
                presplit_kernel<HD, 2, false><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            else if (r.ce == eb::CacheElem::E4M3)
                presplit_kernel<HD, 1, false><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            else if (stream)
                presplit_kernel<HD, 4, true><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            else
                presplit_kernel<HD, 4, false><<<grid, PresplitCfg<HD>::THREADS, 0, st>>>(
                    k, v, ps, r.nkeys, Hkv, presplit_tlo(r), nt, r.hdr);
            const eb_status err = eb::check_launch("attn_prefill (pre-split)");
            if (err != EB_OK) return err;
            // (the records are f16 hi/lo splits whatever the cache's element type)
            if constexpr (PV1) {
                return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, true, false, true>(
                    st, q, k, v, ps, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
            } else {
                if (plain && r.ce == eb::CacheElem::F32)
                    return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, true>(
                        st, q, k, v, ps, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
                return launch_prefill_r<HD, HPW, WPH, KSPLIT, true, 4, true>(
                    st, q, k, v, ps, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
            }
        }
    }
    if constexpr (PV1)
        return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, false, false, true>(
            st, q, k, v, nullptr, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
    if (r.ce == eb::CacheElem::F16)
        return launch_prefill_r<HD, HPW, WPH, KSPLIT, true, 2, false>(
            st, q, k, v, nullptr, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
    if (r.ce == eb::CacheElem::E4M3)
        return launch_prefill_r<HD, HPW, WPH, KSPLIT, true, 1, false>(
            st, q, k, v, nullptr, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
    if (plain)
        return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, false>(
            st, q, k, v, nullptr, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
    return launch_prefill_r<HD, HPW, WPH, KSPLIT, true, 4, false>(
        st, q, k, v, nullptr, o, H, Hkv, r, scale_log2, ch, part_acc, part_ml);
}

// head_dim <= 128:
//  - 4 query heads per KV head or more: 4 heads x 32 rows, as 4 waves without a key split
//    (two workgroups per CU) when the grid is more than one round of those, else as 8
//    waves with two key splits (prefill_shape).
//  - otherwise: 8 waves (2 per SIMD) = 4 (head, 32-row) slots x 2 key splits, which
//    halves the longest per-wave chain where the blocks are 64 or 128 rows tall.
// head_dim 256: the Q fragment and O^T accumulators take ~450 registers per lane, so one
// wave per SIMD: 4 waves, no key split. (prefill_shape restates this choice.)
template <int HD, bool PV1 = false>
eb_status launch_prefill_hd(hipStream_t st, const float *q, const void *k, const void *v,
                            float *o, int H, int Hkv, const PrefillRange &r,
                            float scale_log2) {
    const int g = H / Hkv;
    constexpr int KSPLIT = HD <= 128 ? 2 : 1;
    if (g % 4 == 0) {
        if (KSPLIT == 2 && prefill_shape(HD, H, g, r.rows).ksplit == 2)
            return launch_prefill_t<HD, 4, 1, KSPLIT, PV1>(st, q, k, v, o, H, Hkv, r, scale_log2);
        return launch_prefill_t<HD, 4, 1, 1, PV1>(st, q, k, v, o, H, Hkv, r, scale_log2);
    }
    if (g % 2 == 0)
        return launch_prefill_t<HD, 2, 2, KSPLIT, PV1>(st, q, k, v, o, H, Hkv, r, scale_log2);
    return launch_prefill_t<HD, 1, 4, KSPLIT, PV1>(st, q, k, v, o, H, Hkv, r, scale_log2);
}

// pv1: the scores-accurate mode (PV1 kernels; prompts over f32 K/V, head dims >= 24).
eb_status launch_prefill_range(hipStream_t st, const float *q, const void *k, const void *v,
                               float *o, size_t h, size_t hkv, size_t hd, float scale,
                               const PrefillRange &r, bool pv1 = false) {
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o)) & 15)
        return eb::fail(EB_UNSUPPORTED_CONFIG, "attn_prefill: q/k/v/o must be 16-byte aligned");
    const float sl2 = scale * eb::kLog2e;
    const int H = (int)h, Hk = (int)hkv;
    PrefillRange rr = r;
    rr.hdr = (int)hd;
    const size_t hp = padded_hd(hd);
    const size_t need = workspace_floats(hp, H, Hk, r);
    if (need == 0 || !r.ws || r.ws_floats < need || (reinterpret_cast<uintptr_t>(r.ws) & 15))
        rr.ws = nullptr;  // no pre-split pass (split while staging), no key chunks
    if (pv1) {
        if (r.qbase != 0 || r.window != 0 || r.ce != eb::CacheElem::F32)
            return eb::fail(EB_UNSUPPORTED_CONFIG,
                            "attn_prefill_pv16: prompts from position 0 over f32 K/V only");
        switch (hp) {
            case 32: return launch_prefill_hd<32, true>(st, q, k, v, o, H, Hk, rr, sl2);
            case 64: return launch_prefill_hd<64, true>(st, q, k, v, o, H, Hk, rr, sl2);
            case 128: return launch_prefill_hd<128, true>(st, q, k, v, o, H, Hk, rr, sl2);
            case 256: return launch_prefill_hd<256, true>(st, q, k, v, o, H, Hk, rr, sl2);
            default:
                return eb::fail(EB_UNSUPPORTED_CONFIG, "attn_prefill_pv16: head_dim %zu", hd);
        }
    }
    switch (hp) {
        case 4: return launch_prefill_hd<4>(st, q, k, v, o, H, Hk, rr, sl2);
        case 8: return launch_prefill_hd<8>(st, q, k, v, o, H, Hk, rr, sl2);
        case 16: return launch_prefill_hd<16>(st, q, k, v, o, H, Hk, rr, sl2);
        case 32: return launch_prefill_hd<32>(st, q, k, v, o, H, Hk, rr, sl2);
        case 64: return launch_prefill_hd<64>(st, q, k, v, o, H, Hk, rr, sl2);
        case 128: return launch_prefill_hd<128>(st, q, k, v, o, H, Hk, rr, sl2);
        case 256: return launch_prefill_hd<256>(st, q, k, v, o, H, Hk, rr, sl2);
        default: return eb::fail(EB_UNSUPPORTED_CONFIG, "attn_prefill: head_dim %zu", hd);
    }
}

// The single-product f16 mode for prompts from position 0 (no window), f32 q/k/v, head
// dims 32..256 (padded to 64 / 128 / 256 as the accurate path does).
// f16-mode records: floats of workspace for this shape (0: the mode stages f32 K/V itself).
// Like the pre-split pass, the pre-convert pass pays where at least 3 query blocks share the
// keys; head dims above 128 stage directly.
size_t fast_workspace_floats(size_t hp, int H, int Hkv, int s) {
    if (hp < 32 || hp > 128 || s <= 0) return 0;
    const int qb_rows = kTile * prefill_shape(hp, H, H / Hkv, s).wph;
    if ((s + qb_rows - 1) / qb_rows < kPresplitMinBlocks) return 0;
    const size_t rec = hp == 32 ? PrefillCfg<32, 4, 1, 1>::FPS_FLOATS
                       : hp == 64 ? PrefillCfg<64, 4, 1, 1>::FPS_FLOATS
                                  : PrefillCfg<128, 4, 1, 1>::FPS_FLOATS;
    const size_t nt = (size_t)((s + kTile - 1) / kTile);
    return (size_t)Hkv * nt * rec;
}

// FAST3 (4-wave workgroups without a key split, three per CU) where the grid fills at least
// one round of those slots; below, the causal triangle's longest blocks would leave CUs idle
// (measured at Qwen T=4096, 512 workgroups: 560 -> 470 TFLOP/s; Mistral T=4096, 1024
// workgroups: 673 -> 738), and the 8-wave key-split shape stays.
constexpr int kFast3PerCu = 3;
bool fast3_shape(size_t hp, int H, int Hkv, int rows) {
    if (!EB_PREFILL_FAST_OCC || hp > 128) return false;
    const int g = H / Hkv;
    const int hpw = g % 4 == 0 ? 4 : g % 2 == 0 ? 2 : 1;
    const long qb_rows = (long)kTile * (4 / hpw);
    const long blocks = (rows + qb_rows - 1) / qb_rows * (long)Hkv * (g / hpw);
    return blocks >= (long)kFast3PerCu * kPrefillSlots;
}

template <int HD, int HPW, int WPH, int KSPLIT>
eb_status launch_prefill_fast_t(hipStream_t st, const float *q, const float *k, const float *v,
                                float *o, int H, int Hkv, const PrefillRange &r, float sl2) {
    const PrefillChunks ch{};
    if constexpr (HD <= 128) {
        if (r.ws) {
            const int nt = presplit_nt(r);
            preconvert_kernel<HD><<<dim3((unsigned)nt, (unsigned)Hkv), PresplitCfg<HD>::THREADS,
                                    0, st>>>(k, v, r.ws, r.nkeys, Hkv, nt, r.hdr);
            const eb_status err = eb::check_launch("attn_prefill_fast (pre-convert)");
            if (err != EB_OK) return err;
            return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, true, true>(
                st, q, k, v, r.ws, o, H, Hkv, r, sl2, ch, nullptr, nullptr);
        }
    }
    return launch_prefill_r<HD, HPW, WPH, KSPLIT, false, 4, false, true>(
        st, q, k, v, nullptr, o, H, Hkv, r, sl2, ch, nullptr, nullptr);
}

template <int HD>
eb_status launch_prefill_fast_hd(hipStream_t st, const float *q, const float *k, const float *v,
                                 float *o, int H, int Hkv, const PrefillRange &r, float sl2) {
    const int g = H / Hkv;
    constexpr int KSPLIT = HD <= 128 ? 2 : 1;
    if (fast3_shape(HD, H, Hkv, r.rows)) {  // FAST3: no key split, three per CU
        if (g % 4 == 0) return launch_prefill_fast_t<HD, 4, 1, 1>(st, q, k, v, o, H, Hkv, r, sl2);
        if (g % 2 == 0) return launch_prefill_fast_t<HD, 2, 2, 1>(st, q, k, v, o, H, Hkv, r, sl2);
        return launch_prefill_fast_t<HD, 1, 4, 1>(st, q, k, v, o, H, Hkv, r, sl2);
    }
    if (g % 4 == 0) {  // (the accurate path's choice, prefill_shape)
        if (KSPLIT == 2 && prefill_shape(HD, H, g, r.rows).ksplit == 2)
            return launch_prefill_fast_t<HD, 4, 1, KSPLIT>(st, q, k, v, o, H, Hkv, r, sl2);
        return launch_prefill_fast_t<HD, 4, 1, 1>(st, q, k, v, o, H, Hkv, r, sl2);
    }
    if (g % 2 == 0) return launch_prefill_fast_t<HD, 2, 2, KSPLIT>(st, q, k, v, o, H, Hkv, r, sl2);
    return launch_prefill_fast_t<HD, 1, 4, KSPLIT>(st, q, k, v, o, H, Hkv, r, sl2);
}

}  // namespace

namespace eb {

size_t prefill_fast_workspace_floats(size_t h, size_t hkv, size_t hd, size_t s) {
    if (hkv == 0 || h % hkv != 0 || s == 0) return 0;
    return fast_workspace_floats(padded_hd(hd), (int)h, (int)hkv, (int)s);
}

eb_status launch_attn_prefill_fast(hipStream_t st, const float *q, const float *k, const float *v,
                                   float *o, size_t h, size_t hkv, size_t s, size_t hd,
                                   float scale, float *ws, size_t ws_floats) {
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o) |
         reinterpret_cast<uintptr_t>(ws)) & 15)
        return eb::fail(EB_UNSUPPORTED_CONFIG,
                        "attn_prefill_fast: q/k/v/o/workspace must be 16-byte aligned");
    const size_t need = prefill_fast_workspace_floats(h, hkv, hd, s);
    if (need == 0 || ws_floats < need) ws = nullptr;  // stage f32 K/V in every workgroup
    const PrefillRange r{(int)s, (int)s, 0, 0, CacheElem::F32, ws, ws_floats, (int)hd};
    const float sl2 = scale * kLog2e;
    switch (padded_hd(hd)) {
        case 32: return launch_prefill_fast_hd<32>(st, q, k, v, o, (int)h, (int)hkv, r, sl2);
        case 64: return launch_prefill_fast_hd<64>(st, q, k, v, o, (int)h, (int)hkv, r, sl2);
        case 128: return launch_prefill_fast_hd<128>(st, q, k, v, o, (int)h, (int)hkv, r, sl2);
        case 256: return launch_prefill_fast_hd<256>(st, q, k, v, o, (int)h, (int)hkv, r, sl2);
        default:
            return eb::fail(EB_UNSUPPORTED_CONFIG,
                            "attn_prefill_fast: head_dim %zu (24 to 256)", hd);
    }
}

size_t prefill_workspace_floats(size_t h, size_t hkv, size_t hd, size_t rows, size_t nkeys,
                                size_t qbase, size_t window) {
    if (rows == 0 || hkv == 0 || h % hkv != 0) return 0;
    return workspace_floats(padded_hd(hd), (int)h, (int)hkv,
                            PrefillRange{(int)rows, (int)nkeys, (int)qbase, (int)window, CacheElem::F32,
                                         nullptr, 0, (int)hd});
}

eb_status launch_attn_prefill(hipStream_t st, const float *q, const float *k, const float *v,
                              float *o, size_t h, size_t hkv, size_t s, size_t hd, float scale,
                              float *ws, size_t ws_floats) {
    return launch_prefill_range(st, q, k, v, o, h, hkv, hd, scale,
                                PrefillRange{(int)s, (int)s, 0, 0, CacheElem::F32, ws, ws_floats, (int)hd});
}

eb_status launch_attn_prefill_pv16(hipStream_t st, const float *q, const float *k,
                                   const float *v, float *o, size_t h, size_t hkv, size_t s,
                                   size_t hd, float scale, float *ws, size_t ws_floats) {
    return launch_prefill_range(st, q, k, v, o, h, hkv, hd, scale,
                                PrefillRange{(int)s, (int)s, 0, 0, CacheElem::F32, ws, ws_floats, (int)hd},
                                true);
}

eb_status launch_attn_prefill_chunk(hipStream_t st, const float *q, const float *kc,
                                    const float *vc, float *o, size_t h, size_t hkv,
                                    size_t pos0, size_t rows, size_t hd, float scale,
                                    size_t window, float *ws, size_t ws_floats) {
    return launch_prefill_range(st, q, kc, vc, o, h, hkv, hd, scale,
                                PrefillRange{(int)rows, (int)(pos0 + rows), (int)pos0,
                                             (int)window, CacheElem::F32, ws, ws_floats,
                                             (int)hd});
}

eb_status launch_attn_prefill_chunk_cache(hipStream_t st, const float *q, const void *kc,
                                          const void *vc, float *o, size_t h, size_t hkv,
                                          size_t pos0, size_t rows, size_t hd, float scale,
                                          size_t window, CacheElem ce, float *ws,
                                          size_t ws_floats) {
    return launch_prefill_range(st, q, kc, vc, o, h, hkv, hd, scale,
                                PrefillRange{(int)rows, (int)(pos0 + rows), (int)pos0,
                                             (int)window, ce, ws, ws_floats, (int)hd});
}

}  // namespace eb
