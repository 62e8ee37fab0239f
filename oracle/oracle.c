/*
 * CPU oracle for the eyebrowse attention hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference's own CPU attention path and
 * its helpers. It is the checker the HIP kernels are compared against, and the
 * `cpu_baseline` leg of bench.py times it. Nothing in the product library links,
 * loads or calls it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may use it.
 *
 * The reference is Rust (crates/eyebrowse-kernels/src/testutil.rs) and cannot be
 * compiled in this image (no cargo/rustc), so the functions below follow it loop for
 * loop: same loop order, same 3-pass softmax, f32 accumulation, libm expf/sqrtf.
 * Build with -O2 -ffp-contract=off and without fast-math so that the compiler keeps
 * the f32 operation order (no FMA contraction, no reassociation).
 *
 * Pinning (what each function is checked against) is listed in tests/test_oracle.py
 * next to each test. Every function here has at least one independent check.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* EBO_PLANT selects a deliberately wrong variant for the mutation test in
 * tests/test_oracle.py (it builds a throwaway copy with -DEBO_PLANT=n and checks that
 * the independent checks reject it). The shipped oracle is built with EBO_PLANT = 0. */
#ifndef EBO_PLANT
#define EBO_PLANT 0
#endif

/* Relative L2 error ||a-b|| / (||b|| + 1e-12), accumulated in f64.
 * Follows crates/eyebrowse-kernels/src/testutil.rs:16-26. */
float ebo_rel_l2(const float *a, const float *b, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double d = (double)a[i] - (double)b[i];
        num += d * d;
        den += (double)b[i] * (double)b[i];
    }
    return (float)(sqrt(num) / (sqrt(den) + 1e-12));
}

/* xorshift64 stream in [-1, 1): crates/eyebrowse-nn/src/testutil.rs:30-41.
 * The seed is offset by the golden-ratio constant, shifts are (13, 7, 17), and the top
 * 53 bits become a double in [0, 1). */
void ebo_prng(float *out, size_t n, uint64_t seed) {
    uint64_t s = seed + 0x9E3779B97F4A7C15ull;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        double u = (double)(s >> 11) / (double)(1ull << 53);
        out[i] = (float)(u * 2.0 - 1.0);
    }
}

/* Seeded N(0,1) inputs for the benchmark configs: the same xorshift64 stream as
 * ebo_prng gives uniforms u1 in (0,1] and u2 in [0,1); Box–Muller in f64 then
 * z = sqrt(-2 ln u1) cos(2 pi u2), cast to f32 (one normal per pair of uniforms).
 * This generator is defined by this build (the reference has no normal sampler). */
void ebo_randn(float *out, size_t n, uint64_t seed) {
    uint64_t s = seed + 0x9E3779B97F4A7C15ull;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i) {
        double u[2];
        for (int t = 0; t < 2; ++t) {
            s ^= s << 13;
            s ^= s >> 7;
            s ^= s << 17;
            u[t] = (double)(s >> 11) / (double)(1ull << 53);
        }
        double u1 = 1.0 - u[0]; /* (0, 1]: log is finite */
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u[1]));
    }
}

/* Row RMSNorm over [rows, dim]: y = x * (1/sqrt(sum(x^2)/dim + eps)) * w.
 * Follows crates/eyebrowse-kernels/src/testutil.rs:83-97 (f32 sum of squares in
 * index order, then one reciprocal square root per row). */
void ebo_rmsnorm(const float *x, const float *w, float *out, size_t rows, size_t dim,
                 float eps) {
    for (size_t r = 0; r < rows; ++r) {
        size_t base = r * dim;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; ++i) ss += x[base + i] * x[base + i];
        float inv = 1.0f / sqrtf((ss / (float)dim) + eps);
        for (size_t i = 0; i < dim; ++i) out[base + i] = x[base + i] * inv * w[i];
    }
}

/* Rotary tables [max_seq, hd/2]: angle(s,k) = s * theta^(-2k/hd) in f64 for
 * k < rope_angles, else cos = 1, sin = 0 (pass-through pairs).
 * Follows crates/eyebrowse-nn/src/rope.rs:24-50 (build_partial; build() is
 * rope_angles = hd/2, :18-20). theta arrives as f32 and is widened, as there. */
void ebo_rope_tables(float *cos_out, float *sin_out, size_t max_seq, size_t hd,
                     size_t rope_angles, float theta_f32) {
    size_t half = hd / 2;
    double theta = (double)theta_f32;
    double hdd = (double)hd;
    size_t na = rope_angles < half ? rope_angles : half;
    for (size_t s = 0; s < max_seq; ++s) {
        for (size_t k = 0; k < half; ++k) {
            cos_out[s * half + k] = 1.0f;
            sin_out[s * half + k] = 0.0f;
        }
        for (size_t k = 0; k < na; ++k) {
            double inv_freq = pow(theta, -(2.0 * (double)k) / hdd);
            double angle = (double)s * inv_freq;
            cos_out[s * half + k] = (float)cos(angle);
            sin_out[s * half + k] = (float)sin(angle);
        }
    }
}

/* Half-split RoPE on x [seq, n_heads, hd] with tables [*, hd/2] read at row s+base_pos:
 * x1' = x1 c - x2 s, x2' = x2 c + x1 s for pairs (p, p + hd/2).
 * Follows crates/eyebrowse-kernels/src/testutil.rs:101-125, with the kernel's base_pos
 * offset (crates/eyebrowse-kernels/src/rope.rs:25-26) added; base_pos = 0 is the
 * testutil function exactly. */
void ebo_rope(const float *x, const float *cosb, const float *sinb, float *out, size_t seq,
              size_t n_heads, size_t hd, size_t base_pos) {
    size_t half = hd / 2;
    memcpy(out, x, seq * n_heads * hd * sizeof(float));
    for (size_t s = 0; s < seq; ++s) {
        for (size_t h = 0; h < n_heads; ++h) {
            size_t base = (s * n_heads + h) * hd;
            for (size_t p = 0; p < half; ++p) {
                float c = cosb[(s + base_pos) * half + p];
                float sn = sinb[(s + base_pos) * half + p];
                float x1 = x[base + p];
                float x2 = x[base + half + p];
                out[base + p] = x1 * c - x2 * sn;
                out[base + half + p] = x2 * c + x1 * sn;
            }
        }
    }
}

/* kv_write semantics: cache[((dst + c) * hkv + head) * hd + d] = src[(c * hkv + head) * hd + d]
 * for c < count. Follows the WGSL in crates/eyebrowse-kernels/src/ops.rs:70-87. */
void ebo_kv_write(float *cache, const float *src, size_t hkv, size_t count, size_t hd,
                  size_t dst_start) {
    for (size_t c = 0; c < count; ++c)
        for (size_t head = 0; head < hkv; ++head)
            for (size_t d = 0; d < hd; ++d)
                cache[((dst_start + c) * hkv + head) * hd + d] = src[(c * hkv + head) * hd + d];
}

/* One query row of the reference CPU attention: 3-pass softmax over keys first..=last.
 * Scores: f32 dot with d ascending, then * scale; max; sum of expf(sc - mx); then per
 * key j: w = expf(sc - mx) / sum, o[d] += w * v[d].
 * Follows crates/eyebrowse-kernels/src/testutil.rs:142-169 (prefill) and :190-216
 * (decode), which share this body with first = 0. `scores` is caller scratch of last+1
 * floats. */
static void ebo_attn_row(const float *qrow, const float *k, const float *v, float *orow,
                         size_t hkv, size_t kvh, size_t first, size_t last, size_t hd,
                         float scale, float *scores) {
#if EBO_PLANT == 2 /* planted mistake: causal mask drops the diagonal */
    if (last > 0) last -= 1;
#endif
#if EBO_PLANT == 3 /* planted mistake: scale ignored */
    scale = 1.0f;
#endif
    float mx = -INFINITY;
    for (size_t j = first; j <= last; ++j) {
        const float *kr = k + (j * hkv + kvh) * hd;
        float dot = 0.0f;
        for (size_t d = 0; d < hd; ++d) dot += qrow[d] * kr[d];
        dot *= scale;
        scores[j] = dot;
        mx = fmaxf(mx, dot);
    }
    float sum = 0.0f;
    for (size_t j = first; j <= last; ++j) sum += expf(scores[j] - mx);
    for (size_t d = 0; d < hd; ++d) orow[d] = 0.0f;
    for (size_t j = first; j <= last; ++j) {
        float w = expf(scores[j] - mx) / sum;
#if EBO_PLANT == 4 /* planted mistake: values read from the key tensor */
        const float *vr = k + (j * hkv + kvh) * hd;
        (void)v;
#else
        const float *vr = v + (j * hkv + kvh) * hd;
#endif
        for (size_t d = 0; d < hd; ++d) orow[d] += w * vr[d];
    }
}

/* Causal GQA prefill over rows [row0, row0 + nrows) of the sequence.
 * q [s, h, hd], k/v [s, hkv, hd], o [s, h, hd] (only the requested rows are written).
 * Query head hh uses kv head hh / (h / hkv).
 * Follows crates/eyebrowse-kernels/src/testutil.rs:130-172. The reference hard-codes
 * scale = 1/sqrt(hd) (:140); here scale is an argument so the scale = 1.0 config can
 * run, and ebo_default_scale() gives the reference's value bit for bit. Row subsets
 * compute exactly the same per-row arithmetic as the full function.
 * `threads` > 1 parallelises over (row, head) pairs with OpenMP (the all-core CPU
 * baseline); each pair is computed by the same serial code, so results do not depend
 * on the thread count. */
int ebo_attn_prefill_rows(const float *q, const float *k, const float *v, float *o, size_t h,
                          size_t hkv, size_t s, size_t hd, float scale, size_t row0,
                          size_t nrows, int threads) {
    if (hkv == 0 || h % hkv != 0 || row0 + nrows > s) return -1;
    size_t group = h / hkv;
    long long total = (long long)(nrows * h);
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        float *scores = (float *)malloc((s > 0 ? s : 1) * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (long long t = 0; t < total; ++t) {
            size_t i = row0 + (size_t)t / h;
            size_t hh = (size_t)t % h;
#if EBO_PLANT == 1 /* planted mistake: interleaved instead of contiguous GQA grouping */
            size_t kvh = hh % hkv;
            (void)group;
#else
            size_t kvh = hh / group;
#endif
            size_t qbase = (i * h + hh) * hd;
            ebo_attn_row(q + qbase, k, v, o + qbase, hkv, kvh, 0, i, hd, scale, scores);
        }
        free(scores);
    }
    (void)threads;
    return 0;
}

int ebo_attn_prefill(const float *q, const float *k, const float *v, float *o, size_t h,
                     size_t hkv, size_t s, size_t hd, float scale, int threads) {
    return ebo_attn_prefill_rows(q, k, v, o, h, hkv, s, hd, scale, 0, s, threads);
}

/* Single decode step: q [h, hd] attends keys 0..=pos of a seq-major cache
 * [max_seq, hkv, hd]; o [h, hd]. Follows crates/eyebrowse-kernels/src/testutil.rs:177-218
 * (scale generalised as in ebo_attn_prefill_rows). `threads` parallelises over heads. */
int ebo_attn_decode(const float *q, const float *kc, const float *vc, float *o, size_t h,
                    size_t hkv, size_t pos, size_t hd, size_t max_seq, float scale,
                    int threads) {
    if (hkv == 0 || h % hkv != 0 || pos >= max_seq) return -1;
    size_t group = h / hkv;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        float *scores = (float *)malloc((pos + 1) * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static, 1)
#endif
        for (long long hh = 0; hh < (long long)h; ++hh) {
            size_t kvh = (size_t)hh / group;
            ebo_attn_row(q + (size_t)hh * hd, kc, vc, o + (size_t)hh * hd, hkv, kvh, 0, pos, hd,
                         scale, scores);
        }
        free(scores);
    }
    (void)threads;
    return 0;
}

/* Chunked causal attention with an optional sliding window: query row r < rows of
 * q [rows, h, hd] sits at position p = pos0 + r and attends keys
 * max(0, p - window + 1) ..= p (all of 0..=p when window == 0) of the seq-major k/v
 * [>= pos0 + rows, hkv, hd]; o [rows, h, hd]. The per-row arithmetic is the reference's
 * (testutil.rs:142-169) over that key range: with pos0 = 0 and no window it is
 * ebo_attn_prefill, with rows = 1 and no window ebo_attn_decode at pos0. The reference
 * itself has neither chunked nor windowed attention. */
int ebo_attn_chunk(const float *q, const float *k, const float *v, float *o, size_t h,
                   size_t hkv, size_t pos0, size_t rows, size_t hd, float scale, size_t window,
                   int threads) {
    if (hkv == 0 || h % hkv != 0) return -1;
    size_t group = h / hkv;
    long long total = (long long)(rows * h);
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 1;
#pragma omp parallel num_threads(nt)
#endif
    {
        float *scores = (float *)malloc((pos0 + rows > 0 ? pos0 + rows : 1) * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (long long t = 0; t < total; ++t) {
            size_t r = (size_t)t / h;
            size_t hh = (size_t)t % h;
            size_t p = pos0 + r;
            size_t first = (window > 0 && p + 1 > window) ? p + 1 - window : 0;
            size_t qoff = (r * h + hh) * hd;
            ebo_attn_row(q + qoff, k, v, o + qoff, hkv, hh / group, first, p, hd, scale, scores);
        }
        free(scores);
    }
    (void)threads;
    return 0;
}

/* IEEE binary16 bit pattern -> f32 (exact), from its fields: sign, 5-bit exponent with
 * bias 15, 10-bit fraction; exponent 0 is subnormal (fraction * 2^-24), 31 is inf/NaN. */
float ebo_f16_to_f32(uint16_t h) {
    const int sign = h >> 15, e = (h >> 10) & 31, f = h & 1023;
    float v;
    if (e == 0)
        v = ldexpf((float)f, -24);
    else if (e == 31)
        v = f ? NAN : INFINITY;
    else
        v = ldexpf((float)(1024 + f), e - 25);
    return sign ? -v : v;
}

/* OCP FP8 E4M3 ("e4m3fn": 1 sign bit, 4 exponent bits with bias 7, 3 fraction bits, no
 * infinities, S.1111.111 is NaN, largest finite 448) bit pattern -> f32, from its fields
 * (exact: every E4M3 value is an f32). Exponent 0 is subnormal: fraction * 2^-9. No
 * counterpart in the reference, whose caches are f32. */
float ebo_f8e4m3_to_f32(uint8_t b) {
    const int sign = b >> 7, e = (b >> 3) & 15, f = b & 7;
    float v;
    if (e == 15 && f == 7)
        v = NAN;
    else if (e == 0)
        v = ldexpf((float)f, -9);
    else
        v = ldexpf((float)(8 + f), e - 10);
    return sign ? -v : v;
}

/* f32 -> E4M3 bit pattern, the FP8 cache's kv_write contract: the nearest E4M3 value, ties
 * to the even fraction; finite values at or beyond 448 (the largest) saturate to +-448;
 * inf and NaN become NaN (0x7F with the sign); the sign of zero is kept. Computed on the
 * value grid: below 2^-6 the step is 2^-9, in [2^e, 2^(e+1)) it is 2^(e-3); the count of
 * steps is rounded to nearest even in double (exact: the quotient has at most 24 bits). */
uint8_t ebo_f8e4m3_bits(float x) {
    const uint8_t s = signbit(x) ? 0x80 : 0;
    if (isnan(x) || isinf(x)) return s | 0x7F;
    const double a = fabs((double)x);
    if (a >= 448.0) return s | 0x7E;
    if (a == 0.0) return s;
    int e;
    frexp(a, &e);  /* a = m 2^e, m in [0.5, 1): a in [2^(e-1), 2^e) */
    e -= 1;
    if (e < -6) e = -6;
    const double step = ldexp(1.0, e - 3);
    const double v = rint(a / step) * step;  /* the nearest grid value, ties to even */
    if (v < ldexp(1.0, -6)) return s | (uint8_t)(v / ldexp(1.0, -9));
    int ev;
    const double m = frexp(v, &ev);  /* v = m 2^ev, m in [0.5, 1) */
    const int E = ev - 1 + 7;
    const int F = (int)((2.0 * m - 1.0) * 8.0);
    return (uint8_t)(s | (E << 3) | F);
}

void ebo_f8e4m3_bits_n(const float *x, uint8_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ebo_f8e4m3_bits(x[i]);
}

void ebo_f8e4m3_to_f32_n(const uint8_t *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ebo_f8e4m3_to_f32(b[i]);
}

/* linear_f16w's CPU reference (crates/eyebrowse-kernels/src/testutil.rs:68-80, the
 * weight rounded to f16 as the kernel reads it, matmul.rs:246-247,266-267):
 * y[i, o] = sum_k x[i, k] * w[o, k], f32 accumulation with k ascending. w holds the
 * f16 bit patterns of the logical [out_f, in_f] weight in flat order: the reference's
 * packed-u32 layout (tensor.rs:7-23, low half first) read as little-endian u16. */
void ebo_linear_f16w(const float *x, const uint16_t *w, float *y, size_t m, size_t in_f,
                     size_t out_f, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static) collapse(2)
    for (size_t i = 0; i < m; ++i)
        for (size_t o = 0; o < out_f; ++o) {
            float acc = 0.0f;
            for (size_t k = 0; k < in_f; ++k) {
#if EBO_PLANT == 5 /* planted mistake: weight read transposed ([in, out]) */
                acc += x[i * in_f + k] * ebo_f16_to_f32(w[k * out_f + o]);
#else
                acc += x[i * in_f + k] * ebo_f16_to_f32(w[o * in_f + k]);
#endif
            }
            y[i * out_f + o] = acc;
        }
}

/* argmax (crates/eyebrowse-kernels/src/sampling.rs:6-38) restated step by step: 256
 * lanes, lane t scans i = t, t+256, ... keeping the first strictly larger value (start
 * -3e38, so NaN and values <= -3e38 never win, index 0 if nothing does); then a tree
 * over the lanes, strides 128..1, where the right lane replaces the left only if its
 * value is strictly larger. Ties therefore go to the lane (i mod 256) that comes first
 * in bit-reversed order, then to the smallest i. */
uint32_t ebo_argmax(const float *x, size_t n) {
    float bv[256];
    uint32_t bi[256];
    for (size_t t = 0; t < 256; ++t) {
        bv[t] = -3.0e38f;
        bi[t] = 0;
        for (size_t i = t; i < n; i += 256)
            if (x[i] > bv[t]) {
                bv[t] = x[i];
                bi[t] = (uint32_t)i;
            }
    }
    for (size_t stride = 128; stride > 0; stride >>= 1)
        for (size_t t = 0; t < stride; ++t)
            if (bv[t + stride] > bv[t]) {
                bv[t] = bv[t + stride];
                bi[t] = bi[t + stride];
            }
    return bi[0];
}

/* The reference's hard-coded scale: 1.0 / (hd as f32).sqrt()
 * (crates/eyebrowse-kernels/src/testutil.rs:140,188). */
float ebo_default_scale(size_t hd) { return 1.0f / sqrtf((float)hd); }

/* Number of OpenMP threads the library would use by default (1 when built without it). */
int ebo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
