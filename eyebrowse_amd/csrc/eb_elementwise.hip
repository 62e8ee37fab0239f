// kv_write and RMSNorm for gfx950: memory-bound steps around attention (RoPE and the
// per-head pre-attention pass are in eb_rows.hip). kv_write also fills IEEE-half and OCP
// FP8 E4M3 caches (rounded to nearest even; E4M3 saturating at +-448).
//
//  kv_write  (crates/eyebrowse-kernels/src/ops.rs:70-87,150-179): both sides are
//            seq-major, so the write is one contiguous copy of count*hkv*hd floats to
//            element offset dst*hkv*hd. 128-bit loads/stores when aligned; pure copies,
//            so the result is bit-exact.
//  rmsnorm   (crates/eyebrowse-kernels/src/rmsnorm.rs:6-64): one wave per row, the sum of
//            squares reduced across the wave, y = x * (1/sqrt(ss/dim + eps)) * w.
#include "eb_common.h"
#include "eb_internal.h"

namespace {

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void kv_write_vec4_kernel(float4 *__restrict__ dst,
                                                               const float4 *__restrict__ src,
                                                               size_t n4) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(kBlock) void kv_write_scalar_kernel(float *__restrict__ dst,
                                                                 const float *__restrict__ src,
                                                                 size_t n) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// f32 rows into an IEEE-half cache: round to nearest even (v_cvt_f16_f32), four
// elements per thread (16 bytes read, 8 written); n4 = elements / 4.
__global__ __launch_bounds__(kBlock) void kv_write_f16_kernel(f16x4 *__restrict__ dst,
                                                              const f32x4 *__restrict__ src,
                                                              size_t n4) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride)
        dst[i] = __builtin_convertvector(src[i], f16x4);
}

// f32 rows into an E4M3 cache (eb::f8e4m3_bits: nearest even, saturating), four elements
// per thread (16 bytes read, 4 written); n4 = elements / 4.
__global__ __launch_bounds__(kBlock) void kv_write_f8_kernel(unsigned *__restrict__ dst,
                                                             const f32x4 *__restrict__ src,
                                                             size_t n4) {
    const size_t stride = (size_t)gridDim.x * kBlock;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride)
        dst[i] = eb::f8x4_bits(src[i]);
}

unsigned copy_grid(size_t n) {
    size_t blocks = (n + kBlock - 1) / kBlock;
    if (blocks > 4096) blocks = 4096;  // grid-stride beyond 16 blocks per CU
    return blocks == 0 ? 1u : (unsigned)blocks;
}

// One wave per row; rows_per_block rows per 256-thread block.
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const float *__restrict__ x,
                                                         const float *__restrict__ w,
                                                         float *__restrict__ out, unsigned rows,
                                                         unsigned dim, float eps) {
    const unsigned lane = threadIdx.x & 63;
    const unsigned row = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + (size_t)row * dim;
    float ss = 0.0f;
    for (unsigned i = lane; i < dim; i += 64) {
        float t = xr[i];
        ss += t * t;
    }
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    float *orow = out + (size_t)row * dim;
    for (unsigned i = lane; i < dim; i += 64) orow[i] = xr[i] * inv * w[i];
}

// Self-check of the wave lane exchanges that every reduction in these kernels is built
// from (eb_common.h), on one wave: row r of out holds lane_xor16, lane_xor32, the class
// reductions for FROM = 1, 2, 4, 8, 16, 32 (sums) and 1, 8 (maxima), swap_sum32 and
// swap_sum16 of (a, b), and group_sum over 4 and 16 lanes, for a = in[0..64) and
// b = in[64..128).
__global__ __launch_bounds__(64) void lane_ops_kernel(const float *__restrict__ in,
                                                      float *__restrict__ out) {
    const int l = threadIdx.x;
    const float a = in[l], b = in[64 + l];
    float r[EB_LANE_OPS_ROWS];
    r[0] = eb::lane_xor16(a);
    r[1] = eb::lane_xor32(a);
    r[2] = eb::class_reduce<1, false>(a);
    r[3] = eb::class_reduce<2, false>(a);
    r[4] = eb::class_reduce<4, false>(a);
    r[5] = eb::class_reduce<8, false>(a);
    r[6] = eb::class_reduce<16, false>(a);
    r[7] = eb::class_reduce<32, false>(a);
    r[8] = eb::class_reduce<1, true>(a);
    r[9] = eb::class_reduce<8, true>(a);
    r[10] = eb::swap_sum32(a, b);
    r[11] = eb::swap_sum16(a, b);
    r[12] = eb::group_sum<4>(a);
    r[13] = eb::group_sum<16>(a);
#pragma unroll
    for (int i = 0; i < EB_LANE_OPS_ROWS; ++i) out[i * 64 + l] = r[i];
}

}  // namespace

namespace eb {

eb_status launch_kv_write(hipStream_t st, float *cache, const float *src, size_t hkv,
                          size_t count, size_t hd, size_t dst_start) {
    size_t n = count * hkv * hd;
    float *dst = cache + dst_start * hkv * hd;
    bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    if (aligned && n % 4 == 0) {
        size_t n4 = n / 4;
        kv_write_vec4_kernel<<<copy_grid(n4), kBlock, 0, st>>>(
            reinterpret_cast<float4 *>(dst), reinterpret_cast<const float4 *>(src), n4);
    } else {
        kv_write_scalar_kernel<<<copy_grid(n), kBlock, 0, st>>>(dst, src, n);
    }
    return check_launch("kv_write");
}

eb_status launch_kv_write_f16(hipStream_t st, uint16_t *cache, const float *src, size_t hkv,
                              size_t count, size_t hd, size_t dst_start) {
    const size_t n = count * hkv * hd;  // hd is a multiple of 4
    uint16_t *dst = cache + dst_start * hkv * hd;
    if (((reinterpret_cast<uintptr_t>(dst) & 7) | (reinterpret_cast<uintptr_t>(src) & 15)) != 0)
        return fail(EB_UNSUPPORTED_CONFIG, "kv_write: f16 cache / src must be 8 / 16-byte aligned");
    const size_t n4 = n / 4;
    kv_write_f16_kernel<<<copy_grid(n4), kBlock, 0, st>>>(
        reinterpret_cast<f16x4 *>(dst), reinterpret_cast<const f32x4 *>(src), n4);
    return check_launch("kv_write_f16");
}

eb_status launch_kv_write_f8(hipStream_t st, uint8_t *cache, const float *src, size_t hkv,
                             size_t count, size_t hd, size_t dst_start) {
    const size_t n = count * hkv * hd;  // hd is a multiple of 4
    uint8_t *dst = cache + dst_start * hkv * hd;
    if (((reinterpret_cast<uintptr_t>(dst) & 3) | (reinterpret_cast<uintptr_t>(src) & 15)) != 0)
        return fail(EB_UNSUPPORTED_CONFIG, "kv_write: e4m3 cache / src must be 4 / 16-byte aligned");
    const size_t n4 = n / 4;
    kv_write_f8_kernel<<<copy_grid(n4), kBlock, 0, st>>>(
        reinterpret_cast<unsigned *>(dst), reinterpret_cast<const f32x4 *>(src), n4);
    return check_launch("kv_write_f8");
}

eb_status launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *out,
                         size_t rows, size_t dim, float eps) {
    unsigned blocks = (unsigned)((rows + 3) / 4);
    rmsnorm_kernel<<<blocks, kBlock, 0, st>>>(x, w, out, (unsigned)rows, (unsigned)dim, eps);
    return check_launch("rmsnorm");
}

eb_status launch_lane_ops(hipStream_t st, const float *in, float *out) {
    lane_ops_kernel<<<1, 64, 0, st>>>(in, out);
    return check_launch("lane_ops");
}

}  // namespace eb
