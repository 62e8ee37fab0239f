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

}  // namespace eb
