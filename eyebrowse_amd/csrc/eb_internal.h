// Shared internals of libeyebrowse_hip: error plumbing, validation helpers and the
// launch functions each kernel translation unit exports to the runtime.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "eyebrowse_hip.h"

namespace eb {

// Records a formatted message as this thread's last error and returns `st`.
eb_status fail(eb_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears this thread's last error and returns EB_OK.
eb_status ok();
// Maps a HIP error to a status (hipErrorOutOfMemory -> EB_OUT_OF_MEMORY, else EB_OTHER)
// and records `what` plus HIP's own message.
eb_status hip_fail(hipError_t e, const char *what);

#define EB_HIP_TRY(expr)                                              \
    do {                                                              \
        hipError_t eb_e_ = (expr);                                    \
        if (eb_e_ != hipSuccess) return ::eb::hip_fail(eb_e_, #expr); \
    } while (0)

// After a launch: reports a launch-configuration error as EB_OTHER.
eb_status check_launch(const char *kernel);

// Shared argument checks. Each returns EB_OK or records why the shape is refused.
eb_status check_ptr(const void *p, const char *name);
eb_status check_numel(size_t have, size_t need, const char *name);
eb_status check_heads(size_t h, size_t hkv);
// Head dims the attention kernels serve: 4, every multiple of 8 up to 128 and every multiple
// of 16 up to 256. Decode is instantiated for each (X-macro below); prefill runs the next
// power-of-two instantiation with the extra dims read as zeros and never stored.
bool attn_head_dim_supported(size_t hd);
#define EB_HEAD_DIMS(X) \
    X(4) X(8) X(16) X(24) X(32) X(40) X(48) X(56) X(64) X(72) X(80) X(88) X(96) X(104) \
    X(112) X(120) X(128) X(144) X(160) X(176) X(192) X(208) X(224) X(240) X(256)
// Largest element count a 32-bit-indexed kernel may address.
constexpr size_t kMaxIndex = (size_t)1 << 31;

// The device that owns a tensor.
eb_device *tensor_device(const eb_tensor *t);

// Compute units of the current device (cached per ordinal).
int current_cu_count();

// Element types a KV cache may hold; the value is the element size in bytes. F32 is the
// reference's; F16 is IEEE half and E4M3 OCP FP8 E4M3 (both rounded to nearest even by
// kv_write, E4M3 saturating at +-448), converted to f32 as attention loads them.
enum class CacheElem : int { F32 = 4, F16 = 2, E4M3 = 1 };
// Whether the fused decode step can apply RoPE inside its lane layout: over IEEE-half and
// E4M3 caches a lane's 8-dim loads sit at multiples of 8 dims, and at head dims that are odd
// multiples of 8 a dim's RoPE partner (dim + hd/2) is not on the same lane.
inline bool decode_fuses_rope(size_t hd, CacheElem ce) {
    return ce == CacheElem::F32 || hd % 16 == 0;
}

// ---- kernel launchers (validated arguments, caller's stream) -------------------------
eb_status launch_kv_write(hipStream_t st, float *cache, const float *src, size_t hkv,
                          size_t count, size_t hd, size_t dst_start);
// Prefill workspace: floats of the pre-split K/V records and of the key-chunk partials for
// this shape (0: neither is used). Launches given at least that much (16-byte aligned)
// run the pre-split pass and split the keys into chunks where that pays; with less they
// do neither. No initialisation needed.
size_t prefill_workspace_floats(size_t h, size_t hkv, size_t hd, size_t rows, size_t nkeys,
                                size_t qbase, size_t window);
eb_status launch_attn_prefill(hipStream_t st, const float *q, const float *k, const float *v,
                              float *o, size_t h, size_t hkv, size_t s, size_t hd,
                              float scale, float *ws = nullptr, size_t ws_floats = 0);
// The scores-accurate mode: as launch_attn_prefill, with O^T += V^T P^T as one f16 product
// (head dims 24..256).
eb_status launch_attn_prefill_pv16(hipStream_t st, const float *q, const float *k,
                                   const float *v, float *o, size_t h, size_t hkv, size_t s,
                                   size_t hd, float scale, float *ws, size_t ws_floats);
// The single-product f16 prefill (opt-in): q, K, V and P rounded to f16 once, one f16 MFMA
// per product, f32 softmax and accumulation. Prompts from position 0, f32 q/k/v, head dims
// 32..256 (multiples of 16); no workspace.
// With a workspace of prefill_fast_workspace_floats (16-byte aligned), a pre-convert pass
// rounds K/V to f16 once into records that the attention kernel copies (head_dim <= 128,
// at least 3 query blocks); otherwise every workgroup converts the f32 rows it stages.
size_t prefill_fast_workspace_floats(size_t h, size_t hkv, size_t hd, size_t s);
eb_status launch_attn_prefill_fast(hipStream_t st, const float *q, const float *k, const float *v,
                                   float *o, size_t h, size_t hkv, size_t s, size_t hd,
                                   float scale, float *ws = nullptr, size_t ws_floats = 0);
// Chunked causal prefill: q rows at positions pos0..pos0+rows-1 attend cache keys
// max(0, p - window + 1)..p (window 0: 0..p); kc/vc are the cache bases.
eb_status launch_attn_prefill_chunk(hipStream_t st, const float *q, const float *kc,
                                    const float *vc, float *o, size_t h, size_t hkv,
                                    size_t pos0, size_t rows, size_t hd, float scale,
                                    size_t window, float *ws = nullptr, size_t ws_floats = 0);
// Decode workspace: part_acc [nsplit*h*hd] | part_ml [nsplit*h*2], no initialisation.
size_t decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count,
                               CacheElem ce = CacheElem::F32);
// The largest of the f32, IEEE-half and E4M3 plans' workspaces (the plans split the keys
// differently: their iterations hold different numbers of rows).
size_t decode_workspace_floats_any(size_t h, size_t hkv, size_t pos, size_t hd, int cu_count);
// knew/vnew null: plain attention over keys 0..=pos. Otherwise key `pos` comes from
// knew/vnew ([hkv, hd]) and is also written to cache row `pos` through kc_w/vc_w.
// window > 0 limits the keys to pos - window + 1..=pos. A workspace sized for
// decode_workspace_floats(h, hkv, pos, ...) is enough for any window.
eb_status launch_attn_decode(hipStream_t st, const float *q, const float *kc, const float *vc,
                             float *kc_w, float *vc_w, const float *knew, const float *vnew,
                             float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                             float scale, float *ws, size_t ws_floats, int cu_count,
                             size_t window = 0);
// eb_launch_attn_decode_step after its arguments are resolved: shape checks, the
// workspace size check (workspace_floats must cover decode_workspace_floats), the launch.
// One wave of lane-exchange results (eb_elementwise.hip, eb_launch_selftest_lane_ops).
eb_status launch_lane_ops(hipStream_t st, const float *in, float *out);

// The calling thread's current device's address of the no-allocation scratch array
// (eb_noalloc.hip), looked up once per device; out may be null (set-up only).
eb_status noalloc_scratch_of_current_device(float **out);

eb_status decode_step_raw(hipStream_t st, const float *q, size_t q_numel, const float *knew,
                          const float *vnew, size_t new_numel, float *kc, size_t kc_numel,
                          float *vc, size_t vc_numel, float *o, size_t o_numel, size_t h,
                          size_t hkv, size_t pos, size_t hd, size_t max_seq, float scale,
                          float *workspace, size_t workspace_floats, int cu_count);
// The part of Attention::decode between the projections and the attention, done inside
// the fused step: per-head RMSNorm of q, knew, vnew (null gains: none) and RoPE of q and
// knew at the step's absolute position (null tables: none). Gains [hd], tables
// [max_seq, hd/2], 16-byte aligned.
struct DecodePrologue {
    const float *q_norm, *k_norm, *v_norm;
    float eps;
    const float *rope_cos, *rope_sin;
};
eb_status launch_attn_decode_any(hipStream_t st, const float *q, const void *kc, const void *vc,
                                 void *kc_w, void *vc_w, const float *knew, const float *vnew,
                                 float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                                 float scale, float *ws, size_t ws_floats, int cu_count,
                                 size_t window, CacheElem ce,
                                 const DecodePrologue *pro = nullptr);
// (launch_attn_decode_any over caches of element type ce; f16 and E4M3 caches need
// head_dim >= 8.)
// kv_write into an IEEE-half cache: src f32 rows rounded to nearest even.
eb_status launch_kv_write_f16(hipStream_t st, uint16_t *cache, const float *src, size_t hkv,
                              size_t count, size_t hd, size_t dst_start);
// kv_write into an E4M3 cache: src f32 rows to the nearest E4M3 (ties to even), finite
// values saturating at +-448, inf and NaN to NaN.
eb_status launch_kv_write_f8(hipStream_t st, uint8_t *cache, const float *src, size_t hkv,
                             size_t count, size_t hd, size_t dst_start);
// Chunked prefill over f16 or E4M3 caches (rows converted to f32 as they are staged).
eb_status launch_attn_prefill_chunk_cache(hipStream_t st, const float *q, const void *kc,
                                          const void *vc, float *o, size_t h, size_t hkv,
                                          size_t pos0, size_t rows, size_t hd, float scale,
                                          size_t window, CacheElem ce, float *ws = nullptr,
                                          size_t ws_floats = 0);
// Attention::decode after the projections as one fused step: RMSNorm (null gains: none)
// and RoPE (null tables: none) of q and the new K row, RMSNorm of the new V row, the
// cache-row write and the attention. Handle-level, used by eb_attention_forward_qkv.
eb_status attn_decode_step_fused(eb_recorder *rec, const eb_tensor *q, const eb_tensor *knew,
                                 const eb_tensor *vnew, eb_tensor *kcache, eb_tensor *vcache,
                                 eb_tensor *o, size_t h, size_t hkv, size_t pos, size_t hd,
                                 size_t max_seq, float scale, size_t window,
                                 const eb_tensor *q_norm, const eb_tensor *k_norm,
                                 const eb_tensor *v_norm, float eps, const eb_tensor *rope_cos,
                                 const eb_tensor *rope_sin);
// Attention::prefill between the projections and the attention as one launch: q/k/v
// RMSNorm (null gains: none), RoPE of q and k at base_pos (null tables: none), q into
// q_out [rows, h, hd] and K / V into cache rows base_pos.. (f32 or IEEE-half caches).
// Handle-level, used by eb_attention_forward_qkv.
eb_status attn_rows_fused(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                          const eb_tensor *v, eb_tensor *q_out, eb_tensor *kcache,
                          eb_tensor *vcache, size_t rows, size_t h, size_t hkv, size_t hd,
                          size_t base_pos, size_t max_seq, const eb_tensor *q_norm,
                          const eb_tensor *k_norm, const eb_tensor *v_norm, float eps,
                          const eb_tensor *rope_cos, const eb_tensor *rope_sin);
// linear_f16w: y[i][m, o] = sum_k x[m, k] * w[i][o, k] for nseg (1..kLinearMaxSegs)
// weight/output pairs sharing x; w IEEE half [out_f[i], in_f]. m <= kLinearGemvRows runs
// the weight-streaming kernel; more rows run the split-f16 matrix-core GEMM, which needs
// linear_workspace_floats(m, in_f) floats of workspace (row exponents).
constexpr int kLinearMaxSegs = 3;
constexpr size_t kLinearGemvRows = 8;
size_t linear_workspace_floats(size_t m, size_t in_f);
eb_status launch_linear_f16w_multi(hipStream_t st, const float *x, const uint16_t *const *w,
                                   float *const *y, const size_t *out_f, int nseg, size_t m,
                                   size_t in_f, float *ws, size_t ws_floats);
// argmax (sampling.rs:6-53 semantics): out[0] = winning index of x[0..n); workspace of
// argmax_workspace_floats(n) floats, 8-byte aligned.
size_t argmax_workspace_floats(size_t n);
eb_status launch_argmax(hipStream_t st, const float *x, size_t n, uint32_t *out, float *ws,
                        size_t ws_floats);
eb_status launch_rmsnorm(hipStream_t st, const float *x, const float *w, float *out,
                         size_t rows, size_t dim, float eps);
// Head rows for the pre-attention pass (RMSNorm, RoPE, store into caches or q) of up to
// three segments [rows, nh, hd]; see eb_rows.hip. Arguments validated by the caller; hd
// even; element counts below 2^31.
struct RowSeg {
    const float *src;   // [rows, nh, hd] f32
    void *dst;          // [*, nh, hd], f32, IEEE half or E4M3 elements
    const float *gain;  // [hd] RMSNorm gain, or null: no norm
    int nh;
    int dst_row0;       // destination row of token 0
    bool rope;          // RoPE at table row rope_row0 + token
    int elem;           // bytes per dst element: 4 f32, 2 IEEE half, 1 E4M3 (both
                        // rounded to nearest even, E4M3 saturating at +-448)
};
struct RowsArgs {
    RowSeg seg[3];
    int nseg;
    int rows, hd;
    float eps;
    const float *cosb, *sinb;  // [>= rope_row0 + rows, hd / 2], null without RoPE
    int rope_row0;
    int start[4];  // set by launch_attn_rows: first head row of each segment
};
eb_status launch_attn_rows(hipStream_t st, const RowsArgs &a);
eb_status launch_rope(hipStream_t st, const float *x, const float *cosb, const float *sinb,
                      float *out, size_t seq, size_t n_heads, size_t hd, size_t base_pos);

}  // namespace eb
