/*
 * eyebrowse_hip — MI355X (gfx950) attention hot path behind a C ABI.
 *
 * This header is the drop-in boundary for the eyebrowse runtime's attention path:
 * the eyebrowse-gpu substrate (Device / Tensor / Recorder), the eyebrowse-kernels
 * entry points (attn_prefill, attn_decode, kv_write, rmsnorm, rope) and the
 * eyebrowse-nn pieces around them (Rope tables, KvCache, the Attention forward between
 * the projections). Every declaration cites the reference interface it replaces
 * (paths relative to the reference repository root).
 *
 * Conventions
 *  - All tensors are f32, row-major, seq-major: q [S, H, HD], k/v [S, Hkv, HD], KV cache
 *    [max_seq, Hkv, HD], o [S, H, HD]. Query head h reads KV head h / (H / Hkv).
 *  - Functions return eb_status; on failure eb_last_error() holds a message (thread local).
 *    The reference has no error channel (its kernels return `()`); a Rust shim keeps its
 *    signatures by turning a non-OK status into a panic (see the integration notes).
 *  - One device owns one HIP stream. Recording a kernel enqueues it on that stream, so
 *    record order is execution order, as with the reference's single wgpu queue.
 *  - Raw entry points (eb_launch_*) take a hipStream_t as void* and device pointers with
 *    their element counts; they validate every size before touching the GPU.
 */
#ifndef EYEBROWSE_HIP_H
#define EYEBROWSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors EyebrowseError (crates/eyebrowse-core/src/lib.rs:27-41), 0 = Ok. */
typedef enum eb_status {
    EB_OK = 0,
    EB_DEVICE_UNAVAILABLE = 1,
    EB_LOAD = 2,
    EB_UNSUPPORTED_CONFIG = 3,
    EB_SHAPE_MISMATCH = 4,
    EB_OUT_OF_MEMORY = 5,
    EB_OTHER = 6
} eb_status;

/* EB_F32 .. EB_I32 mirror DType (crates/eyebrowse-core/src/lib.rs:8-25). EB_F8E4M3 (OCP FP8
 * E4M3, one byte per element, for KV caches) has no counterpart in the reference. */
typedef enum eb_dtype { EB_F32 = 0, EB_F16 = 1, EB_U32 = 2, EB_I32 = 3, EB_F8E4M3 = 4 } eb_dtype;

typedef struct eb_device eb_device;
typedef struct eb_tensor eb_tensor;
typedef struct eb_recorder eb_recorder;
typedef struct eb_rope_tables eb_rope_tables;
typedef struct eb_kv_cache eb_kv_cache;
typedef struct eb_attention eb_attention;

/* ---- errors / types -------------------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). */
const char *eb_last_error(void);
/* Name of a status ("Ok", "DeviceUnavailable", ...). */
const char *eb_status_name(eb_status st);
/* DType::size (crates/eyebrowse-core/src/lib.rs:14-24); 0 for an unknown dtype. */
size_t eb_dtype_size(eb_dtype dt);
/* Library version string. */
const char *eb_version(void);

/* ---- device (crates/eyebrowse-gpu/src/device.rs:20-110) --------------------------- */

/* Device::new (device.rs:32-61): HIP device `ordinal`, one stream, an empty pool.
 * EB_DEVICE_UNAVAILABLE when no GPU is visible. */
eb_status eb_device_new(int ordinal, eb_device **out);
/* Drop the caller's reference (the device lives while tensors/recorders hold it). */
void eb_device_release(eb_device *dev);
/* Wait for everything recorded on the device stream. */
eb_status eb_device_synchronize(eb_device *dev);
/* The device's hipStream_t, for callers that time or interleave their own work. */
void *eb_device_stream(eb_device *dev);
/* Compute units of the device (256 on MI355X). */
int eb_device_cu_count(eb_device *dev);
/* Number of free pooled buffers of exactly `bytes` (device.rs:63-70, test hook). */
size_t eb_device_pooled(eb_device *dev, size_t bytes);
/* Largest buffer the pool recycles, MAX_POOLED_BYTES (device.rs:12-14). */
size_t eb_pool_max_bytes(void);

/* ---- tensor (crates/eyebrowse-gpu/src/tensor.rs:34-157) --------------------------- */

/* Tensor::empty (tensor.rs:62-75): uninitialised, drawn from the pool when a free
 * buffer of the exact byte size exists (sizes <= eb_pool_max_bytes()). */
eb_status eb_tensor_empty(eb_device *dev, const size_t *shape, size_t ndim, eb_dtype dt,
                          eb_tensor **out);
/* Tensor::from_f32 / from_u32 (tensor.rs:77-106): a fresh buffer (never drawn from the
 * pool) initialised from host memory (n elements must equal the shape's element count).
 * Like every tensor it is recycled into the pool on release when small enough. */
eb_status eb_tensor_from_f32(eb_device *dev, const size_t *shape, size_t ndim,
                             const float *data, size_t n, eb_tensor **out);
eb_status eb_tensor_from_u32(eb_device *dev, const size_t *shape, size_t ndim,
                             const uint32_t *data, size_t n, eb_tensor **out);
/* Tensor::to_f32 / read_bytes (tensor.rs:118-157): waits for the stream, then copies.
 * `n`/`nbytes` must equal the tensor's element / byte count. */
eb_status eb_tensor_to_f32(const eb_tensor *t, float *host, size_t n);
eb_status eb_tensor_read_bytes(const eb_tensor *t, void *host, size_t nbytes);
/* Drop for Tensor (tensor.rs:41-47): back to the pool (or freed if larger). */
void eb_tensor_release(eb_tensor *t);
size_t eb_tensor_ndim(const eb_tensor *t);
size_t eb_tensor_dim(const eb_tensor *t, size_t i);
size_t eb_tensor_numel(const eb_tensor *t);
size_t eb_tensor_nbytes(const eb_tensor *t);
eb_dtype eb_tensor_dtype(const eb_tensor *t);
/* Device address of the tensor's storage. */
void *eb_tensor_data(const eb_tensor *t);

/* ---- recorder (crates/eyebrowse-gpu/src/recorder.rs:10-35) ------------------------ */

/* Recorder::new: kernels recorded through it are enqueued on the device stream. */
eb_status eb_recorder_new(eb_device *dev, eb_recorder **out);
/* Recorder::submit (recorder.rs:33-35): flush, report any launch error, release. */
eb_status eb_recorder_submit(eb_recorder *rec);
/* Drop a recorder without submitting (work already enqueued still runs; a deferred
 * recorder's work is discarded). */
void eb_recorder_release(eb_recorder *rec);
/* Recorder::new with the reference's deferral (recorder.rs:10-35): nothing recorded runs
 * until eb_recorder_submit, and eb_recorder_release without a submit discards the work.
 * The recording is a capture of the device stream (a HIP graph launched at submit, which
 * then waits for it). While it is open, only this recorder may record on the device;
 * host copies, synchronisation, other captures and a workspace that would have to grow
 * are refused (EB_OTHER), as during eb_device_begin_capture. For callers that rely on a
 * dropped recorder discarding its work (the reference's own callers always submit). */
eb_status eb_recorder_new_deferred(eb_device *dev, eb_recorder **out);

/* ---- graphs: a whole step as one HIP graph ----------------------------------------
 * No counterpart in the reference, whose answer to per-dispatch overhead is one command
 * buffer per step (README.md:43-45, models/src/model.rs:108-175); this is the HIP form:
 * the step's launches are captured once and replayed with one hipGraphLaunch.
 * eb_device_begin_capture starts capturing the device's stream: every kernel recorded on
 * the device until eb_device_end_capture becomes part of the graph instead of running.
 * While capturing: no host copies (eb_tensor_from_*, to_f32, read_bytes, eb_tensor_write)
 * and no synchronize; a device workspace that would have to grow fails the call (run the
 * step once eagerly first, which also fills the buffer pool). Buffers released during the
 * capture stay reserved until the graph is released or updated, and so does the device
 * workspace buffer the captured kernels use, also when later work grows the device's
 * workspace (the outgrown buffer is freed with the last graph using it). Kernels take their
 * shapes and positions as launch arguments, so a decode step at a new position is a new
 * capture: pass the previous graph to eb_device_end_capture to update it in place. */
typedef struct eb_graph eb_graph;
eb_status eb_device_begin_capture(eb_device *dev);
/* *inout NULL: a new graph. *inout a graph of this device: updated in place (its old
 * intermediates are released). */
eb_status eb_device_end_capture(eb_device *dev, eb_graph **inout);
/* Enqueue one replay on the device stream. */
eb_status eb_graph_launch(eb_graph *g);
void eb_graph_release(eb_graph *g);
/* Host -> device copy into an existing tensor (nbytes = its size), synchronous: how a
 * captured step gets new inputs between replays. */
eb_status eb_tensor_write(eb_tensor *t, const void *host, size_t nbytes);

/* ---- kernels (crates/eyebrowse-kernels/src) --------------------------------------- */

/* attn_prefill (attention.rs:94-120): causal GQA attention over q [s,h,hd],
 * k/v [s,hkv,hd] into o [s,h,hd], keys 0..=i for row i, online softmax. */
eb_status eb_attn_prefill(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                          const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv, size_t s,
                          size_t hd, float scale);
/* attn_prefill in the opt-in f16 mode (no counterpart in the reference, whose prefill is
 * f32): q, K, V and the softmax weights are rounded to IEEE half once and each product is
 * one f16 matrix-core instruction (attn_prefill takes three, on exact hi/lo splits); the
 * online softmax, its rescaling and the accumulation stay f32. Tolerance against the f32
 * reference, measured on the BASELINE prefill configs (N(0,1) inputs, scale 1/sqrt(hd)):
 * rel-L2 about 4e-4 and max-abs below 2e-3 (the north-star bar holds). Prompts from
 * position 0, head_dim a multiple of 16 from 32 to 256, |scale| at most 1/sqrt(head_dim):
 * larger scales (Gemma-4's 1.0) make the scores' f16 rounding error exceed that bar and
 * are refused (EB_UNSUPPORTED_CONFIG); inputs must fit f16 (|x| < 65504). */
eb_status eb_attn_prefill_fast(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                               const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv, size_t s,
                               size_t hd, float scale);
/* attn_prefill in the opt-in scores-accurate mode (no counterpart in the reference): the
 * scores q.k are computed as attn_prefill computes them (three f16 products on exact hi/lo
 * splits, to about f32 accuracy, any scale), the softmax and its accumulation in f32, and
 * O += P V as one f16 product: V rounded to f16 once, the softmax weights rounded to f16,
 * their sum taken over the rounded weights. A third fewer matrix-core products than
 * attn_prefill. The rounding of V bounds the error: max-abs <= 2^-11 times the largest |V|
 * element (half an f16 ulp) plus f32 noise; rel-L2 about 2e-4. On the BASELINE prefill
 * configs (N(0,1) inputs, Gemma-4's scale 1.0 included) that is rel-L2 below 1e-3 and
 * max-abs below 2e-3, the north-star bar; V elements of 8 or more in magnitude can exceed
 * that max-abs (use attn_prefill). V must fit f16 (|v| < 65504). Prompts from position 0,
 * head_dim 24 and up. Same workspace as attn_prefill (the device's here). */
eb_status eb_attn_prefill_pv16(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                               const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv,
                               size_t s, size_t hd, float scale);
/* attn_decode (attention.rs:124-162): q [h,hd] attends keys 0..=pos of the seq-major
 * caches [max_seq,hkv,hd]; o [h,hd]. Split-KV with a log-sum-exp merge; the split
 * workspace belongs to the device and is stream ordered. */
eb_status eb_attn_decode(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                         const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                         size_t pos, size_t hd, size_t max_seq, float scale);
/* The kv_write(K), kv_write(V), attn_decode sequence of Attention::decode
 * (crates/eyebrowse-nn/src/attention.rs:149-183) in one launch: knew/vnew [hkv, hd] are
 * copied bit-exactly into cache row pos and q attends keys 0..=pos (key pos taken from
 * knew/vnew). Same cache contents as the three calls, bit for bit; the same output up
 * to f32 rounding (key pos is folded into the softmax after the cached keys). */
eb_status eb_attn_decode_step(eb_recorder *rec, const eb_tensor *q, const eb_tensor *knew,
                              const eb_tensor *vnew, eb_tensor *kcache, eb_tensor *vcache,
                              eb_tensor *o, size_t h, size_t hkv, size_t pos, size_t hd,
                              size_t max_seq, float scale);
/* Windowed variants (no counterpart in the reference, whose attention is always global):
 * with window > 0 a query at position p attends only keys p - window + 1 ..= p (all of
 * 0..=p when window == 0), as sliding-window (local) layers do. */
eb_status eb_attn_decode_window(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                                const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                size_t pos, size_t hd, size_t max_seq, float scale,
                                size_t window);
eb_status eb_attn_decode_step_window(eb_recorder *rec, const eb_tensor *q, const eb_tensor *knew,
                                     const eb_tensor *vnew, eb_tensor *kcache,
                                     eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                     size_t pos, size_t hd, size_t max_seq, float scale,
                                     size_t window);
/* Chunked causal prefill: q [rows,h,hd] holds the queries at positions pos0..pos0+rows-1,
 * whose K/V are already in the caches [max_seq,hkv,hd]; row r attends cache keys
 * 0..=pos0+r (or the last `window` of them). With pos0 == 0 and no window this is
 * attn_prefill over the cache; with rows == 1 it is attn_decode at pos0. No counterpart
 * in the reference, which defers chunked prefill (README.md:25): its Attention::forward
 * sends a multi-row call at base_pos > 0 to decode (nn/src/attention.rs:40-44), which
 * projects and attends only the first row (:120-185). */
eb_status eb_attn_prefill_chunk(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                                const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                size_t pos0, size_t rows, size_t hd, size_t max_seq,
                                float scale, size_t window);
/* kv_write (ops.rs:150-179): copy src [count,hkv,hd] into cache rows
 * [dst_start, dst_start+count) of [max_seq,hkv,hd]; bit-exact. Unlike the reference,
 * dst_start + count > max_seq is rejected (EB_SHAPE_MISMATCH). */
eb_status eb_kv_write(eb_recorder *rec, eb_tensor *cache, const eb_tensor *src, size_t hkv,
                      size_t count, size_t hd, size_t max_seq, size_t dst_start);
/* rmsnorm (rmsnorm.rs:42-64): out = x / sqrt(mean(x^2) + eps) * weight per row. */
eb_status eb_rmsnorm(eb_recorder *rec, const eb_tensor *x, const eb_tensor *weight,
                     eb_tensor *out, size_t rows, size_t dim, float eps);
/* rope (rope.rs:38-69): half-split rotary on x [seq,n_heads,hd] with cos/sin tables
 * [max_seq,hd/2] read at rows base_pos.. */
eb_status eb_rope(eb_recorder *rec, const eb_tensor *x, const eb_tensor *cos,
                  const eb_tensor *sin, eb_tensor *out, size_t seq, size_t n_heads,
                  size_t head_dim, size_t base_pos);

/* ---- raw launches: the same kernels on caller memory ----------------------------- */

eb_status eb_launch_kv_write(void *stream, float *cache, size_t cache_numel,
                             const float *src, size_t src_numel, size_t hkv, size_t count,
                             size_t hd, size_t max_seq, size_t dst_start);
eb_status eb_launch_attn_prefill(void *stream, const float *q, size_t q_numel,
                                 const float *k, size_t k_numel, const float *v,
                                 size_t v_numel, float *o, size_t o_numel, size_t h,
                                 size_t hkv, size_t s, size_t hd, float scale);
/* eb_attn_prefill_pv16 on caller memory: without a workspace every workgroup splits the K/V
 * rows it stages; with eb_attn_prefill_workspace_floats(h, hkv, hd, 0, s) floats (16-byte
 * aligned, no initialisation) it runs the pre-split pass and key chunks as
 * eb_launch_attn_prefill_ws does. */
eb_status eb_launch_attn_prefill_pv16(void *stream, const float *q, size_t q_numel,
                                      const float *k, size_t k_numel, const float *v,
                                      size_t v_numel, float *o, size_t o_numel, size_t h,
                                      size_t hkv, size_t s, size_t hd, float scale);
eb_status eb_launch_attn_prefill_pv16_ws(void *stream, const float *q, size_t q_numel,
                                         const float *k, size_t k_numel, const float *v,
                                         size_t v_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t s, size_t hd, float scale,
                                         float *workspace, size_t workspace_floats);
eb_status eb_launch_attn_prefill_fast(void *stream, const float *q, size_t q_numel,
                                      const float *k, size_t k_numel, const float *v,
                                      size_t v_numel, float *o, size_t o_numel, size_t h,
                                      size_t hkv, size_t s, size_t hd, float scale);
/* The f16 mode with a workspace: at head_dim <= 128 with at least 3 query blocks sharing
 * the keys, a pre-convert pass rounds every key to f16 once into records that the
 * attention kernel only copies into LDS (same bits as without; eb_attn_prefill_fast uses
 * the device's workspace). Floats needed (0: none used); no initialisation. */
size_t eb_attn_prefill_fast_workspace_floats(size_t h, size_t hkv, size_t hd, size_t s);
eb_status eb_launch_attn_prefill_fast_ws(void *stream, const float *q, size_t q_numel,
                                         const float *k, size_t k_numel, const float *v,
                                         size_t v_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t s, size_t hd, float scale,
                                         float *workspace, size_t workspace_floats);
eb_status eb_launch_attn_prefill_chunk(void *stream, const float *q, size_t q_numel,
                                       const float *kc, size_t kc_numel, const float *vc,
                                       size_t vc_numel, float *o, size_t o_numel, size_t h,
                                       size_t hkv, size_t pos0, size_t rows, size_t hd,
                                       size_t max_seq, float scale, size_t window);
/* Prefill with a workspace (no counterpart in the reference). With head_dim 32..256 and
 * at least 3 query blocks sharing the keys (2 at head_dim 256; a block is 32, 64 or 128
 * rows by the GQA ratio), the _ws launches first split every key they can see once into
 * workspace records (K and V rows scaled by powers of two into f16 hi/lo halves, V
 * transposed), so that the attention kernel only copies them into LDS; the plain raw
 * launches split the keys again in every workgroup that stages them (same bits). When
 * the query blocks alone give fewer than 128 workgroups, the keys of each block are also
 * cut into chunks, one workgroup each, whose partial states (in the workspace) a second
 * launch merges: the sums are then taken in another order than the plain launch's.
 * Floats of workspace for h query heads over hkv KV heads and q rows pos0..pos0+rows-1
 * (pos0 0 for eb_launch_attn_prefill_ws) with this window; 0 when neither is done (the
 * workspace may then be null). No
 * initialisation needed; launches sharing a workspace must not overlap. The recorder
 * entry points (eb_attn_prefill, eb_attn_prefill_chunk) use the device's workspace. */
size_t eb_attn_prefill_workspace_floats(size_t h, size_t hkv, size_t hd, size_t pos0,
                                        size_t rows, size_t window);
eb_status eb_launch_attn_prefill_ws(void *stream, const float *q, size_t q_numel,
                                    const float *k, size_t k_numel, const float *v,
                                    size_t v_numel, float *o, size_t o_numel, size_t h,
                                    size_t hkv, size_t s, size_t hd, float scale,
                                    float *workspace, size_t workspace_floats);
eb_status eb_launch_attn_prefill_chunk_ws(void *stream, const float *q, size_t q_numel,
                                          const float *kc, size_t kc_numel, const float *vc,
                                          size_t vc_numel, float *o, size_t o_numel, size_t h,
                                          size_t hkv, size_t pos0, size_t rows, size_t hd,
                                          size_t max_seq, float scale, size_t window,
                                          float *workspace, size_t workspace_floats);
eb_status eb_launch_attn_prefill_chunk_f16_ws(void *stream, const float *q, size_t q_numel,
                                              const uint16_t *kc, size_t kc_numel,
                                              const uint16_t *vc, size_t vc_numel, float *o,
                                              size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                              size_t rows, size_t hd, size_t max_seq,
                                              float scale, size_t window, float *workspace,
                                              size_t workspace_floats);
/* Floats of workspace eb_launch_attn_decode(_step) needs for this shape on this many CUs
 * (0 when the split count is 1 and no workspace is used). Its contents need no
 * initialisation. Launches that share a workspace must not overlap (use one stream). */
size_t eb_attn_decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd,
                                       int cu_count);
eb_status eb_launch_attn_decode(void *stream, const float *q, size_t q_numel,
                                const float *kc, size_t kc_numel, const float *vc,
                                size_t vc_numel, float *o, size_t o_numel, size_t h,
                                size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                float scale, float *workspace, size_t workspace_floats,
                                int cu_count);
/* eb_attn_decode_window on caller memory (a workspace sized for pos fits any window). */
eb_status eb_launch_attn_decode_window(void *stream, const float *q, size_t q_numel,
                                       const float *kc, size_t kc_numel, const float *vc,
                                       size_t vc_numel, float *o, size_t o_numel, size_t h,
                                       size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                       float scale, size_t window, float *workspace,
                                       size_t workspace_floats, int cu_count);
/* eb_attn_decode_step on caller memory; knew/vnew each hold new_numel >= hkv*hd floats. */
eb_status eb_launch_attn_decode_step(void *stream, const float *q, size_t q_numel,
                                     const float *knew, const float *vnew, size_t new_numel,
                                     float *kc, size_t kc_numel, float *vc, size_t vc_numel,
                                     float *o, size_t o_numel, size_t h, size_t hkv, size_t pos,
                                     size_t hd, size_t max_seq, float scale, float *workspace,
                                     size_t workspace_floats, int cu_count);
/* eb_launch_attn_decode_step without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. The split-KV partials live in a
 * static device array of eb_attn_decode_noalloc_max_floats() floats (4 MiB) that every GPU
 * the library runs on holds until the process ends; the call allocates nothing. Shapes
 * whose partials need more (eb_attn_decode_workspace_floats above the limit) are refused
 * with EB_UNSUPPORTED_CONFIG. All calls on one GPU share its array: calls that overlap on
 * one GPU race, so order them (one stream). Same kernels, same bits as
 * eb_launch_attn_decode_step with a workspace. */
size_t eb_attn_decode_noalloc_max_floats(void);
eb_status eb_launch_attn_decode_step_noalloc(void *stream, const float *q, size_t q_numel,
                                             const float *knew, const float *vnew,
                                             size_t new_numel, float *kc, size_t kc_numel,
                                             float *vc, size_t vc_numel, float *o,
                                             size_t o_numel, size_t h, size_t hkv, size_t pos,
                                             size_t hd, size_t max_seq, float scale,
                                             int cu_count);
eb_status eb_launch_rmsnorm(void *stream, const float *x, size_t x_numel,
                            const float *weight, size_t w_numel, float *out,
                            size_t out_numel, size_t rows, size_t dim, float eps);
eb_status eb_launch_rope(void *stream, const float *x, size_t x_numel, const float *cos,
                         const float *sin, size_t table_numel, float *out, size_t out_numel,
                         size_t seq, size_t n_heads, size_t head_dim, size_t base_pos);
/* The part of Attention::prefill between the projections and the attention
 * (crates/eyebrowse-nn/src/attention.rs:62-97: q_norm / k_norm / v_norm RMSNorm, rope.apply
 * of q and k at base_pos, kv_write of K and V) in one launch. q [rows,h,hd] and k / v
 * [rows,hkv,hd] from the projections; per head row: RMSNorm with the [hd] gain when one is
 * given (NULL: none; a weightless norm passes ones), then RoPE with the [table rows, hd/2]
 * tables at row base_pos + token for q and k (NULL tables: none). The rotated q goes to
 * q_out [rows,h,hd]; K and V go to cache rows base_pos.. of [max_seq,hkv,hd] caches of
 * cache_dtype (EB_F32, or EB_F16 / EB_F8E4M3 rounded to nearest even, E4M3 saturating at
 * +-448). RoPE is computed without fused
 * multiply-adds, as the reference's f32 arithmetic does; rows without a norm are copied
 * bit-exactly. hd even. The reference records 6 kernels for this (3 rmsnorm, 2 rope,
 * 2 kv_write less the norms it skips). */
eb_status eb_launch_attn_prologue(void *stream, const float *q, size_t q_numel, const float *k,
                                  size_t k_numel, const float *v, size_t v_numel, size_t rows,
                                  size_t h, size_t hkv, size_t hd, const float *q_norm,
                                  const float *k_norm, const float *v_norm, float eps,
                                  const float *rope_cos, const float *rope_sin,
                                  size_t table_numel, size_t base_pos, float *q_out,
                                  size_t q_out_numel, void *kcache, size_t kc_numel,
                                  void *vcache, size_t vc_numel, size_t max_seq,
                                  eb_dtype cache_dtype);

/* ---- projections: linear_f16w (crates/eyebrowse-kernels/src/matmul.rs:84-144) -------
 * c [m, out_f] = a [m, in_f] . w^T, a and c f32, w the packed-f16 weight of logical shape
 * [out_f, in_f] (HF Linear layout, crates/eyebrowse-nn/src/linear.rs:5-23): an EB_U32
 * tensor of ceil(out_f*in_f/2) words, two halves per word, low half first (the
 * reference's Tensor::from_f16_packed, crates/eyebrowse-gpu/src/tensor.rs:108-116), or
 * an EB_F16 tensor of out_f*in_f elements. Accumulation is f32 (m <= 8: f32 multiply-adds
 * on the halves; more rows: matrix cores on an exact f16 split of a, to about f32
 * accuracy; the two differ from the reference only in summation order). */
eb_status eb_linear_f16w(eb_recorder *rec, const eb_tensor *a, const eb_tensor *w, eb_tensor *c,
                         size_t m, size_t in_f, size_t out_f);
/* n (1..3) projections of the same a in one launch, e.g. a layer's q/k/v
 * (crates/eyebrowse-nn/src/attention.rs:58-60,129-131): c[i] = a . w[i]^T, c[i]
 * [m, out_f[i]]. No counterpart in the reference (three linear_f16w calls there). */
eb_status eb_linear_f16w_multi(eb_recorder *rec, const eb_tensor *a, size_t n,
                               const eb_tensor *const *w, eb_tensor *const *c,
                               const size_t *out_f, size_t m, size_t in_f);
/* Raw form: w holds w_halves IEEE halves (the packed words read as uint16_t). Rows m > 8
 * need eb_linear_workspace_floats(m, in_f) floats of workspace (row exponents; no
 * initialisation needed). */
size_t eb_linear_workspace_floats(size_t m, size_t in_f);
eb_status eb_launch_linear_f16w(void *stream, const float *a, size_t a_numel, const uint16_t *w,
                                size_t w_halves, float *c, size_t c_numel, size_t m, size_t in_f,
                                size_t out_f, float *workspace, size_t workspace_floats);

/* ---- greedy sampling: argmax (crates/eyebrowse-kernels/src/sampling.rs:6-53) -------
 * out_idx[0] = the index of the largest of logits[0..vocab), with the reference's choice
 * on ties (its 256-lane scan then tree: the lane i mod 256 first in bit-reversed order,
 * then the smallest i); NaN and values <= -3e38 never win; 0 if nothing does. out_idx is
 * a [1] u32 tensor. Two launches over many workgroups (the reference uses one). */
eb_status eb_argmax(eb_recorder *rec, const eb_tensor *logits, eb_tensor *out_idx,
                    size_t vocab);
size_t eb_argmax_workspace_floats(size_t vocab);
eb_status eb_launch_argmax(void *stream, const float *logits, size_t logits_numel,
                           uint32_t *out_idx, size_t vocab, float *workspace,
                           size_t workspace_floats);

/* ---- raw launches over IEEE-half (f16) KV caches ----------------------------------
 * Caches hold uint16_t IEEE half bit patterns, [max_seq, hkv, hd], numel in elements.
 * kv_write rounds the f32 rows to nearest even; attention loads the halves, converts
 * them to f32 and computes as the f32 entry points do (the fused step's key pos uses the
 * rounded new row, the value the cache then holds). Head dims 8..256 (f16 rows of 8
 * halves per 16-byte load). No counterpart in the reference (its caches are f32). The
 * handle entry points (eb_kv_write, eb_attn_decode*, eb_attn_prefill_chunk) take f16
 * caches too, dispatching on the cache tensors' dtype. */
eb_status eb_launch_kv_write_f16(void *stream, uint16_t *cache, size_t cache_numel,
                                 const float *src, size_t src_numel, size_t hkv, size_t count,
                                 size_t hd, size_t max_seq, size_t dst_start);
eb_status eb_launch_attn_prefill_chunk_f16(void *stream, const float *q, size_t q_numel,
                                           const uint16_t *kc, size_t kc_numel,
                                           const uint16_t *vc, size_t vc_numel, float *o,
                                           size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                           size_t rows, size_t hd, size_t max_seq, float scale,
                                           size_t window);
eb_status eb_launch_attn_decode_f16(void *stream, const float *q, size_t q_numel,
                                    const uint16_t *kc, size_t kc_numel, const uint16_t *vc,
                                    size_t vc_numel, float *o, size_t o_numel, size_t h,
                                    size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                    float scale, size_t window, float *workspace,
                                    size_t workspace_floats, int cu_count);
eb_status eb_launch_attn_decode_step_f16(void *stream, const float *q, size_t q_numel,
                                         const float *knew, const float *vnew, size_t new_numel,
                                         uint16_t *kc, size_t kc_numel, uint16_t *vc,
                                         size_t vc_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                         float scale, size_t window, float *workspace,
                                         size_t workspace_floats, int cu_count);

/* ---- raw launches over OCP FP8 E4M3 KV caches --------------------------------------
 * Caches hold uint8_t E4M3 patterns ("e4m3fn": sign, 4 exponent bits with bias 7, 3
 * fraction bits, no infinities, 0x7F / 0xFF NaN, largest finite 448), [max_seq, hkv, hd],
 * numel in elements: a quarter of the f32 cache bytes. kv_write stores the nearest E4M3
 * value of each f32 (ties to the even fraction); finite values at or beyond 448 saturate
 * to +-448, inf and NaN become NaN. Attention converts the stored values to f32 exactly and
 * computes as the f32 entry points do (the fused step's key pos uses the rounded new row).
 * With 3 fraction bits the stored rows carry up to 2^-4 relative error, which reaches the
 * outputs at about 4e-2 rel-L2 on N(0,1) caches at scale 1/sqrt(hd)
 * does not apply to this format. Head dims 8..256 (4, 8 and multiples of 16). No
 * counterpart in the reference (its caches are f32). The handle entry points (eb_kv_write,
 * eb_attn_decode*, eb_attn_prefill_chunk, eb_attention_forward*) take EB_F8E4M3 caches
 * too, dispatching on the cache tensors' dtype. */
eb_status eb_launch_kv_write_f8(void *stream, uint8_t *cache, size_t cache_numel,
                                const float *src, size_t src_numel, size_t hkv, size_t count,
                                size_t hd, size_t max_seq, size_t dst_start);
eb_status eb_launch_attn_prefill_chunk_f8(void *stream, const float *q, size_t q_numel,
                                          const uint8_t *kc, size_t kc_numel, const uint8_t *vc,
                                          size_t vc_numel, float *o, size_t o_numel, size_t h,
                                          size_t hkv, size_t pos0, size_t rows, size_t hd,
                                          size_t max_seq, float scale, size_t window);
eb_status eb_launch_attn_prefill_chunk_f8_ws(void *stream, const float *q, size_t q_numel,
                                             const uint8_t *kc, size_t kc_numel,
                                             const uint8_t *vc, size_t vc_numel, float *o,
                                             size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                             size_t rows, size_t hd, size_t max_seq,
                                             float scale, size_t window, float *workspace,
                                             size_t workspace_floats);
eb_status eb_launch_attn_decode_f8(void *stream, const float *q, size_t q_numel,
                                   const uint8_t *kc, size_t kc_numel, const uint8_t *vc,
                                   size_t vc_numel, float *o, size_t o_numel, size_t h,
                                   size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                   float scale, size_t window, float *workspace,
                                   size_t workspace_floats, int cu_count);
eb_status eb_launch_attn_decode_step_f8(void *stream, const float *q, size_t q_numel,
                                        const float *knew, const float *vnew, size_t new_numel,
                                        uint8_t *kc, size_t kc_numel, uint8_t *vc,
                                        size_t vc_numel, float *o, size_t o_numel, size_t h,
                                        size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                        float scale, size_t window, float *workspace,
                                        size_t workspace_floats, int cu_count);

/* ---- nn (crates/eyebrowse-nn/src) -------------------------------------------------- */

/* Rope::build_partial (rope.rs:24-50): host f64 tables -> f32 device tensors
 * [max_seq, head_dim/2]; rope_angles = head_dim/2 is Rope::build (rope.rs:18-20). */
eb_status eb_rope_build_partial(eb_device *dev, size_t max_seq, size_t head_dim,
                                size_t rope_angles, float theta, eb_rope_tables **out);
void eb_rope_tables_release(eb_rope_tables *rope);
const eb_tensor *eb_rope_tables_cos(const eb_rope_tables *rope);
const eb_tensor *eb_rope_tables_sin(const eb_rope_tables *rope);
/* Rope::apply (rope.rs:54-75): returns a new tensor [seq, n_heads, head_dim]. */
eb_status eb_rope_apply(const eb_rope_tables *rope, eb_recorder *rec, const eb_tensor *x,
                        size_t seq, size_t n_heads, size_t base_pos, eb_tensor **out);

/* KvCache::new_per_layer (kv_cache.rs:29-50): per layer l, K and V tensors
 * [max_seq, n_kv_heads, head_dims[l]] from Tensor::empty. */
eb_status eb_kv_cache_new_per_layer(eb_device *dev, const size_t *head_dims, size_t n_layers,
                                    size_t max_seq, size_t n_kv_heads, eb_kv_cache **out);
/* The same with the caches' element type: EB_F32 (the reference's), EB_F16 (IEEE half:
 * half the cache bytes) or EB_F8E4M3 (OCP FP8 E4M3: a quarter); kv_write rounds to nearest
 * even (E4M3 saturating at +-448), attention computes in f32 on the rounded values. No
 * counterpart in the reference, whose caches are f32 (kv_cache.rs:37,41). */
eb_status eb_kv_cache_new_per_layer_dtype(eb_device *dev, const size_t *head_dims,
                                          size_t n_layers, size_t max_seq, size_t n_kv_heads,
                                          eb_dtype dtype, eb_kv_cache **out);
void eb_kv_cache_release(eb_kv_cache *kv);
eb_tensor *eb_kv_cache_k(eb_kv_cache *kv, size_t layer);
eb_tensor *eb_kv_cache_v(eb_kv_cache *kv, size_t layer);
size_t eb_kv_cache_max_seq(const eb_kv_cache *kv);

/* The Attention fields (crates/eyebrowse-nn/src/attention.rs:10-23). Norm weights are
 * [head_dim] f32 tensors or NULL (None). Projections are packed-f16 weights in the
 * linear_f16w format: q_proj [n_heads*head_dim, hidden], k_proj and v_proj
 * [n_kv_heads*head_dim, hidden], o_proj [hidden, n_heads*head_dim]; all four or none
 * (none: only eb_attention_forward_qkv is available). The module borrows every tensor:
 * they must outlive it, as the reference's Attention owns them. */
typedef struct eb_attention_desc {
    size_t n_heads;
    size_t n_kv_heads;
    size_t head_dim;
    float scale;
    float norm_eps;
    const eb_tensor *q_norm; /* may be NULL */
    const eb_tensor *k_norm; /* may be NULL */
    const eb_tensor *v_norm; /* may be NULL */
    size_t window;           /* sliding window of a local layer; 0 = global attention */
    const eb_tensor *q_proj; /* may be NULL (then all four are) */
    const eb_tensor *k_proj;
    const eb_tensor *v_proj;
    const eb_tensor *o_proj;
    size_t hidden;           /* model width (the projections' in / out features) */
} eb_attention_desc;

eb_status eb_attention_new(const eb_attention_desc *desc, eb_attention **out);
void eb_attention_release(eb_attention *attn);
/* Attention::forward (attention.rs:30-45, 49-117, 120-185) from the projected
 * q [rows, n_heads*hd], k/v [rows, n_kv_heads*hd] on: optional q/k/v RMSNorm, RoPE at
 * base_pos, kv_write of K and V at base_pos, then attn_prefill (base_pos == 0 and
 * rows > 1), chunked prefill over the cache (base_pos > 0 and rows > 1), or the fused
 * decode step (rows == 1); desc.window > 0 restricts every query to its last `window`
 * keys. *out is a new tensor [rows, n_heads*hd] (the input of o_proj). */
eb_status eb_attention_forward_qkv(const eb_attention *attn, eb_recorder *rec,
                                   const eb_tensor *q, const eb_tensor *k, const eb_tensor *v,
                                   const eb_rope_tables *rope, eb_kv_cache *kv, size_t layer,
                                   size_t rows, size_t base_pos, eb_tensor **out);
/* Attention::forward (attention.rs:30-45) whole: x [rows, hidden] f32; q/k/v projections
 * in one launch, then eb_attention_forward_qkv, then o_proj. *out is a new tensor
 * [rows, hidden]. Needs the projection weights in the descriptor. */
eb_status eb_attention_forward(const eb_attention *attn, eb_recorder *rec, const eb_tensor *x,
                               const eb_rope_tables *rope, eb_kv_cache *kv, size_t layer,
                               size_t rows, size_t base_pos, eb_tensor **out);

/* ---- self-check (no counterpart in the reference) ----------------------------------
 * One wave applies the lane exchanges that every wave reduction in the kernels is built
 * from (16- and 32-lane swaps, DPP row rotations and mirrors) to in[0..64) = a and
 * in[64..128) = b, writing EB_LANE_OPS_ROWS rows of 64 floats to out (device memory):
 * a from lane l ^ 16; a from lane l ^ 32; sums of a over the lanes sharing lane bits
 * [0, log2 F) for F = 1, 2, 4, 8, 16, 32; maxima of a for F = 1, 8; a + b over lanes
 * l, l ^ 32 with lanes 0-31 holding the sum of a and 32-63 that of b; the same over l,
 * l ^ 16 (even 16-lane rows a, odd rows b); sums of a over aligned groups of 4 and of 16
 * lanes. For callers (and tests) that want a compiler change in these exchanges to show
 * directly rather than through attention outputs. */
#define EB_LANE_OPS_ROWS 14
eb_status eb_launch_selftest_lane_ops(void *stream, const float *in, float *out);

#ifdef __cplusplus
}
#endif

#endif /* EYEBROWSE_HIP_H */
