// libeyebrowse_hip runtime: the eyebrowse-gpu substrate on HIP.
//
//  - eb_device: one HIP device, one stream (the reference has one wgpu queue,
//    crates/eyebrowse-gpu/src/device.rs:20-28), an exact-size buffer pool
//    (device.rs:82-110) and the split-KV decode workspace.
//  - eb_tensor: a typed device buffer that goes back to the pool when released
//    (crates/eyebrowse-gpu/src/tensor.rs:34-47,62-75).
//  - eb_recorder: recording = enqueueing on the device stream; submit reports errors
//    (crates/eyebrowse-gpu/src/recorder.rs:10-35).
//  - The kernel entry points validate shapes and forward to the launchers in the
//    kernel translation units.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "eb_internal.h"

// ------------------------------------------------------------------ errors ---------------

namespace eb {

static thread_local std::string g_last_error;

eb_status fail(eb_status st, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = std::string(eb_status_name(st)) + ": " + buf;
    return st;
}

eb_status ok() {
    g_last_error.clear();
    return EB_OK;
}

eb_status hip_fail(hipError_t e, const char *what) {
    eb_status st = (e == hipErrorOutOfMemory) ? EB_OUT_OF_MEMORY : EB_OTHER;
    return fail(st, "%s failed: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

eb_status check_launch(const char *kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(EB_OTHER, "launch of %s failed: %s", kernel,
                                     hipGetErrorString(e));
    return EB_OK;
}

eb_status check_ptr(const void *p, const char *name) {
    if (p == nullptr) return fail(EB_SHAPE_MISMATCH, "%s is null", name);
    return EB_OK;
}

eb_status check_numel(size_t have, size_t need, const char *name);

// The product of a shape's dims, refused when it wraps (a caller's absurd sizes must not
// pass the element-count checks below as a small number).
eb_status shape_numel(std::initializer_list<size_t> dims, const char *name, size_t *out) {
    size_t n = 1;
    for (size_t d : dims)
        if (__builtin_mul_overflow(n, d, &n))
            return fail(EB_UNSUPPORTED_CONFIG, "%s: shape size overflows", name);
    *out = n;
    return EB_OK;
}

eb_status check_numel(size_t have, std::initializer_list<size_t> dims, const char *name) {
    size_t need = 0;
    const eb_status st = shape_numel(dims, name, &need);
    return st != EB_OK ? st : check_numel(have, need, name);
}

eb_status check_numel(size_t have, size_t need, const char *name) {
    if (have < need)
        return fail(EB_SHAPE_MISMATCH, "%s holds %zu elements, the shape needs %zu", name, have,
                    need);
    if (need >= kMaxIndex)
        return fail(EB_UNSUPPORTED_CONFIG, "%s needs %zu elements, above the 2^31 index limit",
                    name, need);
    return EB_OK;
}

eb_status check_heads(size_t h, size_t hkv) {
    if (h == 0 || hkv == 0) return fail(EB_SHAPE_MISMATCH, "head counts must be positive");
    if (h % hkv != 0)
        return fail(EB_SHAPE_MISMATCH, "n_heads %zu is not a multiple of n_kv_heads %zu", h, hkv);
    return EB_OK;
}

bool attn_head_dim_supported(size_t hd) {
    return hd == 4 || (hd % 8 == 0 && hd >= 8 && hd <= 128) || (hd % 16 == 0 && hd <= 256);
}

int current_cu_count() {
    static std::mutex mu;
    static std::unordered_map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    cache[dev] = n;
    return n;
}

}  // namespace eb

using eb::fail;

#define EB_TRY(expr)                     \
    do {                                 \
        eb_status eb_s_ = (expr);        \
        if (eb_s_ != EB_OK) return eb_s_; \
    } while (0)

// ------------------------------------------------------------------ handles --------------

// Buffers at or below this size are recycled; larger ones are freed on release
// (MAX_POOLED_BYTES, crates/eyebrowse-gpu/src/device.rs:12-14).
static constexpr size_t kMaxPooledBytes = (size_t)64 << 20;

// A device buffer handed back while a graph capture was running: it stays out of the
// pool for as long as the graph that may write it exists.
struct Parked {
    void *p;
    size_t bytes;
    bool poolable;
};

struct eb_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    int cu_count = 256;
    std::atomic<int> refs{1};
    std::mutex pool_mu;
    std::unordered_map<size_t, std::vector<void *>> pool;  // exact byte size -> free buffers
    std::mutex ws_mu;
    float *ws = nullptr;  // split / pre-split / partials workspace, grow-only, stream ordered
    size_t ws_floats = 0;
    // Graphs whose kernels were captured with a workspace buffer in their arguments keep
    // that buffer alive: live graph references per buffer, and buffers the workspace has
    // outgrown that a graph still references (freed with the last such graph). ws_mu.
    std::unordered_map<float *, int> ws_graph_refs;
    std::vector<float *> ws_retired;
    bool ws_in_capture = false;  // the running capture handed out the current workspace
    std::atomic<bool> capturing{false};  // the stream is being captured into a graph
    std::vector<Parked> parked;          // buffers released during the capture (pool_mu)
    std::atomic<eb_recorder *> deferred{nullptr};  // the deferred recorder owning the capture
};

struct eb_graph {
    eb_device *dev = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<Parked> held;  // intermediates the graph's kernels read and write
    float *ws = nullptr;       // the device workspace its kernels use (null: none)
};

struct eb_tensor {
    eb_device *dev = nullptr;
    void *ptr = nullptr;
    std::vector<size_t> shape;
    eb_dtype dtype = EB_F32;
    size_t bytes = 0;  // allocation size
    bool poolable = false;
};

struct eb_recorder {
    eb_device *dev = nullptr;
    bool deferred = false;  // its work is a capture of the device stream, run at submit
};

static eb_status not_capturing(const eb_device *d, const char *what) {
    if (d && d->capturing.load())
        return fail(EB_OTHER, "%s: not allowed while the device's stream is being captured", what);
    return EB_OK;
}

static void device_retain(eb_device *d) { d->refs.fetch_add(1); }

eb_device *eb::tensor_device(const eb_tensor *t) { return t ? t->dev : nullptr; }

static void device_destroy(eb_device *d) {
    (void)hipSetDevice(d->ordinal);
    (void)hipStreamSynchronize(d->stream);
    for (auto &kv : d->pool)
        for (void *p : kv.second) (void)hipFree(p);
    if (d->ws) (void)hipFree(d->ws);
    for (float *p : d->ws_retired) (void)hipFree(p);
    (void)hipStreamDestroy(d->stream);
    delete d;
}

static void device_unref(eb_device *d) {
    if (d && d->refs.fetch_sub(1) == 1) device_destroy(d);
}

// Elements of a shape, or SIZE_MAX when the product wraps.
static size_t shape_numel(const size_t *shape, size_t ndim) {
    size_t n = 1;
    for (size_t i = 0; i < ndim; ++i)
        if (__builtin_mul_overflow(n, shape[i], &n)) return SIZE_MAX;
    return n;
}

extern "C" {

const char *eb_last_error(void) { return eb::g_last_error.c_str(); }

const char *eb_status_name(eb_status st) {
    switch (st) {
        case EB_OK: return "Ok";
        case EB_DEVICE_UNAVAILABLE: return "DeviceUnavailable";
        case EB_LOAD: return "Load";
        case EB_UNSUPPORTED_CONFIG: return "UnsupportedConfig";
        case EB_SHAPE_MISMATCH: return "ShapeMismatch";
        case EB_OUT_OF_MEMORY: return "OutOfMemory";
        case EB_OTHER: return "Other";
    }
    return "Unknown";
}

size_t eb_dtype_size(eb_dtype dt) {
    switch (dt) {
        case EB_F32: case EB_U32: case EB_I32: return 4;
        case EB_F16: return 2;
        case EB_F8E4M3: return 1;
    }
    return 0;
}

const char *eb_version(void) { return "eyebrowse_hip 0.1.0 (gfx950)"; }

size_t eb_pool_max_bytes(void) { return kMaxPooledBytes; }

// ---- device ---------------------------------------------------------------------------

eb_status eb_device_new(int ordinal, eb_device **out) {
    if (!out) return fail(EB_OTHER, "out is null");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(EB_DEVICE_UNAVAILABLE, "no HIP device visible (%s)",
                    e == hipSuccess ? "count 0" : hipGetErrorString(e));
    if (ordinal < 0 || ordinal >= count)
        return fail(EB_DEVICE_UNAVAILABLE, "device ordinal %d out of range (%d devices)",
                    ordinal, count);
    EB_HIP_TRY(hipSetDevice(ordinal));
    auto *d = new eb_device();
    d->ordinal = ordinal;
    e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete d;
        return eb::hip_fail(e, "hipStreamCreateWithFlags");
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, ordinal) ==
            hipSuccess &&
        n > 0)
        d->cu_count = n;
    // Look up this device's no-allocation scratch now, so that no later call (one under a
    // graph capture, say) has to; a failure here is reported again by that entry point.
    (void)eb::noalloc_scratch_of_current_device(nullptr);
    *out = d;
    return eb::ok();
}

void eb_device_release(eb_device *dev) { device_unref(dev); }

eb_status eb_device_synchronize(eb_device *dev) {
    if (!dev) return fail(EB_OTHER, "device is null");
    EB_TRY(not_capturing(dev, "synchronize"));
    EB_HIP_TRY(hipSetDevice(dev->ordinal));
    EB_HIP_TRY(hipStreamSynchronize(dev->stream));
    return eb::ok();
}

void *eb_device_stream(eb_device *dev) { return dev ? (void *)dev->stream : nullptr; }

int eb_device_cu_count(eb_device *dev) { return dev ? dev->cu_count : 0; }

size_t eb_device_pooled(eb_device *dev, size_t bytes) {
    if (!dev) return 0;
    std::lock_guard<std::mutex> lk(dev->pool_mu);
    auto it = dev->pool.find(bytes);
    return it == dev->pool.end() ? 0 : it->second.size();
}

// ---- tensor ---------------------------------------------------------------------------

static eb_status tensor_alloc(eb_device *dev, const size_t *shape, size_t ndim, eb_dtype dt,
                              bool from_pool, eb_tensor **out) {
    if (!dev) return fail(EB_OTHER, "device is null");
    if (!out) return fail(EB_OTHER, "out is null");
    if (ndim > 0 && !shape) return fail(EB_SHAPE_MISMATCH, "shape is null");
    *out = nullptr;
    size_t esz = eb_dtype_size(dt);
    if (esz == 0) return fail(EB_OTHER, "unknown dtype %d", (int)dt);
    size_t numel = shape_numel(shape, ndim);
    size_t nbytes_check = 0;
    if (numel == SIZE_MAX || __builtin_mul_overflow(numel, esz, &nbytes_check))
        return fail(EB_OUT_OF_MEMORY, "tensor of %zu dims: size overflows", ndim);
    // (numel * size).max(size): a zero-element tensor still owns one element
    // (crates/eyebrowse-gpu/src/tensor.rs:67).
    size_t bytes = numel * esz;
    if (bytes < esz) bytes = esz;
    void *p = nullptr;
    bool poolable = bytes <= kMaxPooledBytes;
    if (from_pool && poolable) {
        std::lock_guard<std::mutex> lk(dev->pool_mu);
        auto it = dev->pool.find(bytes);
        if (it != dev->pool.end() && !it->second.empty()) {
            p = it->second.back();
            it->second.pop_back();
        }
    }
    if (!p) {
        EB_HIP_TRY(hipSetDevice(dev->ordinal));
        EB_HIP_TRY(hipMalloc(&p, bytes));
    }
    auto *t = new eb_tensor();
    t->dev = dev;
    device_retain(dev);
    t->ptr = p;
    t->shape.assign(shape, shape + ndim);
    t->dtype = dt;
    t->bytes = bytes;
    t->poolable = poolable;
    *out = t;
    return eb::ok();
}

eb_status eb_tensor_empty(eb_device *dev, const size_t *shape, size_t ndim, eb_dtype dt,
                          eb_tensor **out) {
    return tensor_alloc(dev, shape, ndim, dt, true, out);
}

static eb_status tensor_from_host(eb_device *dev, const size_t *shape, size_t ndim,
                                  eb_dtype dt, const void *data, size_t n, eb_tensor **out) {
    EB_TRY(not_capturing(dev, "from_host"));
    if (n != shape_numel(shape, ndim))
        return fail(EB_SHAPE_MISMATCH, "from_host: data len %zu != shape numel %zu", n,
                    shape_numel(shape, ndim));
    if (n > 0 && !data) return fail(EB_SHAPE_MISMATCH, "from_host: data is null");
    // Host-initialised tensors never draw from the pool (tensor.rs:77-96).
    eb_status st = tensor_alloc(dev, shape, ndim, dt, false, out);
    if (st != EB_OK) return st;
    if (n > 0) {
        hipError_t e = hipMemcpyAsync((*out)->ptr, data, n * eb_dtype_size(dt),
                                      hipMemcpyHostToDevice, dev->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
        if (e != hipSuccess) {
            eb_tensor_release(*out);
            *out = nullptr;
            return eb::hip_fail(e, "upload");
        }
    }
    return eb::ok();
}

eb_status eb_tensor_from_f32(eb_device *dev, const size_t *shape, size_t ndim,
                             const float *data, size_t n, eb_tensor **out) {
    return tensor_from_host(dev, shape, ndim, EB_F32, data, n, out);
}

eb_status eb_tensor_from_u32(eb_device *dev, const size_t *shape, size_t ndim,
                             const uint32_t *data, size_t n, eb_tensor **out) {
    return tensor_from_host(dev, shape, ndim, EB_U32, data, n, out);
}

eb_status eb_tensor_read_bytes(const eb_tensor *t, void *host, size_t nbytes) {
    if (!t) return fail(EB_OTHER, "tensor is null");
    EB_TRY(not_capturing(t->dev, "read_bytes"));
    size_t want = shape_numel(t->shape.data(), t->shape.size()) * eb_dtype_size(t->dtype);
    if (nbytes != want)
        return fail(EB_SHAPE_MISMATCH, "read_bytes: asked for %zu bytes, tensor has %zu", nbytes,
                    want);
    if (nbytes == 0) return eb::ok();
    if (!host) return fail(EB_SHAPE_MISMATCH, "read_bytes: host buffer is null");
    EB_HIP_TRY(hipSetDevice(t->dev->ordinal));
    EB_HIP_TRY(hipMemcpyAsync(host, t->ptr, nbytes, hipMemcpyDeviceToHost, t->dev->stream));
    EB_HIP_TRY(hipStreamSynchronize(t->dev->stream));
    return eb::ok();
}

eb_status eb_tensor_to_f32(const eb_tensor *t, float *host, size_t n) {
    if (!t) return fail(EB_OTHER, "tensor is null");
    if (t->dtype != EB_F32) return fail(EB_SHAPE_MISMATCH, "to_f32 on a non-f32 tensor");
    return eb_tensor_read_bytes(t, host, n * sizeof(float));
}

void eb_tensor_release(eb_tensor *t) {
    if (!t) return;
    eb_device *d = t->dev;
    if (d->capturing.load()) {
        // A captured kernel may still use this buffer on every replay of the graph.
        std::lock_guard<std::mutex> lk(d->pool_mu);
        d->parked.push_back(Parked{t->ptr, t->bytes, t->poolable});
    } else if (t->poolable) {
        // Stream-ordered reuse: every kernel runs on the device's single stream, so a
        // later user of this buffer is queued after every earlier one.
        std::lock_guard<std::mutex> lk(d->pool_mu);
        d->pool[t->bytes].push_back(t->ptr);
    } else {
        (void)hipSetDevice(d->ordinal);
        (void)hipStreamSynchronize(d->stream);
        (void)hipFree(t->ptr);
    }
    delete t;
    device_unref(d);
}

size_t eb_tensor_ndim(const eb_tensor *t) { return t ? t->shape.size() : 0; }
size_t eb_tensor_dim(const eb_tensor *t, size_t i) {
    return (t && i < t->shape.size()) ? t->shape[i] : 0;
}
size_t eb_tensor_numel(const eb_tensor *t) {
    return t ? shape_numel(t->shape.data(), t->shape.size()) : 0;
}
size_t eb_tensor_nbytes(const eb_tensor *t) {
    return t ? eb_tensor_numel(t) * eb_dtype_size(t->dtype) : 0;
}
eb_dtype eb_tensor_dtype(const eb_tensor *t) { return t ? t->dtype : EB_F32; }
void *eb_tensor_data(const eb_tensor *t) { return t ? t->ptr : nullptr; }

// ---- recorder -------------------------------------------------------------------------

eb_status eb_recorder_new(eb_device *dev, eb_recorder **out) {
    if (!dev || !out) return fail(EB_OTHER, "device/out is null");
    auto *r = new eb_recorder();
    r->dev = dev;
    device_retain(dev);
    *out = r;
    return eb::ok();
}

// Ends a deferred recorder's capture: with run, the captured work is launched and waited
// for; without, it is discarded. The graph is released either way.
static eb_status finish_deferred(eb_recorder *rec, bool run) {
    eb_device *d = rec->dev;
    eb_recorder *owner = rec;
    if (!d->deferred.compare_exchange_strong(owner, nullptr)) return EB_OK;  // (finished)
    eb_graph *g = nullptr;
    eb_status st = eb_device_end_capture(d, &g);
    if (st == EB_OK && run) st = eb_graph_launch(g);
    if (g) eb_graph_release(g);  // (drains the stream first)
    return st;
}

eb_status eb_recorder_new_deferred(eb_device *dev, eb_recorder **out) {
    if (!dev || !out) return fail(EB_OTHER, "device/out is null");
    EB_TRY(eb_device_begin_capture(dev));  // (refused while another capture is running)
    auto *r = new eb_recorder();
    r->dev = dev;
    r->deferred = true;
    dev->deferred.store(r);
    device_retain(dev);
    *out = r;
    return eb::ok();
}

eb_status eb_recorder_submit(eb_recorder *rec) {
    if (!rec) return fail(EB_OTHER, "recorder is null");
    if (rec->deferred) {
        const eb_status st = finish_deferred(rec, true);
        device_unref(rec->dev);
        delete rec;
        return st == EB_OK ? eb::ok() : st;
    }
    hipError_t e = hipGetLastError();
    eb_recorder_release(rec);
    if (e != hipSuccess) return eb::hip_fail(e, "submit");
    return eb::ok();
}

void eb_recorder_release(eb_recorder *rec) {
    if (!rec) return;
    if (rec->deferred) (void)finish_deferred(rec, false);
    device_unref(rec->dev);
    delete rec;
}


eb_status eb_tensor_write(eb_tensor *t, const void *host, size_t nbytes) {
    if (!t) return fail(EB_OTHER, "tensor is null");
    EB_TRY(not_capturing(t->dev, "tensor_write"));
    size_t want = shape_numel(t->shape.data(), t->shape.size()) * eb_dtype_size(t->dtype);
    if (nbytes != want)
        return fail(EB_SHAPE_MISMATCH, "tensor_write: %zu bytes given, tensor has %zu", nbytes,
                    want);
    if (nbytes == 0) return eb::ok();
    if (!host) return fail(EB_SHAPE_MISMATCH, "tensor_write: host buffer is null");
    EB_HIP_TRY(hipSetDevice(t->dev->ordinal));
    EB_HIP_TRY(hipMemcpyAsync(t->ptr, host, nbytes, hipMemcpyHostToDevice, t->dev->stream));
    EB_HIP_TRY(hipStreamSynchronize(t->dev->stream));
    return eb::ok();
}

// ---- graphs ---------------------------------------------------------------------------

// Hands parked buffers back: pooled sizes to the pool (stream-ordered reuse, like any
// release), larger ones freed once the stream has drained.
static void return_buffers(eb_device *d, std::vector<Parked> &v) {
    bool synced = false;
    for (const Parked &b : v) {
        if (b.poolable) {
            std::lock_guard<std::mutex> lk(d->pool_mu);
            d->pool[b.bytes].push_back(b.p);
        } else {
            if (!synced) (void)hipStreamSynchronize(d->stream);
            synced = true;
            (void)hipFree(b.p);
        }
    }
    v.clear();
}

// The graph reference on the workspace buffer that the finished capture handed to its
// kernels (null when it used none).
static float *ws_capture_ref(eb_device *d) {
    std::lock_guard<std::mutex> lk(d->ws_mu);
    float *p = d->ws_in_capture ? d->ws : nullptr;
    d->ws_in_capture = false;
    if (p) ++d->ws_graph_refs[p];
    return p;
}

// Drops a graph's workspace reference. A buffer the workspace has outgrown is freed with
// its last graph (the caller has drained the stream, so no replay still runs).
static void ws_graph_unref(eb_device *d, float *p) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(d->ws_mu);
    auto it = d->ws_graph_refs.find(p);
    if (it == d->ws_graph_refs.end() || --it->second > 0) return;
    d->ws_graph_refs.erase(it);
    auto r = std::find(d->ws_retired.begin(), d->ws_retired.end(), p);
    if (r != d->ws_retired.end()) {
        d->ws_retired.erase(r);
        (void)hipFree(p);
    }
}

eb_status eb_device_begin_capture(eb_device *dev) {
    if (!dev) return fail(EB_OTHER, "device is null");
    EB_TRY(not_capturing(dev, "begin_capture"));
    EB_HIP_TRY(hipSetDevice(dev->ordinal));
    EB_HIP_TRY(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeRelaxed));
    dev->capturing.store(true);
    return eb::ok();
}

eb_status eb_device_end_capture(eb_device *dev, eb_graph **inout) {
    if (!dev || !inout) return fail(EB_OTHER, "device/graph is null");
    if (!dev->capturing.load()) return fail(EB_OTHER, "end_capture: no capture is running");
    EB_HIP_TRY(hipSetDevice(dev->ordinal));
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(dev->stream, &g);
    std::vector<Parked> held;
    {
        std::lock_guard<std::mutex> lk(dev->pool_mu);
        held.swap(dev->parked);
    }
    dev->capturing.store(false);
    float *ws_used = ws_capture_ref(dev);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return_buffers(dev, held);
        ws_graph_unref(dev, ws_used);
        return eb::hip_fail(e, "hipStreamEndCapture (a call during the capture failed?)");
    }
    eb_graph *gr = *inout;
    if (gr && gr->dev != dev) {
        (void)hipGraphDestroy(g);
        return_buffers(dev, held);
        ws_graph_unref(dev, ws_used);
        return fail(EB_OTHER, "end_capture: the graph belongs to another device");
    }
    if (gr) {
        // Same topology: update the executable in place; otherwise instantiate anew. The
        // stream is drained first so that no launch of the old version still runs.
        e = hipStreamSynchronize(dev->stream);
        if (e == hipSuccess) {
            hipGraphNode_t err_node = nullptr;
            hipGraphExecUpdateResult res;
            if (hipGraphExecUpdate(gr->exec, g, &err_node, &res) != hipSuccess) {
                (void)hipGetLastError();
                (void)hipGraphExecDestroy(gr->exec);
                gr->exec = nullptr;
                e = hipGraphInstantiate(&gr->exec, g, nullptr, nullptr, 0);
            }
        }
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            return_buffers(dev, held);
            ws_graph_unref(dev, ws_used);
            return eb::hip_fail(e, "graph update");
        }
        return_buffers(dev, gr->held);
        gr->held.swap(held);
        ws_graph_unref(dev, gr->ws);
        gr->ws = ws_used;
        return eb::ok();
    }
    auto *ng = new eb_graph();
    ng->dev = dev;
    e = hipGraphInstantiate(&ng->exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        delete ng;
        return_buffers(dev, held);
        ws_graph_unref(dev, ws_used);
        return eb::hip_fail(e, "hipGraphInstantiate");
    }
    device_retain(dev);
    ng->held.swap(held);
    ng->ws = ws_used;
    *inout = ng;
    return eb::ok();
}

eb_status eb_graph_launch(eb_graph *g) {
    if (!g || !g->exec) return fail(EB_OTHER, "graph is null");
    EB_TRY(not_capturing(g->dev, "graph_launch"));
    EB_HIP_TRY(hipSetDevice(g->dev->ordinal));
    EB_HIP_TRY(hipGraphLaunch(g->exec, g->dev->stream));
    return eb::ok();
}

void eb_graph_release(eb_graph *g) {
    if (!g) return;
    eb_device *d = g->dev;
    (void)hipSetDevice(d->ordinal);
    (void)hipStreamSynchronize(d->stream);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    return_buffers(d, g->held);
    ws_graph_unref(d, g->ws);
    delete g;
    device_unref(d);
}

}  // extern "C"

// ------------------------------------------------------------------ kernel entry points -

static eb_status rec_ready(eb_recorder *rec) {
    if (!rec) return fail(EB_OTHER, "recorder is null");
    const eb_recorder *owner = rec->dev->deferred.load();
    if (owner && owner != rec)
        return fail(EB_OTHER, "a deferred recorder is open on this device: only it may record "
                              "until it is submitted or released");
    EB_HIP_TRY(hipSetDevice(rec->dev->ordinal));
    return EB_OK;
}

static eb_status tensor_f32(const eb_tensor *t, const char *name, eb_device *dev) {
    if (!t) return fail(EB_SHAPE_MISMATCH, "%s is null", name);
    if (t->dtype != EB_F32) return fail(EB_SHAPE_MISMATCH, "%s must be f32", name);
    if (t->dev != dev) return fail(EB_OTHER, "%s lives on another device", name);
    return EB_OK;
}

// A KV cache: f32, IEEE-half or E4M3 elements; *ce reports which.
static eb_status tensor_cache(const eb_tensor *t, const char *name, eb_device *dev,
                              eb::CacheElem *ce) {
    if (!t) return fail(EB_SHAPE_MISMATCH, "%s is null", name);
    if (t->dtype != EB_F32 && t->dtype != EB_F16 && t->dtype != EB_F8E4M3)
        return fail(EB_SHAPE_MISMATCH, "%s must be f32, f16 or f8e4m3", name);
    if (t->dev != dev) return fail(EB_OTHER, "%s lives on another device", name);
    *ce = t->dtype == EB_F16      ? eb::CacheElem::F16
          : t->dtype == EB_F8E4M3 ? eb::CacheElem::E4M3
                                  : eb::CacheElem::F32;
    return EB_OK;
}


// Float-buffer views with element counts, shared by the handle and raw entry points.
static eb_status kv_write_checked(hipStream_t st, void *cache, size_t cache_n,
                                  const float *src, size_t src_n, size_t hkv, size_t count,
                                  size_t hd, size_t max_seq, size_t dst,
                                  eb::CacheElem ce = eb::CacheElem::F32) {
    if (hkv == 0 || hd == 0) return fail(EB_SHAPE_MISMATCH, "kv_write: hkv and hd must be > 0");
    if (dst > max_seq || count > max_seq - dst)
        return fail(EB_SHAPE_MISMATCH, "kv_write: rows [%zu, %zu) exceed max_seq %zu", dst,
                    dst + count, max_seq);
    EB_TRY(eb::check_numel(cache_n, {max_seq, hkv, hd}, "cache"));
    EB_TRY(eb::check_numel(src_n, {count, hkv, hd}, "src"));
    if (count == 0) return eb::ok();
    EB_TRY(eb::check_ptr(cache, "cache"));
    EB_TRY(eb::check_ptr(src, "src"));
    if (ce != eb::CacheElem::F32 && hd % 4 != 0)
        return fail(EB_UNSUPPORTED_CONFIG, "kv_write: f16 and e4m3 caches need hd %% 4 == 0");
    if (ce == eb::CacheElem::F16) {
        EB_TRY(eb::launch_kv_write_f16(st, static_cast<uint16_t *>(cache), src, hkv, count, hd,
                                       dst));
    } else if (ce == eb::CacheElem::E4M3) {
        EB_TRY(eb::launch_kv_write_f8(st, static_cast<uint8_t *>(cache), src, hkv, count, hd,
                                      dst));
    } else {
        EB_TRY(eb::launch_kv_write(st, static_cast<float *>(cache), src, hkv, count, hd, dst));
    }
    return eb::ok();
}

// The device workspace is handed out with its mutex held (in *lk) until the caller's launch
// is enqueued: another thread that grows it in between would free a buffer the launch is
// about to use.
using WsLock = std::unique_lock<std::mutex>;
static eb_status device_workspace(eb_device *dev, size_t floats, float **out, WsLock &lk);

// Where a prefill's pre-split workspace comes from: the device's grow-only workspace
// (recorder launches), the caller's buffer (raw _ws launches; null with 0 floats is allowed
// only where the shape needs none), or nowhere (raw launches without one: the prefill
// splits K/V while staging).
struct PrefillWs {
    eb_device *dev = nullptr;
    bool caller = false;
    float *ptr = nullptr;
    size_t floats = 0;
};

static eb_status prefill_ws(const PrefillWs &src, size_t h, size_t hkv, size_t hd, size_t rows,
                            size_t nkeys, size_t qbase, size_t window, float **ws, size_t *wsn,
                            WsLock &lk) {
    *ws = nullptr;
    *wsn = 0;
    if (!src.dev && !src.caller) return EB_OK;
    const size_t need = eb::prefill_workspace_floats(h, hkv, hd, rows, nkeys, qbase, window);
    if (need == 0) return EB_OK;
    if (src.dev) {
        EB_TRY(device_workspace(src.dev, need, ws, lk));
    } else {
        if (src.floats < need)
            return fail(EB_SHAPE_MISMATCH, "attn_prefill: workspace holds %zu floats, needs %zu",
                        src.floats, need);
        EB_TRY(eb::check_ptr(src.ptr, "workspace"));
        if (reinterpret_cast<uintptr_t>(src.ptr) & 15)
            return fail(EB_UNSUPPORTED_CONFIG, "attn_prefill: workspace must be 16-byte aligned");
        *ws = src.ptr;
    }
    *wsn = need;
    return EB_OK;
}

// pv1: the scores-accurate mode (eb_attn_prefill_pv16), head dims 24 and up.
static eb_status prefill_checked(hipStream_t st, const float *q, size_t qn, const float *k,
                                 size_t kn, const float *v, size_t vn, float *o, size_t on,
                                 size_t h, size_t hkv, size_t s, size_t hd, float scale,
                                 const PrefillWs &wsrc = PrefillWs(), bool pv1 = false) {
    EB_TRY(eb::check_heads(h, hkv));
    if (!eb::attn_head_dim_supported(hd))
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill: head_dim %zu (supported: 4, multiples of 8 up to 128, "
                    "multiples of 16 up to 256)", hd);
    if (pv1 && hd < 24)
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill_pv16: head_dim %zu (24 and up; smaller head dims run "
                    "attn_prefill, in f32)", hd);
    EB_TRY(eb::check_numel(qn, {s, h, hd}, "q"));
    EB_TRY(eb::check_numel(kn, {s, hkv, hd}, "k"));
    EB_TRY(eb::check_numel(vn, {s, hkv, hd}, "v"));
    EB_TRY(eb::check_numel(on, {s, h, hd}, "o"));
    if (s == 0) return eb::ok();
    EB_TRY(eb::check_ptr(q, "q"));
    EB_TRY(eb::check_ptr(k, "k"));
    EB_TRY(eb::check_ptr(v, "v"));
    EB_TRY(eb::check_ptr(o, "o"));
    float *ws;
    size_t wsn;
    WsLock lk;
    EB_TRY(prefill_ws(wsrc, h, hkv, hd, s, s, 0, 0, &ws, &wsn, lk));
    if (pv1)
        EB_TRY(eb::launch_attn_prefill_pv16(st, q, k, v, o, h, hkv, s, hd, scale, ws, wsn));
    else
        EB_TRY(eb::launch_attn_prefill(st, q, k, v, o, h, hkv, s, hd, scale, ws, wsn));
    return eb::ok();
}

// The single-product f16 prefill (opt-in): the checks of prefill_checked, then the scale
// bound that keeps the f16 rounding of q and K inside the stated tolerance.
static eb_status prefill_fast_checked(hipStream_t st, const float *q, size_t qn, const float *k,
                                      size_t kn, const float *v, size_t vn, float *o, size_t on,
                                      size_t h, size_t hkv, size_t s, size_t hd, float scale,
                                      const PrefillWs &wsrc = PrefillWs()) {
    EB_TRY(eb::check_heads(h, hkv));
    if (hd < 24 || !eb::attn_head_dim_supported(hd))
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill_fast: head_dim %zu (multiples of 8 from 24 to 128, of 16 "
                    "to 256)", hd);
    if (!(std::fabs(scale) * std::sqrt((double)hd) <= 1.0001))
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill_fast: scale %g above 1/sqrt(head_dim): the f16 rounding of "
                    "the scores would exceed the mode's tolerance (use attn_prefill)",
                    (double)scale);
    EB_TRY(eb::check_numel(qn, {s, h, hd}, "q"));
    EB_TRY(eb::check_numel(kn, {s, hkv, hd}, "k"));
    EB_TRY(eb::check_numel(vn, {s, hkv, hd}, "v"));
    EB_TRY(eb::check_numel(on, {s, h, hd}, "o"));
    if (s == 0) return eb::ok();
    EB_TRY(eb::check_ptr(q, "q"));
    EB_TRY(eb::check_ptr(k, "k"));
    EB_TRY(eb::check_ptr(v, "v"));
    EB_TRY(eb::check_ptr(o, "o"));
    float *ws = nullptr;
    size_t wsn = 0;
    WsLock lk;
    const size_t need = eb::prefill_fast_workspace_floats(h, hkv, hd, s);
    if (need > 0 && wsrc.dev) {
        EB_TRY(device_workspace(wsrc.dev, need, &ws, lk));
        wsn = need;
    } else if (need > 0 && wsrc.caller) {
        if (wsrc.floats < need)
            return fail(EB_SHAPE_MISMATCH,
                        "attn_prefill_fast: workspace holds %zu floats, needs %zu", wsrc.floats,
                        need);
        EB_TRY(eb::check_ptr(wsrc.ptr, "workspace"));
        ws = wsrc.ptr;
        wsn = need;
    }
    EB_TRY(eb::launch_attn_prefill_fast(st, q, k, v, o, h, hkv, s, hd, scale, ws, wsn));
    return eb::ok();
}

static eb_status prefill_chunk_checked(hipStream_t st, const float *q, size_t qn,
                                       const void *kc, size_t kcn, const void *vc, size_t vcn,
                                       float *o, size_t on, size_t h, size_t hkv, size_t pos0,
                                       size_t rows, size_t hd, size_t max_seq, float scale,
                                       size_t window, eb::CacheElem ce = eb::CacheElem::F32,
                                       const PrefillWs &wsrc = PrefillWs()) {
    EB_TRY(eb::check_heads(h, hkv));
    if (!eb::attn_head_dim_supported(hd))
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill_chunk: head_dim %zu (supported: 4, multiples of 8 up to 128, multiples of 16 up to 256)",
                    hd);
    if (ce != eb::CacheElem::F32 && hd < 8)
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_prefill_chunk: f16 and e4m3 caches need head_dim >= 8");
    if (pos0 > max_seq || rows > max_seq - pos0)
        return fail(EB_SHAPE_MISMATCH, "attn_prefill_chunk: rows [%zu, %zu) exceed max_seq %zu",
                    pos0, pos0 + rows, max_seq);
    EB_TRY(eb::check_numel(qn, {rows, h, hd}, "q"));
    EB_TRY(eb::check_numel(kcn, {max_seq, hkv, hd}, "kcache"));
    EB_TRY(eb::check_numel(vcn, {max_seq, hkv, hd}, "vcache"));
    EB_TRY(eb::check_numel(on, {rows, h, hd}, "o"));
    if (rows == 0) return eb::ok();
    EB_TRY(eb::check_ptr(q, "q"));
    EB_TRY(eb::check_ptr(kc, "kcache"));
    EB_TRY(eb::check_ptr(vc, "vcache"));
    EB_TRY(eb::check_ptr(o, "o"));
    float *ws;
    size_t wsn;
    WsLock lk;
    EB_TRY(prefill_ws(wsrc, h, hkv, hd, rows, pos0 + rows, pos0, window, &ws, &wsn, lk));
    if (ce != eb::CacheElem::F32)
        EB_TRY(eb::launch_attn_prefill_chunk_cache(st, q, kc, vc, o, h, hkv, pos0, rows, hd,
                                                   scale, window, ce, ws, wsn));
    else
        EB_TRY(eb::launch_attn_prefill_chunk(st, q, static_cast<const float *>(kc),
                                             static_cast<const float *>(vc), o, h, hkv, pos0,
                                             rows, hd, scale, window, ws, wsn));
    return eb::ok();
}

static eb_status decode_shape_checked(const float *q, size_t qn, const void *kc, size_t kcn,
                                      const void *vc, size_t vcn, const float *o, size_t on,
                                      size_t h, size_t hkv, size_t pos, size_t hd,
                                      size_t max_seq,
                                      eb::CacheElem ce = eb::CacheElem::F32) {
    EB_TRY(eb::check_heads(h, hkv));
    if (!eb::attn_head_dim_supported(hd))
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attn_decode: head_dim %zu (supported: 4, multiples of 8 up to 128, multiples of 16 up to 256)", hd);
    if (ce != eb::CacheElem::F32 && hd < 8)
        return fail(EB_UNSUPPORTED_CONFIG, "attn_decode: f16 and e4m3 caches need head_dim >= 8");
    if (pos >= max_seq)
        return fail(EB_SHAPE_MISMATCH, "attn_decode: pos %zu >= max_seq %zu", pos, max_seq);
    EB_TRY(eb::check_numel(qn, {h, hd}, "q"));
    EB_TRY(eb::check_numel(kcn, {max_seq, hkv, hd}, "kcache"));
    EB_TRY(eb::check_numel(vcn, {max_seq, hkv, hd}, "vcache"));
    EB_TRY(eb::check_numel(on, {h, hd}, "o"));
    EB_TRY(eb::check_ptr(q, "q"));
    EB_TRY(eb::check_ptr(kc, "kcache"));
    EB_TRY(eb::check_ptr(vc, "vcache"));
    EB_TRY(eb::check_ptr(o, "o"));
    return EB_OK;
}

static eb_status rmsnorm_checked(hipStream_t st, const float *x, size_t xn, const float *w,
                                 size_t wn, float *out, size_t outn, size_t rows, size_t dim,
                                 float eps) {
    if (dim == 0) return fail(EB_SHAPE_MISMATCH, "rmsnorm: dim must be > 0");
    EB_TRY(eb::check_numel(xn, {rows, dim}, "x"));
    EB_TRY(eb::check_numel(wn, dim, "weight"));
    EB_TRY(eb::check_numel(outn, {rows, dim}, "out"));
    if (rows == 0) return eb::ok();
    EB_TRY(eb::check_ptr(x, "x"));
    EB_TRY(eb::check_ptr(w, "weight"));
    EB_TRY(eb::check_ptr(out, "out"));
    EB_TRY(eb::launch_rmsnorm(st, x, w, out, rows, dim, eps));
    return eb::ok();
}

static eb_status rope_checked(hipStream_t st, const float *x, size_t xn, const float *c,
                              const float *s, size_t tn, float *out, size_t outn, size_t seq,
                              size_t nh, size_t hd, size_t base_pos) {
    if (hd == 0 || hd % 2 != 0) return fail(EB_SHAPE_MISMATCH, "rope: head_dim must be even");
    EB_TRY(eb::check_numel(xn, {seq, nh, hd}, "x"));
    EB_TRY(eb::check_numel(outn, {seq, nh, hd}, "out"));
    EB_TRY(eb::check_numel(tn, {(seq + base_pos), (hd / 2)}, "cos/sin tables"));
    if (seq == 0 || nh == 0) return eb::ok();
    EB_TRY(eb::check_ptr(x, "x"));
    EB_TRY(eb::check_ptr(c, "cos"));
    EB_TRY(eb::check_ptr(s, "sin"));
    EB_TRY(eb::check_ptr(out, "out"));
    EB_TRY(eb::launch_rope(st, x, c, s, out, seq, nh, hd, base_pos));
    return eb::ok();
}

// Attention::prefill between the projections and the attention (nn/src/attention.rs:62-97)
// in one launch: q/k/v RMSNorm (null gains: none), RoPE of q and k at base_pos (null
// tables: none), q into q_out [rows, h, hd], K and V into cache rows base_pos.. (f32 or
// IEEE half).
static eb_status prologue_checked(hipStream_t st, const float *q, size_t qn, const float *k,
                                  size_t kn, const float *v, size_t vn, size_t rows, size_t h,
                                  size_t hkv, size_t hd, const float *gq, const float *gk,
                                  const float *gv, float eps, const float *rc, const float *rs,
                                  size_t tn, size_t base_pos, float *q_out, size_t qon,
                                  void *kc, size_t kcn, void *vc, size_t vcn, size_t max_seq,
                                  eb::CacheElem ce) {
    EB_TRY(eb::check_heads(h, hkv));
    if (hd == 0 || hd % 2 != 0)
        return fail(EB_SHAPE_MISMATCH, "attention prologue: head_dim must be even and > 0");
    if (base_pos > max_seq || rows > max_seq - base_pos)
        return fail(EB_SHAPE_MISMATCH, "attention prologue: rows [%zu, %zu) exceed max_seq %zu",
                    base_pos, base_pos + rows, max_seq);
    EB_TRY(eb::check_numel(qn, {rows, h, hd}, "q"));
    EB_TRY(eb::check_numel(kn, {rows, hkv, hd}, "k"));
    EB_TRY(eb::check_numel(vn, {rows, hkv, hd}, "v"));
    EB_TRY(eb::check_numel(qon, {rows, h, hd}, "q_out"));
    EB_TRY(eb::check_numel(kcn, {max_seq, hkv, hd}, "kcache"));
    EB_TRY(eb::check_numel(vcn, {max_seq, hkv, hd}, "vcache"));
    if ((rc == nullptr) != (rs == nullptr)) return fail(EB_OTHER, "RoPE needs both tables");
    if (rc) EB_TRY(eb::check_numel(tn, {(base_pos + rows), (hd / 2)}, "rope tables"));
    if (rows == 0) return eb::ok();
    EB_TRY(eb::check_ptr(q, "q"));
    EB_TRY(eb::check_ptr(k, "k"));
    EB_TRY(eb::check_ptr(v, "v"));
    EB_TRY(eb::check_ptr(q_out, "q_out"));
    EB_TRY(eb::check_ptr(kc, "kcache"));
    EB_TRY(eb::check_ptr(vc, "vcache"));
    eb::RowsArgs a{};
    a.nseg = 3;
    const bool rope = rc != nullptr;
    a.seg[0] = eb::RowSeg{q, q_out, gq, (int)h, 0, rope, 4};
    a.seg[1] = eb::RowSeg{k, kc, gk, (int)hkv, (int)base_pos, rope, (int)ce};
    a.seg[2] = eb::RowSeg{v, vc, gv, (int)hkv, (int)base_pos, false, (int)ce};
    a.rows = (int)rows;
    a.hd = (int)hd;
    a.eps = eps;
    a.cosb = rc;
    a.sinb = rs;
    a.rope_row0 = (int)base_pos;
    EB_TRY(eb::launch_attn_rows(st, a));
    return eb::ok();
}

// Checks the new-token rows of a fused decode step ([hkv, hd] each).
static eb_status step_rows_checked(const float *knew, const float *vnew, size_t new_n,
                                   size_t hkv, size_t hd) {
    EB_TRY(eb::check_numel(new_n, {hkv, hd}, "knew/vnew"));
    EB_TRY(eb::check_ptr(knew, "knew"));
    EB_TRY(eb::check_ptr(vnew, "vnew"));
    return EB_OK;
}

// Grows the device's workspace. Stream ordered: the old buffer is freed only after the
// stream drains, and not at all while a captured graph still has it in its kernels'
// arguments (it is then retired, and freed with the last such graph). Returns with
// dev->ws_mu held in lk.
static eb_status device_workspace(eb_device *dev, size_t floats, float **out, WsLock &lk) {
    lk = WsLock(dev->ws_mu);
    if (floats > dev->ws_floats) {
        if (dev->capturing.load())
            return fail(EB_OTHER,
                        "the device workspace would have to grow during a graph capture "
                        "(run the captured step once outside the capture first)");
        if (dev->ws) {
            if (dev->ws_graph_refs.count(dev->ws)) {
                dev->ws_retired.push_back(dev->ws);
            } else {
                EB_HIP_TRY(hipStreamSynchronize(dev->stream));
                EB_HIP_TRY(hipFree(dev->ws));
            }
            dev->ws = nullptr;
            dev->ws_floats = 0;
        }
        EB_HIP_TRY(hipMalloc((void **)&dev->ws, floats * sizeof(float)));
        dev->ws_floats = floats;
    }
    if (dev->capturing.load()) dev->ws_in_capture = true;
    *out = dev->ws;
    return EB_OK;
}

// Shared by eb_attn_decode / eb_attn_decode_step: device workspace, then one launch.
static eb_status device_decode(eb_device *dev, const float *q, const void *kc, const void *vc,
                               void *kc_w, void *vc_w, const float *knew, const float *vnew,
                               float *o, size_t h, size_t hkv, size_t pos, size_t hd,
                               float scale, size_t window = 0,
                               eb::CacheElem ce = eb::CacheElem::F32,
                               const eb::DecodePrologue *pro = nullptr) {
    size_t wsn = eb::decode_workspace_floats(h, hkv, pos, hd, dev->cu_count, ce);
    float *ws = nullptr;
    WsLock lk;
    if (wsn > 0) EB_TRY(device_workspace(dev, wsn, &ws, lk));
    EB_TRY(eb::launch_attn_decode_any(dev->stream, q, kc, vc, kc_w, vc_w, knew, vnew, o, h, hkv,
                                      pos, hd, scale, ws, wsn, dev->cu_count, window, ce, pro));
    return eb::ok();
}

// A packed-f16 weight: EB_U32 words holding two halves each, low half first (the
// reference's from_f16_packed, crates/eyebrowse-gpu/src/tensor.rs:108-116), or EB_F16
// elements. *halves = how many halves it holds.
static eb_status tensor_weight(const eb_tensor *t, const char *name, eb_device *dev,
                               size_t *halves) {
    if (!t) return fail(EB_SHAPE_MISMATCH, "%s is null", name);
    if (t->dev != dev) return fail(EB_OTHER, "%s lives on another device", name);
    if (t->dtype == EB_U32)
        *halves = 2 * eb_tensor_numel(t);
    else if (t->dtype == EB_F16)
        *halves = eb_tensor_numel(t);
    else
        return fail(EB_SHAPE_MISMATCH, "%s must be packed f16 (u32 words) or f16", name);
    return EB_OK;
}

// linear_f16w over nseg weight/output pairs that share x.
static eb_status linear_checked(hipStream_t st, const float *x, size_t xn,
                                const uint16_t *const *w, const size_t *w_halves,
                                float *const *y, const size_t *yn, const size_t *out_f, int nseg,
                                size_t m, size_t in_f, float *ws, size_t wsn) {
    if (nseg < 1 || nseg > eb::kLinearMaxSegs)
        return fail(EB_OTHER, "linear_f16w: 1 to %d weights per launch", eb::kLinearMaxSegs);
    EB_TRY(eb::check_numel(xn, {m, in_f}, "a"));
    for (int i = 0; i < nseg; ++i) {
        EB_TRY(eb::check_numel(w_halves[i], {out_f[i], in_f}, "w"));
        EB_TRY(eb::check_numel(yn[i], {m, out_f[i]}, "c"));
    }
    if (m == 0) return eb::ok();
    if (in_f > 0) EB_TRY(eb::check_ptr(x, "a"));
    for (int i = 0; i < nseg; ++i) {
        if (out_f[i] == 0) continue;
        if (in_f > 0) EB_TRY(eb::check_ptr(w[i], "w"));
        EB_TRY(eb::check_ptr(y[i], "c"));
    }
    const size_t need = eb::linear_workspace_floats(m, in_f);
    if (wsn < need)
        return fail(EB_SHAPE_MISMATCH, "linear_f16w: workspace holds %zu floats, needs %zu", wsn,
                    need);
    if (need > 0) EB_TRY(eb::check_ptr(ws, "workspace"));
    EB_TRY(eb::launch_linear_f16w_multi(st, x, w, y, out_f, nseg, m, in_f, ws, wsn));
    return eb::ok();
}

static eb_status device_linear(eb_device *dev, const eb_tensor *a,
                               const eb_tensor *const *w, eb_tensor *const *c,
                               const size_t *out_f, int nseg, size_t m, size_t in_f) {
    EB_TRY(tensor_f32(a, "a", dev));
    if (nseg < 1 || nseg > eb::kLinearMaxSegs || !w || !c || !out_f)
        return fail(EB_OTHER, "linear_f16w: 1 to %d weights per launch", eb::kLinearMaxSegs);
    const uint16_t *wp[eb::kLinearMaxSegs];
    float *yp[eb::kLinearMaxSegs];
    size_t wh[eb::kLinearMaxSegs], yn[eb::kLinearMaxSegs];
    for (int i = 0; i < nseg; ++i) {
        EB_TRY(tensor_weight(w[i], "w", dev, &wh[i]));
        EB_TRY(tensor_f32(c[i], "c", dev));
        wp[i] = static_cast<const uint16_t *>(w[i]->ptr);
        yp[i] = static_cast<float *>(c[i]->ptr);
        yn[i] = eb_tensor_numel(c[i]);
    }
    const size_t wsn = eb::linear_workspace_floats(m, in_f);
    float *ws = nullptr;
    WsLock lk;
    if (wsn > 0) EB_TRY(device_workspace(dev, wsn, &ws, lk));
    return linear_checked(dev->stream, static_cast<const float *>(a->ptr), eb_tensor_numel(a),
                          wp, wh, yp, yn, out_f, nseg, m, in_f, ws, wsn);
}

// Both caches of one layer share a dtype.
static eb_status cache_pair(const eb_tensor *kc, const eb_tensor *vc, eb_device *dev,
                            eb::CacheElem *ce) {
    eb::CacheElem ek = eb::CacheElem::F32, ev = eb::CacheElem::F32;
    EB_TRY(tensor_cache(kc, "kcache", dev, &ek));
    EB_TRY(tensor_cache(vc, "vcache", dev, &ev));
    if (ek != ev) return fail(EB_SHAPE_MISMATCH, "kcache and vcache dtypes differ");
    *ce = ek;
    return EB_OK;
}


extern "C" {

eb_status eb_kv_write(eb_recorder *rec, eb_tensor *cache, const eb_tensor *src, size_t hkv,
                      size_t count, size_t hd, size_t max_seq, size_t dst_start) {
    EB_TRY(rec_ready(rec));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(tensor_cache(cache, "cache", rec->dev, &ce));
    EB_TRY(tensor_f32(src, "src", rec->dev));
    return kv_write_checked(rec->dev->stream, cache->ptr, eb_tensor_numel(cache),
                            (const float *)src->ptr, eb_tensor_numel(src), hkv, count, hd,
                            max_seq, dst_start, ce);
}

eb_status eb_attn_prefill(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                          const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv, size_t s,
                          size_t hd, float scale) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(k, "k", rec->dev));
    EB_TRY(tensor_f32(v, "v", rec->dev));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    return prefill_checked(rec->dev->stream, (const float *)q->ptr, eb_tensor_numel(q),
                           (const float *)k->ptr, eb_tensor_numel(k), (const float *)v->ptr,
                           eb_tensor_numel(v), (float *)o->ptr, eb_tensor_numel(o), h, hkv, s,
                           hd, scale, PrefillWs{rec->dev});
}

eb_status eb_attn_prefill_pv16(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                               const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv,
                               size_t s, size_t hd, float scale) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(k, "k", rec->dev));
    EB_TRY(tensor_f32(v, "v", rec->dev));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    return prefill_checked(rec->dev->stream, (const float *)q->ptr, eb_tensor_numel(q),
                           (const float *)k->ptr, eb_tensor_numel(k), (const float *)v->ptr,
                           eb_tensor_numel(v), (float *)o->ptr, eb_tensor_numel(o), h, hkv, s,
                           hd, scale, PrefillWs{rec->dev}, true);
}

eb_status eb_attn_prefill_fast(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                               const eb_tensor *v, eb_tensor *o, size_t h, size_t hkv, size_t s,
                               size_t hd, float scale) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(k, "k", rec->dev));
    EB_TRY(tensor_f32(v, "v", rec->dev));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    return prefill_fast_checked(rec->dev->stream, (const float *)q->ptr, eb_tensor_numel(q),
                                (const float *)k->ptr, eb_tensor_numel(k), (const float *)v->ptr,
                                eb_tensor_numel(v), (float *)o->ptr, eb_tensor_numel(o), h, hkv, s,
                                hd, scale, PrefillWs{rec->dev});
}

eb_status eb_launch_attn_prefill_fast(void *stream, const float *q, size_t q_numel,
                                      const float *k, size_t k_numel, const float *v,
                                      size_t v_numel, float *o, size_t o_numel, size_t h,
                                      size_t hkv, size_t s, size_t hd, float scale) {
    return prefill_fast_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o,
                                o_numel, h, hkv, s, hd, scale);
}

size_t eb_attn_prefill_fast_workspace_floats(size_t h, size_t hkv, size_t hd, size_t s) {
    return eb::prefill_fast_workspace_floats(h, hkv, hd, s);
}

eb_status eb_launch_attn_prefill_fast_ws(void *stream, const float *q, size_t q_numel,
                                         const float *k, size_t k_numel, const float *v,
                                         size_t v_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t s, size_t hd, float scale,
                                         float *workspace, size_t workspace_floats) {
    return prefill_fast_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o,
                                o_numel, h, hkv, s, hd, scale,
                                PrefillWs{nullptr, true, workspace, workspace_floats});
}

eb_status eb_attn_decode(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                         const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                         size_t pos, size_t hd, size_t max_seq, float scale) {
    return eb_attn_decode_window(rec, q, kcache, vcache, o, h, hkv, pos, hd, max_seq, scale, 0);
}

eb_status eb_attn_prefill_chunk(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                                const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                size_t pos0, size_t rows, size_t hd, size_t max_seq,
                                float scale, size_t window) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(cache_pair(kcache, vcache, rec->dev, &ce));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    return prefill_chunk_checked(rec->dev->stream, (const float *)q->ptr, eb_tensor_numel(q),
                                 kcache->ptr, eb_tensor_numel(kcache), vcache->ptr,
                                 eb_tensor_numel(vcache), (float *)o->ptr, eb_tensor_numel(o), h,
                                 hkv, pos0, rows, hd, max_seq, scale, window, ce,
                                 PrefillWs{rec->dev});
}

eb_status eb_attn_decode_window(eb_recorder *rec, const eb_tensor *q, const eb_tensor *kcache,
                                const eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                size_t pos, size_t hd, size_t max_seq, float scale,
                                size_t window) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(cache_pair(kcache, vcache, rec->dev, &ce));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    EB_TRY(decode_shape_checked((const float *)q->ptr, eb_tensor_numel(q), kcache->ptr,
                                eb_tensor_numel(kcache), vcache->ptr, eb_tensor_numel(vcache),
                                (const float *)o->ptr, eb_tensor_numel(o), h, hkv, pos, hd,
                                max_seq, ce));
    return device_decode(rec->dev, (const float *)q->ptr, kcache->ptr, vcache->ptr, nullptr,
                         nullptr, nullptr, nullptr, (float *)o->ptr, h, hkv, pos, hd, scale,
                         window, ce);
}

eb_status eb_attn_decode_step(eb_recorder *rec, const eb_tensor *q, const eb_tensor *knew,
                              const eb_tensor *vnew, eb_tensor *kcache, eb_tensor *vcache,
                              eb_tensor *o, size_t h, size_t hkv, size_t pos, size_t hd,
                              size_t max_seq, float scale) {
    return eb_attn_decode_step_window(rec, q, knew, vnew, kcache, vcache, o, h, hkv, pos, hd,
                                      max_seq, scale, 0);
}

eb_status eb_attn_decode_step_window(eb_recorder *rec, const eb_tensor *q, const eb_tensor *knew,
                                     const eb_tensor *vnew, eb_tensor *kcache,
                                     eb_tensor *vcache, eb_tensor *o, size_t h, size_t hkv,
                                     size_t pos, size_t hd, size_t max_seq, float scale,
                                     size_t window) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(knew, "knew", rec->dev));
    EB_TRY(tensor_f32(vnew, "vnew", rec->dev));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(cache_pair(kcache, vcache, rec->dev, &ce));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    EB_TRY(decode_shape_checked((const float *)q->ptr, eb_tensor_numel(q), kcache->ptr,
                                eb_tensor_numel(kcache), vcache->ptr, eb_tensor_numel(vcache),
                                (const float *)o->ptr, eb_tensor_numel(o), h, hkv, pos, hd,
                                max_seq, ce));
    size_t nn = eb_tensor_numel(knew) < eb_tensor_numel(vnew) ? eb_tensor_numel(knew)
                                                              : eb_tensor_numel(vnew);
    EB_TRY(step_rows_checked((const float *)knew->ptr, (const float *)vnew->ptr, nn, hkv, hd));
    return device_decode(rec->dev, (const float *)q->ptr, kcache->ptr, vcache->ptr, kcache->ptr,
                         vcache->ptr, (const float *)knew->ptr, (const float *)vnew->ptr,
                         (float *)o->ptr, h, hkv, pos, hd, scale, window, ce);
}

}  // extern "C"

// eb_launch_attn_decode_step's body, shared with the no-allocation entry point.
eb_status eb::decode_step_raw(hipStream_t st, const float *q, size_t q_numel, const float *knew,
                              const float *vnew, size_t new_numel, float *kc, size_t kc_numel,
                              float *vc, size_t vc_numel, float *o, size_t o_numel, size_t h,
                              size_t hkv, size_t pos, size_t hd, size_t max_seq, float scale,
                              float *workspace, size_t workspace_floats, int cu_count) {
    EB_TRY(decode_shape_checked(q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                pos, hd, max_seq));
    EB_TRY(step_rows_checked(knew, vnew, new_numel, hkv, hd));
    int cus = cu_count > 0 ? cu_count : 256;
    size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus);
    if (workspace_floats < need)
        return fail(EB_SHAPE_MISMATCH, "attn_decode_step: workspace holds %zu floats, needs %zu",
                    workspace_floats, need);
    if (need > 0) EB_TRY(eb::check_ptr(workspace, "workspace"));
    EB_TRY(eb::launch_attn_decode(st, q, kc, vc, kc, vc, knew, vnew, o, h, hkv, pos, hd, scale,
                                  workspace, workspace_floats, cus));
    return eb::ok();
}

// Attention::decode's post-projection part in one fused step (see DecodePrologue):
// q [h, hd], knew / vnew [hkv, hd] straight from the projections.
eb_status eb::attn_decode_step_fused(eb_recorder *rec, const eb_tensor *q,
                                     const eb_tensor *knew, const eb_tensor *vnew,
                                     eb_tensor *kcache, eb_tensor *vcache, eb_tensor *o,
                                     size_t h, size_t hkv, size_t pos, size_t hd,
                                     size_t max_seq, float scale, size_t window,
                                     const eb_tensor *q_norm, const eb_tensor *k_norm,
                                     const eb_tensor *v_norm, float eps,
                                     const eb_tensor *rope_cos, const eb_tensor *rope_sin) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(knew, "knew", rec->dev));
    EB_TRY(tensor_f32(vnew, "vnew", rec->dev));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(cache_pair(kcache, vcache, rec->dev, &ce));
    EB_TRY(tensor_f32(o, "o", rec->dev));
    EB_TRY(decode_shape_checked((const float *)q->ptr, eb_tensor_numel(q), kcache->ptr,
                                eb_tensor_numel(kcache), vcache->ptr, eb_tensor_numel(vcache),
                                (const float *)o->ptr, eb_tensor_numel(o), h, hkv, pos, hd,
                                max_seq, ce));
    size_t nn = eb_tensor_numel(knew) < eb_tensor_numel(vnew) ? eb_tensor_numel(knew)
                                                              : eb_tensor_numel(vnew);
    EB_TRY(step_rows_checked((const float *)knew->ptr, (const float *)vnew->ptr, nn, hkv, hd));
    eb::DecodePrologue pro{};
    pro.eps = eps;
    const eb_tensor *norms[3] = {q_norm, k_norm, v_norm};
    const float **slots[3] = {&pro.q_norm, &pro.k_norm, &pro.v_norm};
    for (int i = 0; i < 3; ++i) {
        if (!norms[i]) continue;
        EB_TRY(tensor_f32(norms[i], "norm gain", rec->dev));
        if (eb_tensor_numel(norms[i]) != hd)
            return fail(EB_SHAPE_MISMATCH, "norm gain holds %zu, head_dim is %zu",
                        eb_tensor_numel(norms[i]), hd);
        *slots[i] = (const float *)norms[i]->ptr;
    }
    if ((rope_cos == nullptr) != (rope_sin == nullptr))
        return fail(EB_OTHER, "RoPE needs both tables");
    if (rope_cos) {
        EB_TRY(tensor_f32(rope_cos, "rope cos", rec->dev));
        EB_TRY(tensor_f32(rope_sin, "rope sin", rec->dev));
        EB_TRY(eb::check_numel(eb_tensor_numel(rope_cos), {(pos + 1), (hd / 2)}, "rope cos"));
        EB_TRY(eb::check_numel(eb_tensor_numel(rope_sin), {(pos + 1), (hd / 2)}, "rope sin"));
        pro.rope_cos = (const float *)rope_cos->ptr;
        pro.rope_sin = (const float *)rope_sin->ptr;
    }
    return device_decode(rec->dev, (const float *)q->ptr, kcache->ptr, vcache->ptr, kcache->ptr,
                         vcache->ptr, (const float *)knew->ptr, (const float *)vnew->ptr,
                         (float *)o->ptr, h, hkv, pos, hd, scale, window, ce, &pro);
}

// The prefill counterpart of attn_decode_step_fused: the handle form of prologue_checked.
eb_status eb::attn_rows_fused(eb_recorder *rec, const eb_tensor *q, const eb_tensor *k,
                              const eb_tensor *v, eb_tensor *q_out, eb_tensor *kcache,
                              eb_tensor *vcache, size_t rows, size_t h, size_t hkv, size_t hd,
                              size_t base_pos, size_t max_seq, const eb_tensor *q_norm,
                              const eb_tensor *k_norm, const eb_tensor *v_norm, float eps,
                              const eb_tensor *rope_cos, const eb_tensor *rope_sin) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(q, "q", rec->dev));
    EB_TRY(tensor_f32(k, "k", rec->dev));
    EB_TRY(tensor_f32(v, "v", rec->dev));
    EB_TRY(tensor_f32(q_out, "q_out", rec->dev));
    eb::CacheElem ce = eb::CacheElem::F32;
    EB_TRY(cache_pair(kcache, vcache, rec->dev, &ce));
    const eb_tensor *norms[3] = {q_norm, k_norm, v_norm};
    const float *g[3] = {nullptr, nullptr, nullptr};
    for (int i = 0; i < 3; ++i) {
        if (!norms[i]) continue;
        EB_TRY(tensor_f32(norms[i], "norm gain", rec->dev));
        if (eb_tensor_numel(norms[i]) != hd)
            return fail(EB_SHAPE_MISMATCH, "norm gain holds %zu, head_dim is %zu",
                        eb_tensor_numel(norms[i]), hd);
        g[i] = static_cast<const float *>(norms[i]->ptr);
    }
    if ((rope_cos == nullptr) != (rope_sin == nullptr))
        return fail(EB_OTHER, "RoPE needs both tables");
    size_t tn = 0;
    if (rope_cos) {
        EB_TRY(tensor_f32(rope_cos, "rope cos", rec->dev));
        EB_TRY(tensor_f32(rope_sin, "rope sin", rec->dev));
        tn = std::min(eb_tensor_numel(rope_cos), eb_tensor_numel(rope_sin));
    }
    return prologue_checked(
        rec->dev->stream, static_cast<const float *>(q->ptr), eb_tensor_numel(q),
        static_cast<const float *>(k->ptr), eb_tensor_numel(k), static_cast<const float *>(v->ptr),
        eb_tensor_numel(v), rows, h, hkv, hd, g[0], g[1], g[2], eps,
        rope_cos ? static_cast<const float *>(rope_cos->ptr) : nullptr,
        rope_sin ? static_cast<const float *>(rope_sin->ptr) : nullptr, tn, base_pos,
        static_cast<float *>(q_out->ptr), eb_tensor_numel(q_out), kcache->ptr,
        eb_tensor_numel(kcache), vcache->ptr, eb_tensor_numel(vcache), max_seq, ce);
}

extern "C" {

eb_status eb_rmsnorm(eb_recorder *rec, const eb_tensor *x, const eb_tensor *weight,
                     eb_tensor *out, size_t rows, size_t dim, float eps) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(x, "x", rec->dev));
    EB_TRY(tensor_f32(weight, "weight", rec->dev));
    EB_TRY(tensor_f32(out, "out", rec->dev));
    return rmsnorm_checked(rec->dev->stream, (const float *)x->ptr, eb_tensor_numel(x),
                           (const float *)weight->ptr, eb_tensor_numel(weight),
                           (float *)out->ptr, eb_tensor_numel(out), rows, dim, eps);
}

eb_status eb_rope(eb_recorder *rec, const eb_tensor *x, const eb_tensor *cos,
                  const eb_tensor *sin, eb_tensor *out, size_t seq, size_t n_heads,
                  size_t head_dim, size_t base_pos) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(x, "x", rec->dev));
    EB_TRY(tensor_f32(cos, "cos", rec->dev));
    EB_TRY(tensor_f32(sin, "sin", rec->dev));
    EB_TRY(tensor_f32(out, "out", rec->dev));
    size_t tn = eb_tensor_numel(cos) < eb_tensor_numel(sin) ? eb_tensor_numel(cos)
                                                            : eb_tensor_numel(sin);
    return rope_checked(rec->dev->stream, (const float *)x->ptr, eb_tensor_numel(x),
                        (const float *)cos->ptr, (const float *)sin->ptr, tn, (float *)out->ptr,
                        eb_tensor_numel(out), seq, n_heads, head_dim, base_pos);
}

// ---- raw launches ---------------------------------------------------------------------

eb_status eb_launch_kv_write(void *stream, float *cache, size_t cache_numel, const float *src,
                             size_t src_numel, size_t hkv, size_t count, size_t hd,
                             size_t max_seq, size_t dst_start) {
    return kv_write_checked((hipStream_t)stream, cache, cache_numel, src, src_numel, hkv, count,
                            hd, max_seq, dst_start);
}

eb_status eb_launch_attn_prefill(void *stream, const float *q, size_t q_numel, const float *k,
                                 size_t k_numel, const float *v, size_t v_numel, float *o,
                                 size_t o_numel, size_t h, size_t hkv, size_t s, size_t hd,
                                 float scale) {
    return prefill_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o, o_numel,
                           h, hkv, s, hd, scale);
}

eb_status eb_launch_attn_prefill_chunk(void *stream, const float *q, size_t q_numel,
                                       const float *kc, size_t kc_numel, const float *vc,
                                       size_t vc_numel, float *o, size_t o_numel, size_t h,
                                       size_t hkv, size_t pos0, size_t rows, size_t hd,
                                       size_t max_seq, float scale, size_t window) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window);
}

size_t eb_attn_prefill_workspace_floats(size_t h, size_t hkv, size_t hd, size_t pos0, size_t rows,
                                        size_t window) {
    if (h == 0 || hkv == 0 || h % hkv != 0 || !eb::attn_head_dim_supported(hd)) return 0;
    return eb::prefill_workspace_floats(h, hkv, hd, rows, pos0 + rows, pos0, window);
}

eb_status eb_launch_attn_prefill_ws(void *stream, const float *q, size_t q_numel, const float *k,
                                    size_t k_numel, const float *v, size_t v_numel, float *o,
                                    size_t o_numel, size_t h, size_t hkv, size_t s, size_t hd,
                                    float scale, float *workspace, size_t workspace_floats) {
    return prefill_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o, o_numel,
                           h, hkv, s, hd, scale,
                           PrefillWs{nullptr, true, workspace, workspace_floats});
}

eb_status eb_launch_attn_prefill_pv16(void *stream, const float *q, size_t q_numel,
                                      const float *k, size_t k_numel, const float *v,
                                      size_t v_numel, float *o, size_t o_numel, size_t h,
                                      size_t hkv, size_t s, size_t hd, float scale) {
    return prefill_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o, o_numel,
                           h, hkv, s, hd, scale, PrefillWs(), true);
}

eb_status eb_launch_attn_prefill_pv16_ws(void *stream, const float *q, size_t q_numel,
                                         const float *k, size_t k_numel, const float *v,
                                         size_t v_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t s, size_t hd, float scale,
                                         float *workspace, size_t workspace_floats) {
    return prefill_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, o, o_numel,
                           h, hkv, s, hd, scale,
                           PrefillWs{nullptr, true, workspace, workspace_floats}, true);
}

eb_status eb_launch_attn_prefill_chunk_ws(void *stream, const float *q, size_t q_numel,
                                          const float *kc, size_t kc_numel, const float *vc,
                                          size_t vc_numel, float *o, size_t o_numel, size_t h,
                                          size_t hkv, size_t pos0, size_t rows, size_t hd,
                                          size_t max_seq, float scale, size_t window,
                                          float *workspace, size_t workspace_floats) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window,
                                 eb::CacheElem::F32,
                                 PrefillWs{nullptr, true, workspace, workspace_floats});
}

eb_status eb_launch_attn_prefill_chunk_f16_ws(void *stream, const float *q, size_t q_numel,
                                              const uint16_t *kc, size_t kc_numel,
                                              const uint16_t *vc, size_t vc_numel, float *o,
                                              size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                              size_t rows, size_t hd, size_t max_seq,
                                              float scale, size_t window, float *workspace,
                                              size_t workspace_floats) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window,
                                 eb::CacheElem::F16,
                                 PrefillWs{nullptr, true, workspace, workspace_floats});
}

size_t eb_attn_decode_workspace_floats(size_t h, size_t hkv, size_t pos, size_t hd,
                                       int cu_count) {
    if (h == 0 || hkv == 0 || h % hkv != 0 || !eb::attn_head_dim_supported(hd)) return 0;
    return eb::decode_workspace_floats_any(h, hkv, pos, hd, cu_count > 0 ? cu_count : 256);
}

eb_status eb_launch_attn_decode(void *stream, const float *q, size_t q_numel, const float *kc,
                                size_t kc_numel, const float *vc, size_t vc_numel, float *o,
                                size_t o_numel, size_t h, size_t hkv, size_t pos, size_t hd,
                                size_t max_seq, float scale, float *workspace,
                                size_t workspace_floats, int cu_count) {
    EB_TRY(decode_shape_checked(q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                pos, hd, max_seq));
    int cus = cu_count > 0 ? cu_count : 256;
    size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus);
    if (workspace_floats < need)
        return fail(EB_SHAPE_MISMATCH, "attn_decode: workspace holds %zu floats, needs %zu",
                    workspace_floats, need);
    if (need > 0) EB_TRY(eb::check_ptr(workspace, "workspace"));
    EB_TRY(eb::launch_attn_decode((hipStream_t)stream, q, kc, vc, nullptr, nullptr, nullptr,
                                  nullptr, o, h, hkv, pos, hd, scale, workspace,
                                  workspace_floats, cus));
    return eb::ok();
}

eb_status eb_launch_attn_decode_window(void *stream, const float *q, size_t q_numel,
                                       const float *kc, size_t kc_numel, const float *vc,
                                       size_t vc_numel, float *o, size_t o_numel, size_t h,
                                       size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                       float scale, size_t window, float *workspace,
                                       size_t workspace_floats, int cu_count) {
    EB_TRY(decode_shape_checked(q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                pos, hd, max_seq));
    int cus = cu_count > 0 ? cu_count : 256;
    size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus);
    if (workspace_floats < need)
        return fail(EB_SHAPE_MISMATCH, "attn_decode: workspace holds %zu floats, needs %zu",
                    workspace_floats, need);
    if (need > 0) EB_TRY(eb::check_ptr(workspace, "workspace"));
    EB_TRY(eb::launch_attn_decode((hipStream_t)stream, q, kc, vc, nullptr, nullptr, nullptr,
                                  nullptr, o, h, hkv, pos, hd, scale, workspace,
                                  workspace_floats, cus, window));
    return eb::ok();
}

eb_status eb_launch_attn_decode_step(void *stream, const float *q, size_t q_numel,
                                     const float *knew, const float *vnew, size_t new_numel,
                                     float *kc, size_t kc_numel, float *vc, size_t vc_numel,
                                     float *o, size_t o_numel, size_t h, size_t hkv, size_t pos,
                                     size_t hd, size_t max_seq, float scale, float *workspace,
                                     size_t workspace_floats, int cu_count) {
    return eb::decode_step_raw((hipStream_t)stream, q, q_numel, knew, vnew, new_numel, kc,
                               kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos, hd, max_seq,
                               scale, workspace, workspace_floats, cu_count);
}

// ---- raw launches over IEEE-half and E4M3 KV caches ---------------------------------

}  // extern "C"

static eb_status decode_cache_raw(void *stream, const float *q, size_t q_numel, const void *kc,
                                  size_t kc_numel, const void *vc, size_t vc_numel, float *o,
                                  size_t o_numel, size_t h, size_t hkv, size_t pos, size_t hd,
                                  size_t max_seq, float scale, size_t window, float *workspace,
                                  size_t workspace_floats, int cu_count, eb::CacheElem ce) {
    EB_TRY(decode_shape_checked(q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                pos, hd, max_seq, ce));
    int cus = cu_count > 0 ? cu_count : 256;
    size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus, ce);
    if (workspace_floats < need)
        return fail(EB_SHAPE_MISMATCH, "attn_decode: workspace holds %zu floats, needs %zu",
                    workspace_floats, need);
    if (need > 0) EB_TRY(eb::check_ptr(workspace, "workspace"));
    EB_TRY(eb::launch_attn_decode_any((hipStream_t)stream, q, kc, vc, nullptr, nullptr, nullptr,
                                      nullptr, o, h, hkv, pos, hd, scale, workspace,
                                      workspace_floats, cus, window, ce));
    return eb::ok();
}

static eb_status decode_step_cache_raw(void *stream, const float *q, size_t q_numel,
                                       const float *knew, const float *vnew, size_t new_numel,
                                       void *kc, size_t kc_numel, void *vc, size_t vc_numel,
                                       float *o, size_t o_numel, size_t h, size_t hkv,
                                       size_t pos, size_t hd, size_t max_seq, float scale,
                                       size_t window, float *workspace, size_t workspace_floats,
                                       int cu_count, eb::CacheElem ce) {
    EB_TRY(decode_shape_checked(q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                pos, hd, max_seq, ce));
    EB_TRY(step_rows_checked(knew, vnew, new_numel, hkv, hd));
    int cus = cu_count > 0 ? cu_count : 256;
    size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus, ce);
    if (workspace_floats < need)
        return fail(EB_SHAPE_MISMATCH, "attn_decode_step: workspace holds %zu floats, needs %zu",
                    workspace_floats, need);
    if (need > 0) EB_TRY(eb::check_ptr(workspace, "workspace"));
    EB_TRY(eb::launch_attn_decode_any((hipStream_t)stream, q, kc, vc, kc, vc, knew, vnew, o, h,
                                      hkv, pos, hd, scale, workspace, workspace_floats, cus,
                                      window, ce));
    return eb::ok();
}

extern "C" {

eb_status eb_launch_kv_write_f16(void *stream, uint16_t *cache, size_t cache_numel,
                                 const float *src, size_t src_numel, size_t hkv, size_t count,
                                 size_t hd, size_t max_seq, size_t dst_start) {
    return kv_write_checked((hipStream_t)stream, cache, cache_numel, src, src_numel, hkv, count,
                            hd, max_seq, dst_start, eb::CacheElem::F16);
}

eb_status eb_launch_attn_prefill_chunk_f16(void *stream, const float *q, size_t q_numel,
                                           const uint16_t *kc, size_t kc_numel,
                                           const uint16_t *vc, size_t vc_numel, float *o,
                                           size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                           size_t rows, size_t hd, size_t max_seq, float scale,
                                           size_t window) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window,
                                 eb::CacheElem::F16);
}

eb_status eb_launch_attn_decode_f16(void *stream, const float *q, size_t q_numel,
                                    const uint16_t *kc, size_t kc_numel, const uint16_t *vc,
                                    size_t vc_numel, float *o, size_t o_numel, size_t h,
                                    size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                    float scale, size_t window, float *workspace,
                                    size_t workspace_floats, int cu_count) {
    return decode_cache_raw(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                            pos, hd, max_seq, scale, window, workspace, workspace_floats,
                            cu_count, eb::CacheElem::F16);
}

eb_status eb_launch_attn_decode_step_f16(void *stream, const float *q, size_t q_numel,
                                         const float *knew, const float *vnew, size_t new_numel,
                                         uint16_t *kc, size_t kc_numel, uint16_t *vc,
                                         size_t vc_numel, float *o, size_t o_numel, size_t h,
                                         size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                         float scale, size_t window, float *workspace,
                                         size_t workspace_floats, int cu_count) {
    return decode_step_cache_raw(stream, q, q_numel, knew, vnew, new_numel, kc, kc_numel, vc,
                                 vc_numel, o, o_numel, h, hkv, pos, hd, max_seq, scale, window,
                                 workspace, workspace_floats, cu_count, eb::CacheElem::F16);
}

eb_status eb_launch_kv_write_f8(void *stream, uint8_t *cache, size_t cache_numel,
                                const float *src, size_t src_numel, size_t hkv, size_t count,
                                size_t hd, size_t max_seq, size_t dst_start) {
    return kv_write_checked((hipStream_t)stream, cache, cache_numel, src, src_numel, hkv, count,
                            hd, max_seq, dst_start, eb::CacheElem::E4M3);
}

eb_status eb_launch_attn_prefill_chunk_f8(void *stream, const float *q, size_t q_numel,
                                          const uint8_t *kc, size_t kc_numel, const uint8_t *vc,
                                          size_t vc_numel, float *o, size_t o_numel, size_t h,
                                          size_t hkv, size_t pos0, size_t rows, size_t hd,
                                          size_t max_seq, float scale, size_t window) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window,
                                 eb::CacheElem::E4M3);
}

eb_status eb_launch_attn_prefill_chunk_f8_ws(void *stream, const float *q, size_t q_numel,
                                             const uint8_t *kc, size_t kc_numel,
                                             const uint8_t *vc, size_t vc_numel, float *o,
                                             size_t o_numel, size_t h, size_t hkv, size_t pos0,
                                             size_t rows, size_t hd, size_t max_seq,
                                             float scale, size_t window, float *workspace,
                                             size_t workspace_floats) {
    return prefill_chunk_checked((hipStream_t)stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                 o_numel, h, hkv, pos0, rows, hd, max_seq, scale, window,
                                 eb::CacheElem::E4M3,
                                 PrefillWs{nullptr, true, workspace, workspace_floats});
}

eb_status eb_launch_attn_decode_f8(void *stream, const float *q, size_t q_numel,
                                   const uint8_t *kc, size_t kc_numel, const uint8_t *vc,
                                   size_t vc_numel, float *o, size_t o_numel, size_t h,
                                   size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                   float scale, size_t window, float *workspace,
                                   size_t workspace_floats, int cu_count) {
    return decode_cache_raw(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                            pos, hd, max_seq, scale, window, workspace, workspace_floats,
                            cu_count, eb::CacheElem::E4M3);
}

eb_status eb_launch_attn_decode_step_f8(void *stream, const float *q, size_t q_numel,
                                        const float *knew, const float *vnew, size_t new_numel,
                                        uint8_t *kc, size_t kc_numel, uint8_t *vc,
                                        size_t vc_numel, float *o, size_t o_numel, size_t h,
                                        size_t hkv, size_t pos, size_t hd, size_t max_seq,
                                        float scale, size_t window, float *workspace,
                                        size_t workspace_floats, int cu_count) {
    return decode_step_cache_raw(stream, q, q_numel, knew, vnew, new_numel, kc, kc_numel, vc,
                                 vc_numel, o, o_numel, h, hkv, pos, hd, max_seq, scale, window,
                                 workspace, workspace_floats, cu_count, eb::CacheElem::E4M3);
}

eb_status eb_launch_selftest_lane_ops(void *stream, const float *in, float *out) {
    EB_TRY(eb::check_ptr(in, "in"));
    EB_TRY(eb::check_ptr(out, "out"));
    EB_TRY(eb::launch_lane_ops((hipStream_t)stream, in, out));
    return eb::ok();
}

eb_status eb_launch_rmsnorm(void *stream, const float *x, size_t x_numel, const float *weight,
                            size_t w_numel, float *out, size_t out_numel, size_t rows,
                            size_t dim, float eps) {
    return rmsnorm_checked((hipStream_t)stream, x, x_numel, weight, w_numel, out, out_numel,
                           rows, dim, eps);
}

eb_status eb_launch_attn_prologue(void *stream, const float *q, size_t q_numel, const float *k,
                                  size_t k_numel, const float *v, size_t v_numel, size_t rows,
                                  size_t h, size_t hkv, size_t hd, const float *q_norm,
                                  const float *k_norm, const float *v_norm, float eps,
                                  const float *rope_cos, const float *rope_sin,
                                  size_t table_numel, size_t base_pos, float *q_out,
                                  size_t q_out_numel, void *kcache, size_t kc_numel,
                                  void *vcache, size_t vc_numel, size_t max_seq,
                                  eb_dtype cache_dtype) {
    if (cache_dtype != EB_F32 && cache_dtype != EB_F16 && cache_dtype != EB_F8E4M3)
        return fail(EB_UNSUPPORTED_CONFIG,
                    "attention prologue: caches must be f32, f16 or f8e4m3");
    return prologue_checked((hipStream_t)stream, q, q_numel, k, k_numel, v, v_numel, rows, h, hkv,
                            hd, q_norm, k_norm, v_norm, eps, rope_cos, rope_sin, table_numel,
                            base_pos, q_out, q_out_numel, kcache, kc_numel, vcache, vc_numel,
                            max_seq,
                            cache_dtype == EB_F16      ? eb::CacheElem::F16
                            : cache_dtype == EB_F8E4M3 ? eb::CacheElem::E4M3
                                                       : eb::CacheElem::F32);
}

eb_status eb_launch_rope(void *stream, const float *x, size_t x_numel, const float *cos,
                         const float *sin, size_t table_numel, float *out, size_t out_numel,
                         size_t seq, size_t n_heads, size_t head_dim, size_t base_pos) {
    return rope_checked((hipStream_t)stream, x, x_numel, cos, sin, table_numel, out, out_numel,
                        seq, n_heads, head_dim, base_pos);
}

eb_status eb_linear_f16w(eb_recorder *rec, const eb_tensor *a, const eb_tensor *w, eb_tensor *c,
                         size_t m, size_t in_f, size_t out_f) {
    EB_TRY(rec_ready(rec));
    return device_linear(rec->dev, a, &w, &c, &out_f, 1, m, in_f);
}

eb_status eb_linear_f16w_multi(eb_recorder *rec, const eb_tensor *a, size_t n,
                               const eb_tensor *const *w, eb_tensor *const *c,
                               const size_t *out_f, size_t m, size_t in_f) {
    EB_TRY(rec_ready(rec));
    if (n < 1 || n > (size_t)eb::kLinearMaxSegs)
        return fail(EB_OTHER, "linear_f16w: 1 to %d weights per launch", eb::kLinearMaxSegs);
    return device_linear(rec->dev, a, w, c, out_f, (int)n, m, in_f);
}

size_t eb_linear_workspace_floats(size_t m, size_t in_f) {
    return eb::linear_workspace_floats(m, in_f);
}

eb_status eb_launch_linear_f16w(void *stream, const float *a, size_t a_numel, const uint16_t *w,
                                size_t w_halves, float *c, size_t c_numel, size_t m, size_t in_f,
                                size_t out_f, float *workspace, size_t workspace_floats) {
    return linear_checked((hipStream_t)stream, a, a_numel, &w, &w_halves, &c, &c_numel, &out_f,
                          1, m, in_f, workspace, workspace_floats);
}


static eb_status argmax_checked(hipStream_t st, const float *x, size_t xn, uint32_t *out,
                                size_t out_n, size_t vocab, float *ws, size_t wsn) {
    EB_TRY(eb::check_numel(xn, vocab, "logits"));
    EB_TRY(eb::check_numel(out_n, 1, "out_idx"));
    EB_TRY(eb::check_ptr(out, "out_idx"));
    if (vocab > 0) EB_TRY(eb::check_ptr(x, "logits"));
    const size_t need = eb::argmax_workspace_floats(vocab);
    if (wsn < need)
        return fail(EB_SHAPE_MISMATCH, "argmax: workspace holds %zu floats, needs %zu", wsn, need);
    EB_TRY(eb::check_ptr(ws, "workspace"));
    EB_TRY(eb::launch_argmax(st, x, vocab, out, ws, wsn));
    return eb::ok();
}

eb_status eb_argmax(eb_recorder *rec, const eb_tensor *logits, eb_tensor *out_idx,
                    size_t vocab) {
    EB_TRY(rec_ready(rec));
    EB_TRY(tensor_f32(logits, "logits", rec->dev));
    if (!out_idx || (out_idx->dtype != EB_U32 && out_idx->dtype != EB_I32))
        return fail(EB_SHAPE_MISMATCH, "argmax: out_idx must be a u32 tensor");
    if (out_idx->dev != rec->dev) return fail(EB_OTHER, "out_idx lives on another device");
    const size_t wsn = eb::argmax_workspace_floats(vocab);
    float *ws = nullptr;
    WsLock lk;
    EB_TRY(device_workspace(rec->dev, wsn, &ws, lk));
    return argmax_checked(rec->dev->stream, static_cast<const float *>(logits->ptr),
                          eb_tensor_numel(logits), static_cast<uint32_t *>(out_idx->ptr),
                          eb_tensor_numel(out_idx), vocab, ws, wsn);
}

size_t eb_argmax_workspace_floats(size_t vocab) { return eb::argmax_workspace_floats(vocab); }

eb_status eb_launch_argmax(void *stream, const float *logits, size_t logits_numel,
                           uint32_t *out_idx, size_t vocab, float *workspace,
                           size_t workspace_floats) {
    return argmax_checked((hipStream_t)stream, logits, logits_numel, out_idx, 1, vocab,
                          workspace, workspace_floats);
}

}  // extern "C"
