// The fused decode step on a static scratch area, for callers that cannot allocate device
// memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
//
// eb_launch_attn_decode_step takes a caller workspace for the split-KV partials (part_acc,
// part_ml). This variant keeps them in `scratch`, a file-scope device array of kScratchFloats
// floats (4 MiB) that every GPU the library runs on holds until the process ends. The host
// never passes `scratch` itself to a kernel: in host code the name is a stand-in, not a
// device address. When a device is set up (eb_device_new), or else on the first call on a
// device, with that device current, the device's own address of its copy is looked up
// (hipGetSymbolAddress) and kept per device ordinal; the kernels take that address as
// their workspace argument. The partials need no clearing
// (every slot the merge reads is written first in the same launch sequence). All calls on
// one GPU share its array: calls that overlap on one GPU (different streams, or threads
// without ordering) race, so callers order them, e.g. on one stream.
#include "eb_internal.h"

#include <mutex>

namespace {

constexpr size_t kScratchFloats = (size_t)1 << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices];  // per device ordinal: its copy's device address

}  // namespace

namespace eb {

// The current device's copy of `scratch`, looked up once per device: by eb_device_new (the
// library's set-up call, so that a later capture makes no lookup), or else by the first
// no-allocation call on that device.
eb_status noalloc_scratch_of_current_device(float **out) {
    int dev = -1;
    EB_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return eb::fail(EB_UNSUPPORTED_CONFIG, "no-allocation decode: device ordinal %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        EB_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return eb::fail(EB_OTHER, "no-allocation decode: scratch has no device address");
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    if (out) *out = g_scratch_ptr[dev];
    return EB_OK;
}

}  // namespace eb

extern "C" {

size_t eb_attn_decode_noalloc_max_floats(void) { return kScratchFloats; }

eb_status eb_launch_attn_decode_step_noalloc(void *stream, const float *q, size_t q_numel,
                                             const float *knew, const float *vnew,
                                             size_t new_numel, float *kc, size_t kc_numel,
                                             float *vc, size_t vc_numel, float *o,
                                             size_t o_numel, size_t h, size_t hkv, size_t pos,
                                             size_t hd, size_t max_seq, float scale,
                                             int cu_count) {
    const int cus = cu_count > 0 ? cu_count : 256;
    if (h > 0 && hkv > 0 && h % hkv == 0 && eb::attn_head_dim_supported(hd)) {
        const size_t need = eb::decode_workspace_floats(h, hkv, pos, hd, cus);
        if (need > kScratchFloats)
            return eb::fail(EB_UNSUPPORTED_CONFIG,
                            "attn_decode_step_noalloc: this shape needs %zu floats of split "
                            "partials, the static scratch holds %zu (use "
                            "eb_launch_attn_decode_step with a workspace)",
                            need, kScratchFloats);
    }
    float *ws = nullptr;
    const eb_status st = eb::noalloc_scratch_of_current_device(&ws);
    if (st != EB_OK) return st;
    return eb::decode_step_raw((hipStream_t)stream, q, q_numel, knew, vnew, new_numel, kc,
                               kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos, hd, max_seq,
                               scale, ws, kScratchFloats, cus);
}

}  // extern "C"
