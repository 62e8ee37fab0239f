// eyebrowse-nn pieces around the attention kernels: Rope tables, KvCache and the
// Attention forward between the projections.
//
//  - eb_rope_build_partial: crates/eyebrowse-nn/src/rope.rs:24-50 (host f64 tables).
//  - eb_kv_cache_new_per_layer: crates/eyebrowse-nn/src/kv_cache.rs:29-50.
//  - eb_attention_forward_qkv: crates/eyebrowse-nn/src/attention.rs:30-185 from the
//    projected q/k/v on (the q/k/v/o projections are the caller's).
#include <cmath>
#include <memory>
#include <vector>

#include "eb_internal.h"

struct eb_rope_tables {
    eb_tensor *cos = nullptr;
    eb_tensor *sin = nullptr;
    size_t head_dim = 0;
    size_t max_seq = 0;
};

struct eb_kv_cache {
    std::vector<eb_tensor *> k, v;
    size_t max_seq = 0;
    size_t n_kv_heads = 0;
};

struct eb_attention {
    eb_attention_desc d{};
};

using eb::fail;

#define EB_TRY(expr)                      \
    do {                                  \
        eb_status eb_s_ = (expr);         \
        if (eb_s_ != EB_OK) return eb_s_; \
    } while (0)

namespace {

// Owns a tensor for the duration of a forward; released (back to the pool) on scope exit.
struct Owned {
    eb_tensor *t = nullptr;
    Owned() = default;
    explicit Owned(eb_tensor *x) : t(x) {}
    Owned(const Owned &) = delete;
    Owned &operator=(const Owned &) = delete;
    ~Owned() { eb_tensor_release(t); }
    eb_tensor *release() {
        eb_tensor *x = t;
        t = nullptr;
        return x;
    }
};

eb_device *tensor_device_of(const eb_tensor *t) { return eb::tensor_device(t); }

}  // namespace

extern "C" {

eb_status eb_rope_build_partial(eb_device *dev, size_t max_seq, size_t head_dim,
                                size_t rope_angles, float theta, eb_rope_tables **out) {
    if (!dev || !out) return fail(EB_OTHER, "device/out is null");
    if (head_dim == 0 || head_dim % 2 != 0)
        return fail(EB_SHAPE_MISMATCH, "rope: head_dim must be even and positive");
    *out = nullptr;
    const size_t half = head_dim / 2;
    std::vector<float> c(max_seq * half, 1.0f), s(max_seq * half, 0.0f);
    const double th = (double)theta;
    const double hd = (double)head_dim;
    const size_t na = rope_angles < half ? rope_angles : half;
    for (size_t p = 0; p < max_seq; ++p)
        for (size_t kk = 0; kk < na; ++kk) {
            double inv_freq = std::pow(th, -(2.0 * (double)kk) / hd);
            double angle = (double)p * inv_freq;
            c[p * half + kk] = (float)std::cos(angle);
            s[p * half + kk] = (float)std::sin(angle);
        }
    auto r = std::make_unique<eb_rope_tables>();
    const size_t shape[2] = {max_seq, half};
    EB_TRY(eb_tensor_from_f32(dev, shape, 2, c.data(), c.size(), &r->cos));
    eb_status st = eb_tensor_from_f32(dev, shape, 2, s.data(), s.size(), &r->sin);
    if (st != EB_OK) {
        eb_tensor_release(r->cos);
        return st;
    }
    r->head_dim = head_dim;
    r->max_seq = max_seq;
    *out = r.release();
    return eb::ok();
}

void eb_rope_tables_release(eb_rope_tables *rope) {
    if (!rope) return;
    eb_tensor_release(rope->cos);
    eb_tensor_release(rope->sin);
    delete rope;
}

const eb_tensor *eb_rope_tables_cos(const eb_rope_tables *rope) { return rope ? rope->cos : nullptr; }
const eb_tensor *eb_rope_tables_sin(const eb_rope_tables *rope) { return rope ? rope->sin : nullptr; }

eb_status eb_rope_apply(const eb_rope_tables *rope, eb_recorder *rec, const eb_tensor *x, size_t seq,
                        size_t n_heads, size_t base_pos, eb_tensor **out) {
    if (!rope || !rec || !x || !out) return fail(EB_OTHER, "rope_apply: null argument");
    *out = nullptr;
    if (base_pos + seq > rope->max_seq)
        return fail(EB_SHAPE_MISMATCH, "rope_apply: positions up to %zu exceed the table (%zu)",
                    base_pos + seq, rope->max_seq);
    const size_t shape[3] = {seq, n_heads, rope->head_dim};
    eb_tensor *o = nullptr;
    EB_TRY(eb_tensor_empty(tensor_device_of(x), shape, 3, EB_F32, &o));
    Owned guard(o);
    EB_TRY(eb_rope(rec, x, rope->cos, rope->sin, o, seq, n_heads, rope->head_dim, base_pos));
    *out = guard.release();
    return eb::ok();
}

eb_status eb_kv_cache_new_per_layer(eb_device *dev, const size_t *head_dims, size_t n_layers,
                                    size_t max_seq, size_t n_kv_heads, eb_kv_cache **out) {
    return eb_kv_cache_new_per_layer_dtype(dev, head_dims, n_layers, max_seq, n_kv_heads, EB_F32,
                                           out);
}

eb_status eb_kv_cache_new_per_layer_dtype(eb_device *dev, const size_t *head_dims,
                                          size_t n_layers, size_t max_seq, size_t n_kv_heads,
                                          eb_dtype dtype, eb_kv_cache **out) {
    if (!dev || !out || (n_layers > 0 && !head_dims))
        return fail(EB_OTHER, "kv_cache: null argument");
    if (dtype != EB_F32 && dtype != EB_F16 && dtype != EB_F8E4M3)
        return fail(EB_UNSUPPORTED_CONFIG, "kv_cache: element type must be f32, f16 or f8e4m3");
    *out = nullptr;
    auto kv = std::make_unique<eb_kv_cache>();
    kv->max_seq = max_seq;
    kv->n_kv_heads = n_kv_heads;
    for (size_t l = 0; l < n_layers; ++l) {
        const size_t shape[3] = {max_seq, n_kv_heads, head_dims[l]};
        eb_tensor *kt = nullptr, *vt = nullptr;
        eb_status st = eb_tensor_empty(dev, shape, 3, dtype, &kt);
        if (st == EB_OK) st = eb_tensor_empty(dev, shape, 3, dtype, &vt);
        if (st != EB_OK) {
            eb_tensor_release(kt);
            eb_kv_cache_release(kv.release());
            return st;
        }
        kv->k.push_back(kt);
        kv->v.push_back(vt);
    }
    *out = kv.release();
    return eb::ok();
}

void eb_kv_cache_release(eb_kv_cache *kv) {
    if (!kv) return;
    for (eb_tensor *t : kv->k) eb_tensor_release(t);
    for (eb_tensor *t : kv->v) eb_tensor_release(t);
    delete kv;
}

eb_tensor *eb_kv_cache_k(eb_kv_cache *kv, size_t layer) {
    return (kv && layer < kv->k.size()) ? kv->k[layer] : nullptr;
}
eb_tensor *eb_kv_cache_v(eb_kv_cache *kv, size_t layer) {
    return (kv && layer < kv->v.size()) ? kv->v[layer] : nullptr;
}
size_t eb_kv_cache_max_seq(const eb_kv_cache *kv) { return kv ? kv->max_seq : 0; }

// A packed-f16 weight of n halves: EB_U32 words (two halves each, odd tail padded) or
// EB_F16 elements.
static bool weight_holds(const eb_tensor *w, size_t n) {
    if (eb_tensor_dtype(w) == EB_U32) return eb_tensor_numel(w) == (n + 1) / 2;
    if (eb_tensor_dtype(w) == EB_F16) return eb_tensor_numel(w) == n;
    return false;
}

eb_status eb_attention_new(const eb_attention_desc *desc, eb_attention **out) {
    if (!desc || !out) return fail(EB_OTHER, "attention_new: null argument");
    *out = nullptr;
    EB_TRY(eb::check_heads(desc->n_heads, desc->n_kv_heads));
    if (!eb::attn_head_dim_supported(desc->head_dim))
        return fail(EB_UNSUPPORTED_CONFIG, "attention: head_dim %zu not supported",
                    desc->head_dim);
    const eb_tensor *norms[3] = {desc->q_norm, desc->k_norm, desc->v_norm};
    for (const eb_tensor *n : norms)
        if (n && (eb_tensor_dtype(n) != EB_F32 || eb_tensor_numel(n) != desc->head_dim))
            return fail(EB_SHAPE_MISMATCH, "attention: norm weights must be [head_dim] f32");
    const eb_tensor *proj[4] = {desc->q_proj, desc->k_proj, desc->v_proj, desc->o_proj};
    const size_t qd = desc->n_heads * desc->head_dim, kd = desc->n_kv_heads * desc->head_dim;
    const size_t outs[4] = {qd, kd, kd, desc->hidden};
    const size_t ins[4] = {desc->hidden, desc->hidden, desc->hidden, qd};
    const int given = (proj[0] != nullptr) + (proj[1] != nullptr) + (proj[2] != nullptr) +
                      (proj[3] != nullptr);
    if (given != 0 && given != 4)
        return fail(EB_SHAPE_MISMATCH, "attention: give all four projections or none");
    if (given == 4) {
        if (desc->hidden == 0) return fail(EB_SHAPE_MISMATCH, "attention: hidden must be > 0");
        for (int i = 0; i < 4; ++i)
            if (!weight_holds(proj[i], outs[i] * ins[i]))
                return fail(EB_SHAPE_MISMATCH,
                            "attention: projection %d must be packed f16 [%zu, %zu]", i, outs[i],
                            ins[i]);
    }
    auto a = std::make_unique<eb_attention>();
    a->d = *desc;
    *out = a.release();
    return eb::ok();
}

void eb_attention_release(eb_attention *attn) { delete attn; }

}  // extern "C"


extern "C" eb_status eb_attention_forward_qkv(const eb_attention *attn, eb_recorder *rec,
                                              const eb_tensor *q, const eb_tensor *k,
                                              const eb_tensor *v, const eb_rope_tables *rope,
                                              eb_kv_cache *kv, size_t layer, size_t rows,
                                              size_t base_pos, eb_tensor **out) {
    if (!attn || !rec || !q || !k || !v || !rope || !kv || !out)
        return fail(EB_OTHER, "attention_forward: null argument");
    *out = nullptr;
    const eb_attention_desc &d = attn->d;
    const size_t H = d.n_heads, Hkv = d.n_kv_heads, hd = d.head_dim;
    if (layer >= kv->k.size())
        return fail(EB_SHAPE_MISMATCH, "attention_forward: layer %zu of %zu", layer,
                    kv->k.size());
    if (rope->head_dim != hd)
        return fail(EB_SHAPE_MISMATCH, "attention_forward: rope head_dim %zu != %zu",
                    rope->head_dim, hd);
    eb_tensor *kc = kv->k[layer], *vc = kv->v[layer];
    if (eb_tensor_numel(kc) != kv->max_seq * Hkv * hd)
        return fail(EB_SHAPE_MISMATCH, "attention_forward: cache layer is not [max_seq, %zu, %zu]",
                    Hkv, hd);
    if (rows == 0) return fail(EB_SHAPE_MISMATCH, "attention_forward: rows must be > 0");
    if (base_pos > kv->max_seq || rows > kv->max_seq - base_pos)
        return fail(EB_SHAPE_MISMATCH, "attention_forward: rows [%zu, %zu) exceed max_seq %zu",
                    base_pos, base_pos + rows, kv->max_seq);
    if (eb_tensor_numel(q) != rows * H * hd || eb_tensor_numel(k) != rows * Hkv * hd ||
        eb_tensor_numel(v) != rows * Hkv * hd)
        return fail(EB_SHAPE_MISMATCH, "attention_forward: q/k/v are not [rows, heads*head_dim]");

    const eb::CacheElem ce = eb_tensor_dtype(kc) == EB_F16    ? eb::CacheElem::F16
                             : eb_tensor_dtype(kc) == EB_F8E4M3 ? eb::CacheElem::E4M3
                                                                : eb::CacheElem::F32;
    if (rows == 1 && !eb::decode_fuses_rope(hd, ce)) {
        // The step's lane layout cannot rotate this head dim over a narrow cache: the
        // pre-attention pass (norms, RoPE, cache write of row base_pos), then attn_decode.
        const size_t qshape1[3] = {1, H, hd};
        eb_tensor *qr1 = nullptr;
        EB_TRY(eb_tensor_empty(tensor_device_of(q), qshape1, 3, EB_F32, &qr1));
        Owned qr(qr1);
        EB_TRY(eb::attn_rows_fused(rec, q, k, v, qr.t, kc, vc, 1, H, Hkv, hd, base_pos,
                                   kv->max_seq, d.q_norm, d.k_norm, d.v_norm, d.norm_eps,
                                   rope->cos, rope->sin));
        const size_t oshape1[2] = {1, H * hd};
        eb_tensor *o1 = nullptr;
        EB_TRY(eb_tensor_empty(tensor_device_of(q), oshape1, 2, EB_F32, &o1));
        Owned o(o1);
        EB_TRY(eb_attn_decode_window(rec, qr.t, kc, vc, o.t, H, Hkv, base_pos, hd, kv->max_seq,
                                     d.scale, d.window));
        *out = o.release();
        return eb::ok();
    }
    if (rows == 1) {
        // attention.rs:133-183 after the projections: q/k/v norms, RoPE at pos, kv_write
        // of K and V, attn_decode; all of it inside the fused decode step.
        const size_t oshape1[2] = {1, H * hd};
        eb_tensor *o1 = nullptr;
        EB_TRY(eb_tensor_empty(tensor_device_of(q), oshape1, 2, EB_F32, &o1));
        Owned o(o1);
        EB_TRY(eb::attn_decode_step_fused(rec, q, k, v, kc, vc, o.t, H, Hkv, base_pos, hd,
                                          kv->max_seq, d.scale, d.window, d.q_norm, d.k_norm,
                                          d.v_norm, d.norm_eps, rope->cos, rope->sin));
        *out = o.release();
        return eb::ok();
    }

    // attention.rs:62-97 in one launch: q/k/v norms, RoPE of q and k at base_pos, q into
    // qr, the new rows' K (post-RoPE) and V (post-norm) into the cache at base_pos.
    const size_t qshape[3] = {rows, H, hd};
    eb_tensor *qr_t = nullptr;
    EB_TRY(eb_tensor_empty(tensor_device_of(q), qshape, 3, EB_F32, &qr_t));
    Owned qr(qr_t);
    EB_TRY(eb::attn_rows_fused(rec, q, k, v, qr.t, kc, vc, rows, H, Hkv, hd, base_pos,
                               kv->max_seq, d.q_norm, d.k_norm, d.v_norm, d.norm_eps, rope->cos,
                               rope->sin));
    const size_t oshape[2] = {rows, H * hd};
    eb_tensor *o_t = nullptr;
    EB_TRY(eb_tensor_empty(tensor_device_of(q), oshape, 2, EB_F32, &o_t));
    Owned o(o_t);
    if (base_pos == 0 && d.window == 0 && eb_tensor_dtype(kc) == EB_F32) {
        // attention.rs:104-115 (routing rule :40): a prompt attends its fresh K / V, which
        // are cache rows 0..rows-1 ([rows, Hkv, hd] at the start of the seq-major cache).
        EB_TRY(eb_attn_prefill(rec, qr.t, kc, vc, o.t, H, Hkv, rows, hd, d.scale));
    } else {
        // A continuation chunk, a windowed prompt, or any prompt over an f16 cache
        // (so that prompt and decode read the same rounded K/V) attends the cache.
        EB_TRY(eb_attn_prefill_chunk(rec, qr.t, kc, vc, o.t, H, Hkv, base_pos, rows, hd,
                                     kv->max_seq, d.scale, d.window));
    }
    *out = o.release();
    return eb::ok();
}

// Attention::forward with the projections (attention.rs:30-45; prefill :49-117, decode
// :120-185): q/k/v = x . W^T in one launch, the post-projection part above, then o_proj.
extern "C" eb_status eb_attention_forward(const eb_attention *attn, eb_recorder *rec,
                                          const eb_tensor *x, const eb_rope_tables *rope,
                                          eb_kv_cache *kv, size_t layer, size_t rows,
                                          size_t base_pos, eb_tensor **out) {
    if (!attn || !rec || !x || !out) return fail(EB_OTHER, "attention_forward: null argument");
    *out = nullptr;
    const eb_attention_desc &d = attn->d;
    if (!d.q_proj) return fail(EB_SHAPE_MISMATCH, "attention_forward: no projection weights");
    const size_t qd = d.n_heads * d.head_dim, kd = d.n_kv_heads * d.head_dim;
    if (eb_tensor_dtype(x) != EB_F32 || eb_tensor_numel(x) != rows * d.hidden)
        return fail(EB_SHAPE_MISMATCH, "attention_forward: x is not [rows, hidden] f32");
    eb_device *dev = tensor_device_of(x);
    const size_t qs[2] = {rows, qd}, ks[2] = {rows, kd};
    eb_tensor *qt = nullptr, *kt = nullptr, *vt = nullptr;
    EB_TRY(eb_tensor_empty(dev, qs, 2, EB_F32, &qt));
    Owned q(qt);
    EB_TRY(eb_tensor_empty(dev, ks, 2, EB_F32, &kt));
    Owned k(kt);
    EB_TRY(eb_tensor_empty(dev, ks, 2, EB_F32, &vt));
    Owned v(vt);
    const eb_tensor *w[3] = {d.q_proj, d.k_proj, d.v_proj};
    eb_tensor *c[3] = {q.t, k.t, v.t};
    const size_t of[3] = {qd, kd, kd};
    EB_TRY(eb_linear_f16w_multi(rec, x, 3, w, c, of, rows, d.hidden));
    eb_tensor *ot = nullptr;
    EB_TRY(eb_attention_forward_qkv(attn, rec, q.t, k.t, v.t, rope, kv, layer, rows, base_pos,
                                    &ot));
    Owned o(ot);
    const size_t ys[2] = {rows, d.hidden};
    eb_tensor *yt = nullptr;
    EB_TRY(eb_tensor_empty(dev, ys, 2, EB_F32, &yt));
    Owned y(yt);
    EB_TRY(eb_linear_f16w(rec, o.t, d.o_proj, y.t, rows, qd, d.hidden));
    *out = y.release();
    return eb::ok();
}
