"""The substrate and the eyebrowse-nn pieces on the GPU: buffer-pool semantics
(crates/eyebrowse-gpu/src/device.rs:119-161), RMSNorm / RoPE kernels and tables
(rmsnorm.rs:72-90, rope.rs:92-111, nn/src/rope.rs:82-104, nn/src/tests.rs:152-177),
per-layer caches (kv_cache.rs:56-65), the Attention forward against the oracle chain,
and the prefill/decode consistency invariant (nn/src/tests.rs:181-244)."""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload
from tests._textbook import rel_l2_f64

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- substrate -------------

def test_empty_recycles_buffers_through_the_pool():
    """device.rs:119-139, on a fresh device."""
    note("pool recycle")
    d = eb.Device.new(0)
    size = 64 * 4
    assert d.pooled(size) == 0
    eb.Tensor.empty(d, (64,)).release()
    assert d.pooled(size) == 1
    t = eb.Tensor.empty(d, (64,))
    assert d.pooled(size) == 0
    t.release()
    assert d.pooled(size) == 1


def test_host_initialized_tensors_do_not_draw_from_the_pool():
    """device.rs:141-161."""
    note("pool host-initialized")
    d = eb.Device.new(0)
    eb.Tensor.empty(d, (4,)).release()
    assert d.pooled(16) == 1
    t = eb.Tensor.from_f32(d, (4,), [1.0, 2.0, 3.0, 4.0])
    assert d.pooled(16) == 1
    np.testing.assert_array_equal(t.to_f32(), [1, 2, 3, 4])
    # Drop recycles every buffer up to MAX_POOLED_BYTES, host-initialised ones included
    # (tensor.rs:41-47 calls recycle_buffer unconditionally).
    t.release()
    assert d.pooled(16) == 2


def test_large_buffers_bypass_the_pool():
    d = eb.Device.new(0)
    big = (64 << 20) // 4 + 1
    eb.Tensor.empty(d, (big,)).release()
    assert d.pooled(big * 4) == 0


def test_upload_readback_round_trip(dev):
    x = np.arange(1000, dtype=np.float32) * 0.5 - 3
    t = eb.Tensor.from_f32(dev, (10, 100), x)
    assert t.shape == (10, 100) and t.dtype == eb.DType.F32 and t.numel() == 1000
    np.testing.assert_array_equal(t.to_f32(), x)
    u = eb.Tensor.from_u32(dev, (3,), [1, 2, 0xFFFFFFFF])
    assert np.frombuffer(u.read_bytes(), np.uint32).tolist() == [1, 2, 0xFFFFFFFF]


def test_kv_cache_per_layer_shapes(dev):
    """kv_cache.rs:56-65."""
    cache = eb.KvCache.new_per_layer(dev, [16, 32], 8, 2)
    assert cache.k[0].shape == (8, 2, 16) and cache.k[1].shape == (8, 2, 32)
    assert cache.v[0].shape == (8, 2, 16) and cache.v[1].shape == (8, 2, 32)


# ---------------------------------------------------------------- RMSNorm / RoPE --------

def test_rmsnorm_reference_case(dev):
    """rmsnorm.rs:72-90 (rows 3, dim 320 > 256); reference bar rel_l2 < 1e-4."""
    note("rmsnorm reference case")
    rows, dim, eps = 3, 320, 1e-6
    x = (np.arange(rows * dim) % 17).astype(np.float32) * np.float32(0.05) - np.float32(0.4)
    w = np.float32(1.0) + np.arange(dim, dtype=np.float32) * np.float32(0.001)
    xt, wt = upload(dev, x.reshape(rows, dim)), upload(dev, w)
    ot = eb.Tensor.empty(dev, (rows, dim))
    rec = eb.Recorder(dev)
    eb.rmsnorm(rec, xt, wt, ot, rows, dim, eps)
    rec.submit()
    want = oracle.rmsnorm(x, w, rows, dim, eps)
    assert oracle.rel_l2(ot.to_f32(), want) < 1e-6


def test_rmsnorm_gemma_heads(dev):
    rows, dim = 4096 * 8, 256
    x = oracle.randn((rows, dim), 3)
    w = (1 + 0.1 * oracle.randn((dim,), 4)).astype(np.float32)
    xt, wt = upload(dev, x), upload(dev, w)
    ot = eb.Tensor.empty(dev, (rows, dim))
    rec = eb.Recorder(dev)
    eb.rmsnorm(rec, xt, wt, ot, rows, dim, 1e-6)
    rec.submit()
    assert oracle.rel_l2(ot.to_f32(), oracle.rmsnorm(x, w, rows, dim, 1e-6)) < 1e-6


def test_rope_tables_match_oracle_bitwise(dev):
    """Rope::build / build_partial tables (nn/src/rope.rs:24-50), both f64 then f32."""
    for ms, hd, theta, ra in [(8, 4, 1e4, None), (5, 8, 1e4, 2), (300, 256, 1e6, 32)]:
        r = eb.Rope.build(dev, ms, hd, theta) if ra is None else \
            eb.Rope.build_partial(dev, ms, hd, ra, theta)
        c, s = oracle.rope_tables(ms, hd, theta, rope_angles=ra)
        assert_bitwise(r.cos.to_f32(), c, "cos table")
        assert_bitwise(r.sin.to_f32(), s, "sin table")


@pytest.mark.parametrize("seq,nh,hd,theta,ra,base", [
    (4, 2, 8, 1e4, None, 0),          # rope.rs:92-111 reference case
    (1, 16, 128, 1e6, None, 777),     # a decode row at base_pos
    (300, 8, 256, 1e6, 32, 0),        # Gemma partial rotary
])
def test_rope_kernel(dev, seq, nh, hd, theta, ra, base):
    note(f"rope seq={seq} nh={nh} hd={hd}")
    ms = seq + base
    if (seq, nh, hd) == (4, 2, 8):
        x = np.arange(seq * nh * hd, dtype=np.float32) * np.float32(0.03) - np.float32(0.5)
    else:
        x = oracle.randn((seq * nh * hd,), 9)
    r = eb.Rope.build(dev, ms, hd, theta) if ra is None else eb.Rope.build_partial(dev, ms, hd, ra, theta)
    xt = upload(dev, x.reshape(seq, nh, hd))
    rec = eb.Recorder(dev)
    out = r.apply(rec, xt, seq, nh, base)
    rec.submit()
    c, s = oracle.rope_tables(ms, hd, theta, rope_angles=ra)
    want = oracle.rope(x, c, s, seq, nh, hd, base)
    got = out.to_f32()
    # the kernel rotates without fused multiply-adds, as the reference's f32 code does
    assert_bitwise(got, want, "rope vs the oracle")
    if ra is not None:  # pass-through pairs are exact
        g3, x3 = got.reshape(seq, nh, hd), x.reshape(seq, nh, hd)
        np.testing.assert_array_equal(g3[..., ra:hd // 2], x3[..., ra:hd // 2])
        np.testing.assert_array_equal(g3[..., hd // 2 + ra:], x3[..., hd // 2 + ra:])


@pytest.mark.parametrize("rows,H,Hkv,hd,base,norm,ra,dtype", [
    (37, 16, 8, 128, 0, True, None, "f32"),   # Qwen prompt with QK-norm
    (19, 16, 8, 256, 5, True, 32, "f32"),     # Gemma-4: partial rotary, continuation rows
    (33, 4, 2, 96, 0, False, None, "f32"),    # head_dim 96 (12 lanes of a 16-lane group)
    (9, 6, 3, 6, 2, True, None, "f32"),       # head_dim 6: the wave-per-row kernel
    (21, 8, 4, 128, 3, False, None, "f16"),   # IEEE-half caches
    (21, 8, 4, 64, 0, True, 16, "f16"),
])
def test_attention_prologue(dev, rows, H, Hkv, hd, base, norm, ra, dtype):
    """eb_launch_attn_prologue (attention.rs:62-97 in one launch) against the oracle chain
    rmsnorm -> rope -> kv_write. Without a norm every output is bit-exact (RoPE without
    fused multiply-adds, V copied); with one, the sum of squares is taken in another order
    (rel-L2 <= 1e-6). Cache rows outside [base, base + rows) keep their bits."""
    note(f"attention prologue rows={rows} H={H} Hkv={Hkv} hd={hd} base={base} {dtype}")
    max_seq = base + rows + 3
    eps = 1e-6
    q = oracle.randn((rows, H, hd), 31)
    k = oracle.randn((rows, Hkv, hd), 32)
    v = oracle.randn((rows, Hkv, hd), 33)
    gq = (1 + 0.1 * oracle.randn((hd,), 34)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 35)).astype(np.float32)
    ones = np.ones(hd, np.float32)
    c, s = oracle.rope_tables(max_seq, hd, 1e6, rope_angles=ra)
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    gqt, gkt, gvt = upload(dev, gq), upload(dev, gk), upload(dev, ones)
    ct, st = upload(dev, c), upload(dev, s)
    qo = eb.Tensor.empty(dev, (rows, H, hd))
    fill_k = oracle.randn((max_seq, Hkv, hd), 36)
    fill_v = oracle.randn((max_seq, Hkv, hd), 37)
    if dtype == "f16":
        kc = eb.Tensor.empty(dev, fill_k.shape, eb.DType.F16)
        vc = eb.Tensor.empty(dev, fill_v.shape, eb.DType.F16)
        rec = eb.Recorder(dev)
        eb.kv_write(rec, kc, upload(dev, fill_k), Hkv, max_seq, hd, max_seq, 0)
        eb.kv_write(rec, vc, upload(dev, fill_v), Hkv, max_seq, hd, max_seq, 0)
        rec.submit()
    else:
        kc, vc = upload(dev, fill_k), upload(dev, fill_v)
    eb.launch_attn_prologue(
        dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr, vt.numel(),
        rows, H, Hkv, hd, gqt.data_ptr if norm else 0, gkt.data_ptr if norm else 0,
        gvt.data_ptr if norm else 0, eps, ct.data_ptr, st.data_ptr, ct.numel(), base,
        qo.data_ptr, qo.numel(), kc.data_ptr, kc.numel(), vc.data_ptr, vc.numel(), max_seq,
        eb.DType.F16 if dtype == "f16" else eb.DType.F32)
    dev.synchronize()
    qn = oracle.rmsnorm(q, gq, rows * H, hd, eps) if norm else q.ravel()
    kn = oracle.rmsnorm(k, gk, rows * Hkv, hd, eps) if norm else k.ravel()
    vn = oracle.rmsnorm(v, ones, rows * Hkv, hd, eps) if norm else v.ravel()
    qr = oracle.rope(qn, c, s, rows, H, hd, base)
    kr = oracle.rope(kn, c, s, rows, Hkv, hd, base)
    want_k = oracle.kv_write(fill_k, kr, Hkv, rows, hd, base).reshape(max_seq, -1)
    want_v = oracle.kv_write(fill_v, vn, Hkv, rows, hd, base).reshape(max_seq, -1)
    got_q = qo.to_f32()
    if dtype == "f16":
        got_k = np.frombuffer(kc.read_bytes(), np.uint16).reshape(max_seq, -1)
        got_v = np.frombuffer(vc.read_bytes(), np.uint16).reshape(max_seq, -1)
        wk, wv = oracle.f16_bits(want_k).reshape(max_seq, -1), oracle.f16_bits(want_v).reshape(max_seq, -1)
    else:
        got_k = kc.to_f32().reshape(max_seq, -1)
        got_v = vc.to_f32().reshape(max_seq, -1)
        wk, wv = want_k, want_v
    outside = np.r_[0:base, base + rows:max_seq]
    np.testing.assert_array_equal(got_k[outside], wk[outside])
    np.testing.assert_array_equal(got_v[outside], wv[outside])
    new = slice(base, base + rows)
    if not norm:
        assert_bitwise(got_q, qr, "q_out")
        np.testing.assert_array_equal(got_k[new], wk[new])
        np.testing.assert_array_equal(got_v[new], wv[new])
        return
    assert rel_l2_f64(got_q, qr) < 1e-6
    if dtype == "f16":  # halves of nearly equal f32 values: at most one unit apart
        for g, w in ((got_k[new], wk[new]), (got_v[new], wv[new])):
            d = np.abs(g.astype(np.int32) - w.astype(np.int32))
            assert d.max() <= 1 and (d == 0).mean() > 0.95
    else:
        assert rel_l2_f64(got_k[new], wk[new]) < 1e-6
        assert rel_l2_f64(got_v[new], wv[new]) < 1e-6


def test_attention_prologue_refusals(dev):
    """Shapes the prologue refuses before any launch: rows past max_seq, one table only,
    tables too short, odd head_dim."""
    H, Hkv, hd, rows, max_seq = 4, 2, 8, 3, 8
    q = eb.Tensor.empty(dev, (rows, H, hd))
    k = eb.Tensor.empty(dev, (rows, Hkv, hd))
    kc = eb.Tensor.empty(dev, (max_seq, Hkv, hd))
    ct = eb.Tensor.empty(dev, (max_seq, hd // 2))

    def call(base=0, cos=ct.data_ptr, sin=ct.data_ptr, tn=ct.numel(), hd_=hd):
        eb.launch_attn_prologue(dev.stream, q.data_ptr, q.numel(), k.data_ptr, k.numel(),
                                k.data_ptr, k.numel(), rows, H, Hkv, hd_, 0, 0, 0, 1e-6, cos, sin,
                                tn, base, q.data_ptr, q.numel(), kc.data_ptr, kc.numel(),
                                kc.data_ptr, kc.numel(), max_seq, eb.DType.F32)
    with pytest.raises(eb.ShapeMismatch):
        call(base=6)
    with pytest.raises(eb.EyebrowseError):
        call(sin=0)
    with pytest.raises(eb.ShapeMismatch):
        call(base=4, tn=5 * hd // 2)
    with pytest.raises(eb.ShapeMismatch):
        call(hd_=7)


# ---------------------------------------------------------------- Attention -------------

def _oracle_chain(q, k, v, H, Hkv, hd, rows, base, gq, gk, gv, eps, rope_t, kc, vc, max_seq,
                  scale):
    c, s = rope_t
    qn = oracle.rmsnorm(q, gq, rows * H, hd, eps) if gq is not None else q.ravel()
    kn = oracle.rmsnorm(k, gk, rows * Hkv, hd, eps) if gk is not None else k.ravel()
    vn = oracle.rmsnorm(v, gv, rows * Hkv, hd, eps) if gv is not None else v.ravel()
    qr = oracle.rope(qn, c, s, rows, H, hd, base)
    kr = oracle.rope(kn, c, s, rows, Hkv, hd, base)
    kc = oracle.kv_write(kc, kr, Hkv, rows, hd, base)
    vc = oracle.kv_write(vc, vn, Hkv, rows, hd, base)
    if base == 0 and rows > 1:
        o = oracle.attn_prefill(qr, kr, vn, H, Hkv, rows, hd, scale, threads=16)
    else:
        o = oracle.attn_decode(qr, kc, vc, H, Hkv, base, hd, max_seq, scale, threads=16)
    return o.reshape(rows, H * hd), kc, vc


def test_prefill_decode_consistency(dev):
    """nn/src/tests.rs:181-244 from the projected q/k/v: prefill over 3 rows, then 3 decode
    steps through a fresh cache; the last decode row equals prefill's last row (the
    reference accepts rel_l2 < 2e-3; here the f32 bar)."""
    note("attention prefill/decode consistency")
    H, Hkv, hd, seq, max_seq = 4, 2, 4, 3, 8
    x_q = oracle.prng(seq * H * hd, 21).reshape(seq, H * hd)
    x_k = oracle.prng(seq * Hkv * hd, 22).reshape(seq, Hkv * hd)
    x_v = oracle.prng(seq * Hkv * hd, 23).reshape(seq, Hkv * hd)
    qn = upload(dev, oracle.prng(hd, 15))
    kn = upload(dev, oracle.prng(hd, 16))
    attn = eb.Attention(H, Hkv, hd, float(oracle.default_scale(hd)), q_norm=qn, k_norm=kn)
    rope = eb.Rope.build(dev, max_seq, hd, 10000.0)
    kv_p = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    rec = eb.Recorder(dev)
    pre = attn.forward_qkv(rec, upload(dev, x_q), upload(dev, x_k), upload(dev, x_v), rope, kv_p,
                           0, seq, 0)
    rec.submit()
    pre_out = pre.to_f32().reshape(seq, H * hd)
    kv_d = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    last = None
    for pos in range(seq):
        rec = eb.Recorder(dev)
        out = attn.forward_qkv(rec, upload(dev, x_q[pos:pos + 1]), upload(dev, x_k[pos:pos + 1]),
                               upload(dev, x_v[pos:pos + 1]), rope, kv_d, 0, 1, pos)
        rec.submit()
        last = out.to_f32()
    assert rel_l2_f64(last, pre_out[seq - 1]) < 2e-5
    # both caches hold the same rows 0..seq-1 up to the norm's summation order (the decode
    # step folds RMSNorm and RoPE into its own kernel)
    n = seq * Hkv * hd
    assert rel_l2_f64(kv_d.k[0].to_f32()[:n], kv_p.k[0].to_f32()[:n]) < 1e-6
    assert_bitwise(kv_d.v[0].to_f32()[:n], kv_p.v[0].to_f32()[:n], "V rows (no norm here)")


def test_gemma_attention_forward(dev):
    """BASELINE config 5 through Attention.forward_qkv: per-head QK-RMSNorm with learned
    gains, weightless V-RMSNorm, partial RoPE (32 of 128 pairs, theta 1e6), scale 1.0,
    hd 256; prefill T=4096 (every row) then one decode step at pos 16383 of a max_seq
    16384 cache."""
    H, Hkv, hd, eps = 16, 8, 256, 1e-6
    T, max_seq = 4096, 16384
    note(f"gemma attention prefill T={T}")
    gq = (1 + 0.1 * oracle.randn((hd,), 4)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 5)).astype(np.float32)
    ones = np.ones(hd, np.float32)
    attn = eb.Attention(H, Hkv, hd, 1.0, q_norm=upload(dev, gq), k_norm=upload(dev, gk),
                        v_norm=upload(dev, ones), norm_eps=eps)
    rope = eb.Rope.build_partial(dev, max_seq, hd, 32, 1e6)
    rope_t = oracle.rope_tables(max_seq, hd, 1e6, rope_angles=32)
    q = oracle.randn((T, H * hd), 1)
    k = oracle.randn((T, Hkv * hd), 2)
    v = oracle.randn((T, Hkv * hd), 3)
    kv = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    rec = eb.Recorder(dev)
    out = attn.forward_qkv(rec, upload(dev, q), upload(dev, k), upload(dev, v), rope, kv, 0, T, 0)
    rec.submit()
    got = out.to_f32().reshape(T, H * hd)
    # oracle: norms + rope on the whole prompt, attention on row samples
    qr = oracle.rope(oracle.rmsnorm(q, gq, T * H, hd, eps), *rope_t, T, H, hd)
    kr = oracle.rope(oracle.rmsnorm(k, gk, T * Hkv, hd, eps), *rope_t, T, Hkv, hd)
    vn = oracle.rmsnorm(v, ones, T * Hkv, hd, eps)
    want = oracle.attn_prefill(qr, kr, vn, H, Hkv, T, hd, 1.0, threads=16).reshape(T, H * hd)
    # normalised head_dim-256 rows at scale 1.0: scores of sigma 16, so the f32 bar's max-abs
    # part doubles (2e-4; see test_gpu_prefill.test_baseline_prefill_configs)
    assert_close(got, want, abs_=2e-4, what="gemma prefill, all rows")
    for b0 in range(0, T, 64):
        assert_close(got[b0:b0 + 64], want[b0:b0 + 64], abs_=2e-4,
                     what=f"gemma prefill rows {b0}+64")
    # the cache holds the post-RoPE K and the normed V (attention.rs:78-97); RMSNorm and
    # RoPE round differently from the oracle (reduction order, FMA), so not bitwise
    kc_all = kv.k[0].to_f32()
    assert rel_l2_f64(kc_all[: T * Hkv * hd], kr) < 1e-6
    assert rel_l2_f64(kv.v[0].to_f32()[: T * Hkv * hd], vn) < 1e-6

    # decode at pos 16383 over a filled cache
    note("gemma attention decode pos=16383")
    pos = max_seq - 1
    kfill = oracle.randn((max_seq, Hkv, hd), 6)
    vfill = oracle.randn((max_seq, Hkv, hd), 7)
    kv2 = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, kv2.k[0], upload(dev, kfill), Hkv, max_seq, hd, max_seq, 0)
    eb.kv_write(rec, kv2.v[0], upload(dev, vfill), Hkv, max_seq, hd, max_seq, 0)
    rec.submit()
    q1, k1, v1 = oracle.randn((1, H * hd), 8), oracle.randn((1, Hkv * hd), 9), oracle.randn((1, Hkv * hd), 10)
    rec = eb.Recorder(dev)
    o1 = attn.forward_qkv(rec, upload(dev, q1), upload(dev, k1), upload(dev, v1), rope, kv2, 0, 1, pos)
    rec.submit()
    want1, kc_w, _ = _oracle_chain(q1, k1, v1, H, Hkv, hd, 1, pos, gq, gk, ones, eps, rope_t,
                                   kfill, vfill, max_seq, 1.0)
    assert_close(o1.to_f32().reshape(1, H * hd), want1, what="gemma decode")
    kc_got = kv2.k[0].to_f32().reshape(max_seq, Hkv * hd)
    kc_want = kc_w.reshape(max_seq, Hkv * hd)
    assert_bitwise(kc_got[:pos], kc_want[:pos], "untouched cache rows")
    assert rel_l2_f64(kc_got[pos], kc_want[pos]) < 1e-6


def test_gemma_t32_golden_through_attention(dev):
    """The committed Gemma-4 fixture (tests/golden/gemma_t32_prefill.npz: T=32, hd 256,
    q/k/v norms, partial RoPE, scale 1.0; its inputs and intermediate SHA-256 sums are pinned
    in tests/test_golden.py) through Attention.forward_qkv on the GPU: the fused
    pre-attention pass, then prefill over the cache rows it wrote."""
    g = np.load("tests/golden/gemma_t32_prefill.npz", allow_pickle=False)
    T, H, Hkv, hd = int(g["T"]), int(g["H"]), int(g["Hkv"]), int(g["hd"])
    eps = float(g["eps"])
    note(f"gemma golden T={T} through Attention")
    q = oracle.randn((T, H, hd), 1)
    k = oracle.randn((T, Hkv, hd), 2)
    v = oracle.randn((T, Hkv, hd), 3)
    gq = (1 + 0.1 * oracle.randn((hd,), 4)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 5)).astype(np.float32)
    attn = eb.Attention(H, Hkv, hd, 1.0, q_norm=upload(dev, gq), k_norm=upload(dev, gk),
                        v_norm=upload(dev, np.ones(hd, np.float32)), norm_eps=eps)
    rope = eb.Rope.build_partial(dev, T, hd, int(g["rope_angles"]), float(g["theta"]))
    kv = eb.KvCache.new(dev, 1, T, Hkv, hd)
    rec = eb.Recorder(dev)
    out = attn.forward_qkv(rec, upload(dev, q.reshape(T, -1)), upload(dev, k.reshape(T, -1)),
                           upload(dev, v.reshape(T, -1)), rope, kv, 0, T, 0)
    rec.submit()
    assert_close(out.to_f32().reshape(T, H, hd), g["o"], what="gemma T=32 golden")


def test_forward_routing_and_errors(dev):
    H, Hkv, hd = 4, 2, 8
    attn = eb.Attention(H, Hkv, hd, 0.3)
    rope = eb.Rope.build(dev, 16, hd, 1e4)
    kv = eb.KvCache.new(dev, 1, 16, Hkv, hd)
    q = upload(dev, oracle.randn((2, H * hd), 1))
    k = upload(dev, oracle.randn((2, Hkv * hd), 2))
    rec = eb.Recorder(dev)
    with pytest.raises(eb.ShapeMismatch):           # rows [15, 17) past max_seq 16
        attn.forward_qkv(rec, q, k, k, rope, kv, 0, 2, 15)
    with pytest.raises(eb.ShapeMismatch):           # layer out of range
        attn.forward_qkv(rec, q, k, k, rope, kv, 1, 2, 0)
    rec.submit()
    with pytest.raises(eb.UnsupportedConfig):
        eb.Attention(H, Hkv, 6, 0.3)


# ---------------------------------------------------------------- with projections ------

def _proj(dev, out_f, in_f, seed, scale=0.03):
    w = oracle.randn((out_f, in_f), seed) * np.float32(scale)
    return w, eb.Tensor.from_f16_packed(dev, w.shape, w)


@pytest.mark.parametrize("cfg", ["qwen", "gemma"])
def test_attention_forward_with_projections(dev, cfg):
    """Attention.forward whole (attention.rs:30-45): q/k/v projections, norms, RoPE,
    kv_write, attention, o_proj; a prompt, a continuation chunk and two decode steps,
    each against the oracle chain (linear_f16w, rmsnorm, rope, attention over the cache
    contents the oracle builds itself)."""
    if cfg == "qwen":   # Qwen3-0.6B widths: QK-norm, full RoPE theta 1e6, scale 1/sqrt(hd)
        H, Hkv, hd, hidden, ra, theta = 16, 8, 128, 1024, None, 1e6
        sc = float(oracle.default_scale(hd))
        vgain = None
    else:               # Gemma-4-shaped: QK-norm + weightless V-norm, partial RoPE, scale 1
        H, Hkv, hd, hidden, ra, theta = 8, 4, 256, 640, 32, 1e6
        sc = 1.0
        vgain = np.ones(hd, np.float32)
    eps, max_seq = 1e-6, 512
    note(f"attention forward with projections {cfg}")
    gq = (1 + 0.1 * oracle.randn((hd,), 4)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 5)).astype(np.float32)
    wq, tq = _proj(dev, H * hd, hidden, 11)
    wk, tk = _proj(dev, Hkv * hd, hidden, 12)
    wv, tv = _proj(dev, Hkv * hd, hidden, 13)
    wo, to = _proj(dev, hidden, H * hd, 14)
    attn = eb.Attention(H, Hkv, hd, sc, q_norm=upload(dev, gq), k_norm=upload(dev, gk),
                        v_norm=upload(dev, vgain) if vgain is not None else None, norm_eps=eps,
                        q_proj=tq, k_proj=tk, v_proj=tv, o_proj=to, hidden=hidden)
    if ra is None:
        rope = eb.Rope.build(dev, max_seq, hd, theta)
        cos, sin = oracle.rope_tables(max_seq, hd, theta)
    else:
        rope = eb.Rope.build_partial(dev, max_seq, hd, ra, theta)
        cos, sin = oracle.rope_tables(max_seq, hd, theta, rope_angles=ra)
    kv = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    kc = np.zeros((max_seq, Hkv, hd), np.float32)
    vc = np.zeros((max_seq, Hkv, hd), np.float32)
    bits = {n: oracle.f16_bits(w) for n, w in (("q", wq), ("k", wk), ("v", wv), ("o", wo))}
    for a, b in ((0, 40), (40, 60), (60, 61), (61, 62)):
        rows = b - a
        x = oracle.randn((rows, hidden), 100 + a)
        rec = eb.Recorder(dev)
        y = attn.forward(rec, upload(dev, x), rope, kv, 0, rows, a)
        rec.submit()
        q = oracle.linear_f16w(x, bits["q"], rows, hidden, H * hd, threads=16)
        k = oracle.linear_f16w(x, bits["k"], rows, hidden, Hkv * hd, threads=16)
        v = oracle.linear_f16w(x, bits["v"], rows, hidden, Hkv * hd, threads=16)
        qn = oracle.rmsnorm(q, gq, rows * H, hd, eps)
        kn = oracle.rmsnorm(k, gk, rows * Hkv, hd, eps)
        vn = oracle.rmsnorm(v, vgain, rows * Hkv, hd, eps) if vgain is not None else v
        qr = oracle.rope(qn, cos, sin, rows, H, hd, a)
        kr = oracle.rope(kn, cos, sin, rows, Hkv, hd, a)
        kc[a:b] = kr.reshape(rows, Hkv, hd)
        vc[a:b] = np.asarray(vn).reshape(rows, Hkv, hd)
        o = oracle.attn_chunk(qr.reshape(rows, H, hd), kc, vc, H, Hkv, a, rows, hd, sc,
                              threads=16)
        want = oracle.linear_f16w(o.reshape(rows, H * hd), bits["o"], rows, H * hd, hidden,
                                  threads=16)
        assert_close(y.to_f32().reshape(rows, hidden), want, what=f"{cfg} rows {a}..{b}")


def test_attention_projection_validation(dev):
    note("attention projection validation")
    H, Hkv, hd, hidden = 4, 2, 64, 128
    _, tq = _proj(dev, H * hd, hidden, 1)
    _, tk = _proj(dev, Hkv * hd, hidden, 2)
    _, to = _proj(dev, hidden, H * hd, 3)
    with pytest.raises(eb.ShapeMismatch):  # three of four
        eb.Attention(H, Hkv, hd, 0.1, q_proj=tq, k_proj=tk, v_proj=tk, hidden=hidden)
    with pytest.raises(eb.ShapeMismatch):  # wrong shape (k_proj as q_proj)
        eb.Attention(H, Hkv, hd, 0.1, q_proj=tk, k_proj=tk, v_proj=tk, o_proj=to, hidden=hidden)
    bare = eb.Attention(H, Hkv, hd, 0.1)
    rope = eb.Rope.build(dev, 16, hd, 1e4)
    kv = eb.KvCache.new(dev, 1, 16, Hkv, hd)
    rec = eb.Recorder(dev)
    with pytest.raises(eb.ShapeMismatch):  # no projections: forward_qkv only
        bare.forward(rec, upload(dev, np.zeros((1, hidden), np.float32)), rope, kv, 0, 1, 0)
    rec.submit()
