"""Head dims beyond the powers of two: every multiple of 8 up to 128 and every multiple of
16 up to 256 (the reference builds a pipeline per head_dim,
crates/eyebrowse-kernels/src/attention.rs:113-114, and its config defaults head_dim to
hidden / n_heads, crates/eyebrowse-load/src/config.rs:63).

Decode runs an instantiation per head dim, with each row's lane group padded to a power of
two (the extra lanes hold zeros; odd multiples of 8 run 8 dims per lane); prefill runs the
next power-of-two instantiation with the extra dims read as zeros and never stored. Every
case is held to the oracle at the f32 bar (tests/_gpu.py), on f32, IEEE-half and E4M3
caches (the narrow ones against the oracle on the rounded values), plain and through the
fused steps.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, prefill, upload
from tests._textbook import rel_l2_f64

pytestmark = pytest.mark.gpu

ODD_DIMS = [48, 80, 96, 112, 144, 160, 192, 208, 240]
# Odd multiples of 8 (a half 16-dim step at the end of the row).
EIGHT_DIMS = [24, 40, 56, 72, 88, 104, 120]


@pytest.mark.parametrize("hd", ODD_DIMS + EIGHT_DIMS)
@pytest.mark.parametrize("h,hkv", [(8, 2), (6, 3), (3, 3)])  # 4, 2 and 1 heads per KV head
def test_decode_step(dev, hd, h, hkv):
    """The fused decode step (new row written at pos, attention over pos + 1 keys) at a
    position with key splits and at one without."""
    for pos, max_seq in ((1500, 1600), (5, 8)):
        note(f"decode hd={hd} h={h} hkv={hkv} pos={pos}")
        sc = float(oracle.default_scale(hd))
        q = oracle.randn((h, hd), 1)
        kc = oracle.randn((max_seq, hkv, hd), 2)
        vc = oracle.randn((max_seq, hkv, hd), 3)
        kn = oracle.randn((1, hkv, hd), 4)
        vn = oracle.randn((1, hkv, hd), 5)
        qt, kt, vt, knt, vnt = (upload(dev, a) for a in (q, kc, vc, kn, vn))
        ot = eb.Tensor.empty(dev, (h, hd))
        rec = eb.Recorder(dev)
        eb.attn_decode_step(rec, qt, knt, vnt, kt, vt, ot, h, hkv, pos, hd, max_seq, sc)
        rec.submit()
        kc2 = oracle.kv_write(kc, kn, hkv, 1, hd, pos)
        vc2 = oracle.kv_write(vc, vn, hkv, 1, hd, pos)
        assert_bitwise(kt.to_f32(), kc2, "K cache after the step")
        assert_bitwise(vt.to_f32(), vc2, "V cache after the step")
        want = oracle.attn_decode(q, kc2, vc2, h, hkv, pos, hd, max_seq, sc, threads=8)
        assert_close(ot.to_f32().reshape(h, hd), want.reshape(h, hd), what=f"decode hd={hd}")


def _rounded(a, dtype):
    """The values a cache of `dtype` holds for the f32 rows a (oracle's rounding)."""
    if dtype == "f16":
        return oracle.f16_values(oracle.f16_bits(a)).reshape(a.shape)
    if dtype == "e4m3":
        return oracle.f8_values(oracle.f8_bits(a)).reshape(a.shape)
    return a


DTYPES = {"f32": eb.DType.F32, "f16": eb.DType.F16, "e4m3": eb.DType.F8E4M3}


def _stored(t, dtype):
    """A cache tensor's contents as f32 values (narrow formats decoded by the oracle)."""
    if dtype == "f16":
        return oracle.f16_values(np.frombuffer(t.read_bytes(), np.uint16).copy())
    if dtype == "e4m3":
        return oracle.f8_values(np.frombuffer(t.read_bytes(), np.uint8).copy())
    return t.to_f32()


def _cache(dev, rows, dtype):
    t = eb.Tensor.empty(dev, rows.shape, DTYPES[dtype])
    rec = eb.Recorder(dev)
    eb.kv_write(rec, t, upload(dev, rows), rows.shape[1], rows.shape[0], rows.shape[2],
                rows.shape[0], 0)
    rec.submit()
    return t


@pytest.mark.parametrize("hd,dtype", [(48, "f16"), (80, "f16"), (192, "f16"), (40, "f16"),
                                      (120, "f16"), (24, "e4m3"), (72, "e4m3"), (104, "e4m3")])
def test_decode_narrow_cache(dev, hd, dtype):
    h, hkv, pos, max_seq = 8, 2, 2000, 2048
    note(f"decode {dtype} hd={hd}")
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((h, hd), 11)
    kc = oracle.randn((max_seq, hkv, hd), 12)
    vc = oracle.randn((max_seq, hkv, hd), 13)
    kt, vt = _cache(dev, kc, dtype), _cache(dev, vc, dtype)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode(rec, upload(dev, q), kt, vt, ot, h, hkv, pos, hd, max_seq, sc)
    rec.submit()
    want = oracle.attn_decode(q, _rounded(kc, dtype), _rounded(vc, dtype), h, hkv, pos, hd,
                              max_seq, sc, threads=8)
    assert_close(ot.to_f32().reshape(h, hd), want.reshape(h, hd),
                 what=f"{dtype} decode hd={hd}")


@pytest.mark.parametrize("hd", ODD_DIMS + EIGHT_DIMS + [16])
@pytest.mark.parametrize("h,hkv,T", [(8, 2, 150), (6, 3, 1100), (4, 4, 67)])
def test_prefill(dev, hd, h, hkv, T):
    """Recorder prefill (pre-split pass and key chunks where the shape takes them)."""
    note(f"prefill hd={hd} h={h} hkv={hkv} T={T}")
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((T, h, hd), 21)
    k = oracle.randn((T, hkv, hd), 22)
    v = oracle.randn((T, hkv, hd), 23)
    got = prefill(dev, q, k, v, h, hkv, T, hd, sc)
    want = oracle.attn_prefill(q, k, v, h, hkv, T, hd, sc, threads=16)
    assert_close(got, want, what=f"prefill hd={hd}")


@pytest.mark.parametrize("hd", [80, 96, 192, 72])
def test_raw_prefill_launches(dev, hd):
    """The plain raw launch (split while staging) and the _ws launch (pre-split) give the
    same bits at a padded head dim, and match the oracle (512 query-block workgroups, more
    than the workgroup slots, so the _ws launch cuts no key chunks, which would sum in
    another order)."""
    h, hkv, T = 16, 8, 4096
    note(f"raw prefill hd={hd}")
    sc = float(oracle.default_scale(hd))
    q, k, v = (oracle.randn(s, 30 + i) for i, s in enumerate(((T, h, hd), (T, hkv, hd), (T, hkv, hd))))
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    o1 = eb.Tensor.empty(dev, (T, h, hd))
    o2 = eb.Tensor.empty(dev, (T, h, hd))
    eb.launch_attn_prefill(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                           vt.data_ptr, vt.numel(), o1.data_ptr, o1.numel(), h, hkv, T, hd, sc)
    need = eb.attn_prefill_workspace_floats(h, hkv, hd, 0, T)
    assert need > 0
    ws = eb.Tensor.empty(dev, (need,))
    eb.launch_attn_prefill_ws(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                              vt.data_ptr, vt.numel(), o2.data_ptr, o2.numel(), h, hkv, T, hd, sc,
                              ws.data_ptr, need)
    dev.synchronize()
    assert_bitwise(o2.to_f32(), o1.to_f32(), "pre-split vs split while staging")
    want = oracle.attn_prefill(q, k, v, h, hkv, T, hd, sc, threads=16)
    assert_close(o1.to_f32().reshape(T, h, hd), want, what=f"raw prefill hd={hd}")


@pytest.mark.parametrize("hd,dtype", [(80, "f32"), (112, "f16"), (192, "f32"), (40, "f32"),
                                      (120, "f16"), (56, "e4m3")])
def test_chunked_prefill_over_cache(dev, hd, dtype):
    h, hkv, pos0, rows, max_seq = 8, 2, 700, 130, 900
    note(f"chunk hd={hd} {dtype}")
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 41)
    kc = oracle.randn((max_seq, hkv, hd), 42)
    vc = oracle.randn((max_seq, hkv, hd), 43)
    kt, vt = _cache(dev, kc, dtype), _cache(dev, vc, dtype)
    kc, vc = _rounded(kc, dtype), _rounded(vc, dtype)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, upload(dev, q), kt, vt, ot, h, hkv, pos0, rows, hd, max_seq, sc, 0)
    rec.submit()
    want = oracle.attn_chunk(q, kc, vc, h, hkv, pos0, rows, hd, sc, 0, threads=16)
    assert_close(ot.to_f32().reshape(rows, h, hd), want.reshape(rows, h, hd),
                 what=f"chunk hd={hd} {dtype}")


@pytest.mark.parametrize("hd,dtype", [(80, "f32"), (160, "f32"), (40, "f32"), (120, "f32"),
                                      (40, "f16"), (72, "e4m3"), (48, "f16")])
def test_attention_forward_prompt_then_decode(dev, hd, dtype):
    """Attention.forward_qkv with QK-norm, V-norm and RoPE at a padded head dim: a prompt
    (fused pre-attention pass + prefill over the cache rows it wrote), then a decode step
    (norms and RoPE inside the fused decode kernel; over a narrow cache at an odd multiple
    of 8, the pre-attention pass then attn_decode), against the oracle chain on the values
    the cache holds."""
    H, Hkv, T, max_seq, eps = 8, 2, 96, 128, 1e-6
    note(f"attention hd={hd} {dtype}")
    gq = (1 + 0.1 * oracle.randn((hd,), 51)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 52)).astype(np.float32)
    ones = np.ones(hd, np.float32)
    sc = float(oracle.default_scale(hd))
    attn = eb.Attention(H, Hkv, hd, sc, q_norm=upload(dev, gq), k_norm=upload(dev, gk),
                        v_norm=upload(dev, ones), norm_eps=eps)
    rope = eb.Rope.build(dev, max_seq, hd, 1e4)
    c, s = oracle.rope_tables(max_seq, hd, 1e4)
    kv = eb.KvCache.new(dev, 1, max_seq, Hkv, hd, DTYPES[dtype])
    q = oracle.randn((T + 1, H * hd), 53)
    k = oracle.randn((T + 1, Hkv * hd), 54)
    v = oracle.randn((T + 1, Hkv * hd), 55)
    rec = eb.Recorder(dev)
    out = attn.forward_qkv(rec, upload(dev, q[:T]), upload(dev, k[:T]), upload(dev, v[:T]), rope,
                           kv, 0, T, 0)
    rec.submit()
    qr = oracle.rope(oracle.rmsnorm(q, gq, (T + 1) * H, hd, eps), c, s, T + 1, H, hd)
    kr = oracle.rope(oracle.rmsnorm(k, gk, (T + 1) * Hkv, hd, eps), c, s, T + 1, Hkv, hd)
    vn = oracle.rmsnorm(v, ones, (T + 1) * Hkv, hd, eps)
    n = T * Hkv * hd
    # The rows the cache holds: f32 as computed; narrow caches their rounding of the
    # normed, rotated rows (an ulp of difference before the rounding can move an element by
    # one step, so attention is checked on the stored values, and those against the
    # oracle's rows within the format's step).
    step = {"f32": 1e-6, "f16": 2.0 ** -11, "e4m3": 2.0 ** -4}[dtype]
    kst, vst = _stored(kv.k[0], dtype)[:n], _stored(kv.v[0], dtype)[:n]
    assert rel_l2_f64(kst, kr[:n]) < step and rel_l2_f64(vst, vn[:n]) < step
    want = oracle.attn_prefill(qr[: T * H * hd], kst, vst, H, Hkv, T, hd, sc, threads=16)
    assert_close(out.to_f32().reshape(T, H, hd), want, what=f"prompt hd={hd}")
    rec = eb.Recorder(dev)
    o1 = attn.forward_qkv(rec, upload(dev, q[T:]), upload(dev, k[T:]), upload(dev, v[T:]), rope,
                          kv, 0, 1, T)
    rec.submit()
    n1 = (T + 1) * Hkv * hd
    kst, vst = _stored(kv.k[0], dtype)[:n1], _stored(kv.v[0], dtype)[:n1]
    assert rel_l2_f64(kst, kr[:n1]) < step and rel_l2_f64(vst, vn[:n1]) < step
    kc = np.zeros((max_seq, Hkv, hd), np.float32)
    vc = np.zeros((max_seq, Hkv, hd), np.float32)
    kc[: T + 1] = kst.reshape(T + 1, Hkv, hd)
    vc[: T + 1] = vst.reshape(T + 1, Hkv, hd)
    want1 = oracle.attn_decode(qr[T * H * hd:], kc, vc, H, Hkv, T, hd, max_seq, sc)
    assert_close(o1.to_f32().reshape(H, hd), want1.reshape(H, hd), what=f"decode hd={hd}")


def test_unsupported_head_dims_are_refused(dev):
    """Head dims that are neither 4, a multiple of 8 up to 128 nor a multiple of 16 up to
    256 are refused before any launch."""
    for hd in (12, 20, 136, 248, 272):
        with pytest.raises(eb.UnsupportedConfig):
            eb.Attention(4, 2, hd, 0.1)
