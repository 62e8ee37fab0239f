"""IEEE-half (f16) KV caches on the GPU against the oracle.

The reference's caches are f32 (crates/eyebrowse-nn/src/kv_cache.rs:37,41); an f16 cache
has no counterpart there. Its contract: kv_write stores binary16 rounded to nearest even
(bit-exact against oracle.f16_bits, pinned in tests/test_oracle.py), and attention over
the cache computes in f32 on the rounded values. So every attention output is checked
twice:
- against the oracle on the rounded caches, at the FP32 bar (tests/_gpu.py): the f16
  kernels must be the f32 kernels on different loads;
- against the oracle on the unrounded f32 rows, at the north-star bar (rel-L2 1e-3,
  max-abs 2e-3): what storing the cache in half precision costs.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import (NORTH_MAX_ABS, NORTH_REL_L2, assert_bitwise, assert_close, note,
                        upload)

pytestmark = pytest.mark.gpu


def f16_cache(dev, rows):
    """An f16 cache tensor [max_seq, hkv, hd] holding f16_bits(rows), written by kv_write."""
    rows = np.ascontiguousarray(rows, np.float32)
    max_seq, hkv, hd = rows.shape
    t = eb.Tensor.empty(dev, rows.shape, eb.DType.F16)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, t, upload(dev, rows), hkv, max_seq, hd, max_seq, 0)
    rec.submit()
    return t


def bits_of(t):
    return np.frombuffer(t.read_bytes(), np.uint16).copy()


def rounded(a):
    return oracle.f16_values(oracle.f16_bits(a)).reshape(np.shape(a))


def check_both(got, q, kc, vc, h, hkv, pos0, rows, hd, sc, window, what):
    """got against the oracle on the rounded caches (FP32 bar) and on the f32 caches
    (north-star bar)."""
    want16 = oracle.attn_chunk(q, rounded(kc), rounded(vc), h, hkv, pos0, rows, hd, sc, window,
                               threads=16)
    assert_close(got, want16, what=f"{what} vs rounded-cache oracle")
    want32 = oracle.attn_chunk(q, kc, vc, h, hkv, pos0, rows, hd, sc, window, threads=16)
    assert_close(got, want32, rel=NORTH_REL_L2, abs_=NORTH_MAX_ABS, what=f"{what} vs f32 oracle")


def test_kv_write_f16_bitwise_with_specials(dev):
    """Rows of ordinary values, ties, overflow, subnormals, signed zero, inf and NaN, written
    at an offset; the untouched rows keep their bits."""
    hkv, hd, max_seq, start, count = 2, 8, 12, 5, 4
    note("kv_write f16 specials")
    base = oracle.randn((max_seq, hkv, hd), 1)
    t = f16_cache(dev, base)
    assert_bitwise(bits_of(t).view(np.float16).astype(np.float32),
                   oracle.f16_values(oracle.f16_bits(base)), "initial rows")
    src = oracle.randn((count, hkv, hd), 2).ravel() * 100.0
    specials = [1 + 2 ** -11, 1 + 3 * 2 ** -11, 65504.0, 65519.0, 65520.0, 1e6, -1e6, -0.0,
                2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 3e-6, -7e-7, np.inf, -np.inf, np.nan, 0.1,
                -65535.0]
    src[:len(specials)] = np.array(specials, np.float32)
    src = src.reshape(count, hkv, hd).astype(np.float32)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, t, upload(dev, src), hkv, count, hd, max_seq, start)
    rec.submit()
    got = bits_of(t)
    want = oracle.kv_write_f16(oracle.f16_bits(base), src, hkv, count, hd, start)
    nan_g = (got & 0x7C00) == 0x7C00
    nan_g &= (got & 0x3FF) != 0
    nan_w = ((want & 0x7C00) == 0x7C00) & ((want & 0x3FF) != 0)
    assert np.array_equal(nan_g, nan_w), "NaN positions differ"
    bad = np.count_nonzero(got[~nan_w] != want[~nan_w])
    assert bad == 0, f"{bad} halves differ"


def test_kv_write_f16_prompt_sized_bitwise(dev):
    """A Qwen3 prompt's K rows (4096 x 8 x 128) at row 100 of an 8192-row cache."""
    hkv, hd, max_seq, start, count = 8, 128, 8192, 100, 4096
    note("kv_write f16 qwen prompt")
    src = oracle.randn((count, hkv, hd), 3) * 4.0
    t = eb.Tensor.empty(dev, (max_seq, hkv, hd), eb.DType.F16)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, t, upload(dev, src), hkv, count, hd, max_seq, start)
    rec.submit()
    got = bits_of(t)[start * hkv * hd:(start + count) * hkv * hd]
    assert np.array_equal(got, oracle.f16_bits(src.ravel()))


@pytest.mark.parametrize("h,hkv,hd,pos,window", [
    (16, 8, 128, 8191, 0),    # Qwen3 decode at the bench's L
    (16, 8, 128, 0, 0),       # first token: output is the v row
    (16, 8, 128, 100, 0),     # one split
    (32, 8, 128, 3000, 0),    # GQA 4 (Mistral)
    (16, 8, 256, 5000, 0),    # hd 256 (Gemma)
    (24, 8, 128, 2049, 0),    # g = 3
    (32, 32, 128, 1500, 0),   # MHA
    (8, 2, 64, 777, 0),       # hd 64
    (4, 2, 8, 40, 0),         # smallest f16 head dim
    (16, 8, 128, 6000, 1024), # sliding window
    (4, 2, 8, 40, 1),         # window 1
])
def test_decode_f16_matches_oracle(dev, h, hkv, hd, pos, window):
    note(f"decode f16 h={h} hkv={hkv} hd={hd} pos={pos} window={window}")
    max_seq = pos + 3
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((h, hd), 1)
    kc, vc = oracle.randn((max_seq, hkv, hd), 2), oracle.randn((max_seq, hkv, hd), 3)
    kt, vt = f16_cache(dev, kc), f16_cache(dev, vc)
    qt = upload(dev, q)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode_window(rec, qt, kt, vt, ot, h, hkv, pos, hd, max_seq, sc, window)
    rec.submit()
    check_both(ot.to_f32().reshape(1, h, hd), q.reshape(1, h, hd), kc, vc, h, hkv, pos, 1, hd,
               sc, window, "decode f16")
    if window == 0:
        o2 = eb.Tensor.empty(dev, (h, hd))
        rec = eb.Recorder(dev)
        eb.attn_decode(rec, qt, kt, vt, o2, h, hkv, pos, hd, max_seq, sc)
        rec.submit()
        assert_bitwise(o2.to_f32(), ot.to_f32(), "attn_decode vs window 0")


@pytest.mark.parametrize("h,hkv,hd", [(32, 8, 128), (8, 2, 96), (8, 2, 256)])
def test_decode_f16_rising_scores(dev, h, hkv, hd):
    """Keys whose scale ramps up along the cache (x1 to x5), so that the scores' running max
    moves past the lazy reference many times in the middle of every split: the rescale
    branch (with its own copy of the update at 4 heads per workgroup) runs with factors
    other than 0 and 1. Against the oracle on the rounded caches (FP32 bar)."""
    pos = 4000
    note(f"decode f16 rising scores h={h} hkv={hkv} hd={hd} pos={pos}")
    max_seq = pos + 1
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((h, hd), 21) * np.float32(3.0)
    ramp = (1.0 + 4.0 * np.arange(max_seq, dtype=np.float32) / pos).astype(np.float32)
    kc = (oracle.randn((max_seq, hkv, hd), 22) * ramp[:, None, None]).astype(np.float32)
    vc = oracle.randn((max_seq, hkv, hd), 23)
    kt, vt = f16_cache(dev, kc), f16_cache(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode(rec, upload(dev, q), kt, vt, ot, h, hkv, pos, hd, max_seq, sc)
    rec.submit()
    want = oracle.attn_decode(q, rounded(kc), rounded(vc), h, hkv, pos, hd, max_seq, sc,
                              threads=16)
    assert_close(ot.to_f32().reshape(h, hd), want.reshape(h, hd),
                 what="f16 decode, rising scores, vs rounded-cache oracle")


@pytest.mark.parametrize("h,hkv,hd,pos,window", [
    (16, 8, 128, 8191, 0),
    (16, 8, 128, 0, 0),
    (32, 8, 128, 4097, 0),
    (16, 8, 256, 3001, 512),
    (4, 2, 8, 9, 0),
])
def test_decode_step_f16(dev, h, hkv, hd, pos, window):
    """The fused step: the new rows land in the cache as f16_bits, the output is attention
    over the cache as it then stands."""
    note(f"decode step f16 h={h} hd={hd} pos={pos} window={window}")
    max_seq = pos + 2
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((h, hd), 4)
    kc, vc = oracle.randn((max_seq, hkv, hd), 5), oracle.randn((max_seq, hkv, hd), 6)
    knew, vnew = oracle.randn((1, hkv, hd), 7), oracle.randn((1, hkv, hd), 8)
    kt, vt = f16_cache(dev, kc), f16_cache(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode_step_window(rec, upload(dev, q), upload(dev, knew), upload(dev, vnew), kt, vt,
                               ot, h, hkv, pos, hd, max_seq, sc, window)
    rec.submit()
    kw = oracle.kv_write_f16(oracle.f16_bits(kc), knew, hkv, 1, hd, pos)
    vw = oracle.kv_write_f16(oracle.f16_bits(vc), vnew, hkv, 1, hd, pos)
    assert np.array_equal(bits_of(kt), kw), "K cache bits"
    assert np.array_equal(bits_of(vt), vw), "V cache bits"
    k32 = oracle.kv_write(kc, knew, hkv, 1, hd, pos).reshape(max_seq, hkv, hd)
    v32 = oracle.kv_write(vc, vnew, hkv, 1, hd, pos).reshape(max_seq, hkv, hd)
    check_both(ot.to_f32().reshape(1, h, hd), q.reshape(1, h, hd), k32, v32, h, hkv, pos, 1, hd,
               sc, window, "decode step f16")


@pytest.mark.parametrize("h,hkv,hd,pos0,rows,window", [
    (16, 8, 128, 0, 300, 0),      # a prompt over the cache
    (16, 8, 128, 100, 77, 0),     # continuation chunk
    (32, 8, 128, 1000, 96, 0),    # GQA 4
    (16, 8, 256, 513, 40, 0),     # hd 256
    (4, 2, 8, 5, 3, 0),           # hd 8
    (24, 8, 128, 10, 50, 0),      # g = 3
    (16, 8, 128, 300, 129, 100),  # windowed continuation
])
def test_chunk_f16_matches_oracle(dev, h, hkv, hd, pos0, rows, window):
    note(f"chunk f16 h={h} hd={hd} pos0={pos0} rows={rows} window={window}")
    max_seq = pos0 + rows + 5
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 9)
    kc, vc = oracle.randn((max_seq, hkv, hd), 10), oracle.randn((max_seq, hkv, hd), 11)
    kt, vt = f16_cache(dev, kc), f16_cache(dev, vc)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, upload(dev, q), kt, vt, ot, h, hkv, pos0, rows, hd, max_seq, sc,
                          window)
    rec.submit()
    check_both(ot.to_f32().reshape(rows, h, hd), q, kc, vc, h, hkv, pos0, rows, hd, sc, window,
               "chunk f16")


def test_qwen_prompt_over_f16_cache_sampled_rows(dev):
    """Qwen3 T=4096 prompt as one chunk over an f16 cache, checked on sampled rows."""
    h, hkv, hd, T = 16, 8, 128, 4096
    note("chunk f16 qwen T=4096")
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((T, h, hd), 12)
    kc, vc = oracle.randn((T, hkv, hd), 13), oracle.randn((T, hkv, hd), 14)
    kt, vt = f16_cache(dev, kc), f16_cache(dev, vc)
    ot = eb.Tensor.empty(dev, (T, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, upload(dev, q), kt, vt, ot, h, hkv, 0, T, hd, T, sc)
    rec.submit()
    got = ot.to_f32().reshape(T, h, hd)
    assert np.isfinite(got).all()
    kr, vr = rounded(kc), rounded(vc)
    for r in (0, 1, 63, 64, 1000, 2047, 4094, 4095):
        want = oracle.attn_chunk(q[r:r + 1], kr, vr, h, hkv, r, 1, hd, sc, threads=16)
        assert_close(got[r:r + 1], want, what=f"row {r}")


def test_raw_f16_launches(dev):
    """The stream-level f16 entry points on caller memory (library buffers), on the
    device's stream: kv_write, decode, fused step and chunk."""
    note("raw f16 launches")
    h, hkv, hd, max_seq = 16, 8, 128, 700
    sc = 0.08
    kc, vc = oracle.randn((max_seq, hkv, hd), 20), oracle.randn((max_seq, hkv, hd), 21)
    kt = eb.Tensor.empty(dev, (max_seq, hkv, hd), eb.DType.F16)
    vt = eb.Tensor.empty(dev, (max_seq, hkv, hd), eb.DType.F16)
    ks, vs = upload(dev, kc), upload(dev, vc)
    for dst, src in ((kt, ks), (vt, vs)):
        eb.launch_kv_write_f16(dev.stream, dst.data_ptr, dst.numel(), src.data_ptr, src.numel(),
                               hkv, max_seq, hd, max_seq, 0)
    dev.synchronize()
    assert np.array_equal(bits_of(kt), oracle.f16_bits(kc.ravel()))

    pos0, rows = 600, 33
    q = oracle.randn((rows, h, hd), 22)
    qt = upload(dev, q)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    eb.launch_attn_prefill_chunk_f16(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr,
                                     kt.numel(), vt.data_ptr, vt.numel(), ot.data_ptr,
                                     ot.numel(), h, hkv, pos0, rows, hd, max_seq, sc, 64)
    dev.synchronize()
    check_both(ot.to_f32().reshape(rows, h, hd), q, kc, vc, h, hkv, pos0, rows, hd, sc, 64,
               "raw chunk f16")

    pos = 650
    q1 = upload(dev, q[0])
    o1 = eb.Tensor.empty(dev, (h, hd))
    cus = dev.cu_count
    need = eb.attn_decode_workspace_floats(h, hkv, pos, hd, cus)
    ws = upload(dev, np.full(max(need, 1), np.nan, np.float32))
    eb.launch_attn_decode_f16(dev.stream, q1.data_ptr, q1.numel(), kt.data_ptr, kt.numel(),
                              vt.data_ptr, vt.numel(), o1.data_ptr, o1.numel(), h, hkv, pos, hd,
                              max_seq, sc, 0, ws.data_ptr, need, cus)
    dev.synchronize()
    check_both(o1.to_f32().reshape(1, h, hd), q[0].reshape(1, h, hd), kc, vc, h, hkv, pos, 1,
               hd, sc, 0, "raw decode f16")

    knew, vnew = oracle.randn((1, hkv, hd), 23), oracle.randn((1, hkv, hd), 24)
    kn, vn = upload(dev, knew), upload(dev, vnew)
    eb.launch_attn_decode_step_f16(dev.stream, q1.data_ptr, q1.numel(), kn.data_ptr,
                                   vn.data_ptr, kn.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
                                   vt.numel(), o1.data_ptr, o1.numel(), h, hkv, pos, hd, max_seq,
                                   sc, 0, ws.data_ptr, need, cus)
    dev.synchronize()
    assert np.array_equal(bits_of(kt), oracle.kv_write_f16(oracle.f16_bits(kc), knew, hkv, 1,
                                                           hd, pos))
    k32 = oracle.kv_write(kc, knew, hkv, 1, hd, pos).reshape(max_seq, hkv, hd)
    v32 = oracle.kv_write(vc, vnew, hkv, 1, hd, pos).reshape(max_seq, hkv, hd)
    check_both(o1.to_f32().reshape(1, h, hd), q[0].reshape(1, h, hd), k32, v32, h, hkv, pos, 1,
               hd, sc, 0, "raw decode step f16")


def test_f16_cache_refusals(dev):
    """Head dims below 8 and a mixed f32/f16 cache pair are refused before any launch."""
    note("f16 refusals")
    h, hkv, hd, max_seq = 4, 2, 4, 16
    k16 = eb.Tensor.empty(dev, (max_seq, hkv, hd), eb.DType.F16)
    v16 = eb.Tensor.empty(dev, (max_seq, hkv, hd), eb.DType.F16)
    v32 = eb.Tensor.empty(dev, (max_seq, hkv, hd))
    q = eb.Tensor.empty(dev, (h, hd))
    o = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    with pytest.raises(eb.UnsupportedConfig):
        eb.attn_decode(rec, q, k16, v16, o, h, hkv, 3, hd, max_seq, 0.5)
    with pytest.raises((eb.ShapeMismatch, eb.UnsupportedConfig)):
        eb.attn_decode(rec, q, k16, v32, o, h, hkv, 3, hd, max_seq, 0.5)
    with pytest.raises(eb.UnsupportedConfig):
        eb.KvCache.new(dev, 1, 8, 2, 8, eb.DType.U32)
    rec.submit()


def test_attention_forward_with_f16_cache(dev):
    """Attention.forward_qkv over an f16 KvCache: a 300-row prompt, a 50-row continuation
    and three decode steps. Each output against the oracle on the cache as the layer left
    it (FP32 bar), and against the same layer over an f32 cache."""
    H, Hkv, hd, max_seq = 16, 8, 128, 512
    note("attention forward f16 cache")
    sc = float(oracle.default_scale(hd))
    attn = eb.Attention(H, Hkv, hd, sc)
    rope = eb.Rope.build(dev, max_seq, hd, 1e6)
    kv16 = eb.KvCache.new(dev, 1, max_seq, Hkv, hd, eb.DType.F16)
    kv32 = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    assert kv16.dtype == eb.DType.F16 and kv16.k[0].dtype == eb.DType.F16
    spans = [(0, 300), (300, 350), (350, 351), (351, 352), (352, 353)]
    n = spans[-1][1]
    xq = oracle.randn((n, H * hd), 51)
    xk = oracle.randn((n, Hkv * hd), 52)
    xv = oracle.randn((n, Hkv * hd), 53)
    for a, b in spans:
        rows = b - a
        outs = []
        for kv in (kv16, kv32):
            rec = eb.Recorder(dev)
            qt = upload(dev, xq[a:b])
            out = attn.forward_qkv(rec, qt, upload(dev, xk[a:b]), upload(dev, xv[a:b]), rope, kv,
                                   0, rows, a)
            qr = eb.Tensor.empty(dev, (rows, H, hd))
            eb.rope(rec, qt, rope.cos, rope.sin, qr, rows, H, hd, a)
            rec.submit()
            outs.append((out.to_f32().reshape(rows, H, hd), qr.to_f32().reshape(rows, H, hd)))
        (o16, qr), (o32, _) = outs
        kc = oracle.f16_values(bits_of(kv16.k[0])).reshape(max_seq, Hkv, hd)
        vc = oracle.f16_values(bits_of(kv16.v[0])).reshape(max_seq, Hkv, hd)
        k32 = kv32.k[0].to_f32().reshape(max_seq, Hkv, hd)
        assert np.array_equal(oracle.f16_bits(k32[:b]).ravel(), bits_of(kv16.k[0])[:b * Hkv * hd]), \
            "f16 cache rows are the f32 layer's rows rounded"
        want = oracle.attn_chunk(qr, kc, vc, H, Hkv, a, rows, hd, sc, threads=16)
        assert_close(o16, want, what=f"span {a}..{b} vs oracle on the f16 cache")
        assert_close(o16, o32, rel=NORTH_REL_L2, abs_=NORTH_MAX_ABS,
                     what=f"span {a}..{b} vs f32-cache layer")
