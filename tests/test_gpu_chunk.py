"""Chunked causal prefill and sliding-window attention on the GPU against the oracle.

The reference has neither (its Attention routes rows > 1 at base_pos > 0 to a prefill over
the fresh rows only, crates/eyebrowse-nn/src/attention.rs:40, and its README defers
chunked prefill and sliding windows). The oracle's attn_chunk applies the reference's
per-row softmax (crates/eyebrowse-kernels/src/testutil.rs:142-169) to the key range each
query sees; tests/test_oracle.py pins it against float64 textbook attention and shows it
reduces bitwise to attn_prefill / attn_decode.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, prefill, upload

pytestmark = pytest.mark.gpu


def chunk(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, scale, window=0):
    qt, kt, vt = upload(dev, q), upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, qt, kt, vt, ot, h, hkv, pos0, rows, hd, max_seq, scale, window)
    rec.submit()
    return ot.to_f32().reshape(rows, h, hd)


@pytest.mark.parametrize("h,hkv,hd,pos0,rows,window", [
    (16, 8, 128, 100, 77, 0),    # continuation chunk, unaligned start and length
    (16, 8, 128, 37, 64, 0),
    (32, 8, 128, 1000, 96, 0),   # GQA 4
    (16, 8, 256, 513, 40, 0),    # hd 256
    (4, 2, 8, 5, 3, 0),          # tiny head_dim
    (24, 8, 128, 10, 50, 0),     # g = 3
    (8, 1, 64, 0, 200, 50),      # windowed prompt
    (16, 8, 128, 300, 129, 100), # windowed continuation
    (16, 16, 32, 64, 64, 1),     # window 1: each query sees only itself
    (16, 8, 128, 20, 30, 4096),  # window longer than the context
])
def test_chunk_matches_oracle(dev, h, hkv, hd, pos0, rows, window):
    note(f"chunk h={h} hkv={hkv} hd={hd} pos0={pos0} rows={rows} window={window}")
    max_seq = pos0 + rows + 7
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 1)
    kc = oracle.randn((max_seq, hkv, hd), 2)
    vc = oracle.randn((max_seq, hkv, hd), 3)
    got = chunk(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window)
    want = oracle.attn_chunk(q, kc, vc, h, hkv, pos0, rows, hd, sc, window, threads=16)
    assert_close(got, want, what="chunk")
    if window == 1:
        np.testing.assert_allclose(got, np.repeat(vc[pos0:pos0 + rows], h // hkv, axis=1),
                                   rtol=0, atol=1e-6)


def test_key_chunk_merge_with_v_magnitudes_far_apart(dev):
    """128 rows over 8K cached keys run as key chunks merged by log-sum-exp. The first
    half of the keys score about +100 with V rows near 2^-100; the second half about -100
    with V rows near 2^+100. The second half's weight (about 2^-288) makes its terms
    vanish although its V rows are 2^200 larger, so the merge must take its reference
    exponent from the weighted terms: taken from the V rows alone it would push the first
    half's partials below f32 range and return zeros."""
    h, hkv, hd, max_seq, rows = 16, 8, 128, 8192, 128
    pos0 = max_seq - rows
    note(f"chunk merge, V 2^-100 / 2^+100 halves, rows={rows} over {max_seq} keys")
    sc = float(oracle.default_scale(hd))
    u = oracle.randn((hd,), 61).astype(np.float64)
    a = 100.0 / (sc * float(u @ u))
    half = max_seq // 2
    sign = np.where(np.arange(max_seq) < half, 1.0, -1.0)[:, None, None]
    kc = (sign * a * u[None, None, :] + 0.3 * oracle.randn((max_seq, hkv, hd), 62)).astype(np.float32)
    vmag = np.where(np.arange(max_seq) < half, 2.0 ** -100, 2.0 ** 100)[:, None, None]
    vc = (vmag * oracle.randn((max_seq, hkv, hd), 63)).astype(np.float32)
    q = (u[None, None, :] + 0.01 * oracle.randn((rows, h, hd), 64)).astype(np.float32)
    got = chunk(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc)
    want = oracle.attn_chunk(q, kc, vc, h, hkv, pos0, rows, hd, sc, 0, threads=16)
    assert np.abs(want).max() > 2.0 ** -110, "the first half's V rows must carry the output"
    assert_close(got, want, what="chunk merge, far-apart V magnitudes")


def test_chunk_from_zero_is_prefill_bitwise(dev):
    """With pos0 = 0 and no window the chunk kernel is the prefill kernel over the cache."""
    note("chunk pos0=0 vs prefill")
    h, hkv, hd, T = 16, 8, 128, 200
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((T, h, hd), 1), oracle.randn((T, hkv, hd), 2), oracle.randn((T, hkv, hd), 3)
    a = chunk(dev, q, k, v, h, hkv, 0, T, hd, T, sc)
    b = prefill(dev, q, k, v, h, hkv, T, hd, sc)
    assert_bitwise(a, b, "chunk vs prefill")


def test_qwen_prompt_continuation_rows(dev):
    """Qwen3 shape: the second half of a T=4096 prompt as one chunk at pos0 = 2048, checked
    on sampled rows (each a decode at its position in the oracle)."""
    h, hkv, hd, T, pos0 = 16, 8, 128, 4096, 2048
    rows = T - pos0
    note(f"qwen chunk pos0={pos0} rows={rows}")
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 11)
    kc, vc = oracle.randn((T, hkv, hd), 12), oracle.randn((T, hkv, hd), 13)
    got = chunk(dev, q, kc, vc, h, hkv, pos0, rows, hd, T, sc)
    assert np.isfinite(got).all()
    for r in (0, 1, 31, 32, 777, 1500, rows - 2, rows - 1):
        want = oracle.attn_chunk(q[r:r + 1], kc, vc, h, hkv, pos0 + r, 1, hd, sc, threads=16)
        assert_close(got[r:r + 1], want, what=f"row {r}")


@pytest.mark.parametrize("h,hkv,hd,pos,window", [
    (16, 8, 128, 8191, 1024),
    (16, 8, 256, 5000, 4096),
    (32, 8, 128, 3000, 100),
    (4, 2, 8, 40, 1),
    (16, 8, 128, 200, 5000),  # window longer than the context
])
def test_decode_window_matches_oracle(dev, h, hkv, hd, pos, window):
    note(f"decode window h={h} hd={hd} pos={pos} window={window}")
    max_seq = pos + 3
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((h, hd), 1)
    kc, vc = oracle.randn((max_seq, hkv, hd), 2), oracle.randn((max_seq, hkv, hd), 3)
    qt, kt, vt = upload(dev, q), upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode_window(rec, qt, kt, vt, ot, h, hkv, pos, hd, max_seq, sc, window)
    rec.submit()
    want = oracle.attn_chunk(q.reshape(1, h, hd), kc, vc, h, hkv, pos, 1, hd, sc, window)
    assert_close(ot.to_f32().reshape(1, h, hd), want, what="decode window")

    # fused step with the same window: the new row lands at `pos`, the output matches
    knew, vnew = oracle.randn((1, hkv, hd), 4), oracle.randn((1, hkv, hd), 5)
    k2, v2 = upload(dev, kc), upload(dev, vc)
    o2 = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode_step_window(rec, qt, upload(dev, knew), upload(dev, vnew), k2, v2, o2, h, hkv,
                               pos, hd, max_seq, sc, window)
    rec.submit()
    kw = oracle.kv_write(kc, knew, hkv, 1, hd, pos)
    vw = oracle.kv_write(vc, vnew, hkv, 1, hd, pos)
    assert_bitwise(k2.to_f32(), kw, "K cache")
    assert_bitwise(v2.to_f32(), vw, "V cache")
    want2 = oracle.attn_chunk(q.reshape(1, h, hd), kw, vw, h, hkv, pos, 1, hd, sc, window)
    assert_close(o2.to_f32().reshape(1, h, hd), want2, what="decode step window")


def test_raw_chunk_and_window_launches(dev):
    """The stream-level entry points on caller memory, on the device's stream."""
    note("raw chunk / window launches")
    h, hkv, hd, pos0, rows, max_seq = 16, 8, 128, 500, 33, 600
    sc = 0.07
    q = oracle.randn((rows, h, hd), 1)
    kc, vc = oracle.randn((max_seq, hkv, hd), 2), oracle.randn((max_seq, hkv, hd), 3)
    qt, kt, vt = upload(dev, q), upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    eb.launch_attn_prefill_chunk(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                                 vt.data_ptr, vt.numel(), ot.data_ptr, ot.numel(), h, hkv, pos0,
                                 rows, hd, max_seq, sc, 64)
    dev.synchronize()
    want = oracle.attn_chunk(q, kc, vc, h, hkv, pos0, rows, hd, sc, 64, threads=16)
    assert_close(ot.to_f32().reshape(rows, h, hd), want, what="raw chunk")

    pos, window = 599, 200
    q1 = upload(dev, q[0])
    o1 = eb.Tensor.empty(dev, (h, hd))
    cus = dev.cu_count
    need = eb.attn_decode_workspace_floats(h, hkv, pos, hd, cus)
    ws = upload(dev, np.full(max(need, 1), np.nan, np.float32))
    eb.launch_attn_decode_window(dev.stream, q1.data_ptr, q1.numel(), kt.data_ptr, kt.numel(),
                                 vt.data_ptr, vt.numel(), o1.data_ptr, o1.numel(), h, hkv, pos,
                                 hd, max_seq, sc, window, ws.data_ptr, need, cus)
    dev.synchronize()
    want = oracle.attn_chunk(q[0].reshape(1, h, hd), kc, vc, h, hkv, pos, 1, hd, sc, window)
    assert_close(o1.to_f32().reshape(1, h, hd), want, what="raw decode window")


def test_attention_forward_in_chunks_equals_one_prefill(dev):
    """A prompt fed to Attention.forward_qkv in three chunks (0..100, 100..250, 250..300)
    gives the rows one prefill of all 300 gives, and leaves the same cache."""
    H, Hkv, hd, T, max_seq = 16, 8, 128, 300, 512
    note("attention forward chunks")
    sc = float(oracle.default_scale(hd))
    xq = oracle.randn((T, H * hd), 31)
    xk = oracle.randn((T, Hkv * hd), 32)
    xv = oracle.randn((T, Hkv * hd), 33)
    attn = eb.Attention(H, Hkv, hd, sc)
    rope = eb.Rope.build(dev, max_seq, hd, 1e6)
    kv1 = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    rec = eb.Recorder(dev)
    full = attn.forward_qkv(rec, upload(dev, xq), upload(dev, xk), upload(dev, xv), rope, kv1, 0,
                            T, 0)
    rec.submit()
    full = full.to_f32().reshape(T, H * hd)
    kv2 = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    parts = []
    for a, b in ((0, 100), (100, 250), (250, 300)):
        rec = eb.Recorder(dev)
        out = attn.forward_qkv(rec, upload(dev, xq[a:b]), upload(dev, xk[a:b]),
                               upload(dev, xv[a:b]), rope, kv2, 0, b - a, a)
        rec.submit()
        parts.append(out.to_f32().reshape(b - a, H * hd))
    assert_close(np.concatenate(parts), full, what="chunks vs one prefill")
    n = T * Hkv * hd
    assert_bitwise(kv2.k[0].to_f32()[:n], kv1.k[0].to_f32()[:n], "K cache")
    assert_bitwise(kv2.v[0].to_f32()[:n], kv1.v[0].to_f32()[:n], "V cache")


def test_windowed_attention_forward(dev):
    """A sliding-window layer (window 64) through Attention.forward_qkv: prompt of 150,
    continuation chunk of 50, then two decode steps; every output against the oracle on the
    cache contents (RoPE'd K and V as written by the layer itself)."""
    H, Hkv, hd, W, max_seq = 8, 4, 64, 64, 256
    note("windowed attention forward")
    sc = float(oracle.default_scale(hd))
    attn = eb.Attention(H, Hkv, hd, sc, window=W)
    rope = eb.Rope.build(dev, max_seq, hd, 1e4)
    kv = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    spans = [(0, 150), (150, 200), (200, 201), (201, 202)]
    xq = oracle.randn((202, H * hd), 41)
    xk = oracle.randn((202, Hkv * hd), 42)
    xv = oracle.randn((202, Hkv * hd), 43)
    for a, b in spans:
        rows = b - a
        rec = eb.Recorder(dev)
        qt = upload(dev, xq[a:b])
        out = attn.forward_qkv(rec, qt, upload(dev, xk[a:b]), upload(dev, xv[a:b]), rope, kv, 0,
                               rows, a)
        # the rotated q the layer attended with
        qr = eb.Tensor.empty(dev, (rows, H, hd))
        eb.rope(rec, qt, rope.cos, rope.sin, qr, rows, H, hd, a)
        rec.submit()
        kc = kv.k[0].to_f32().reshape(max_seq, Hkv, hd)
        vc = kv.v[0].to_f32().reshape(max_seq, Hkv, hd)
        want = oracle.attn_chunk(qr.to_f32().reshape(rows, H, hd), kc, vc, H, Hkv, a, rows, hd,
                                 sc, W, threads=16)
        assert_close(out.to_f32().reshape(rows, H, hd), want, what=f"window span {a}..{b}")
