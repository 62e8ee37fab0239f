"""Seeded random shapes through every attention entry point on the GPU, against the oracle.

Each case draws head_dim, GQA ratio, lengths, positions, window, scale and cache dtype
from a fixed seed, so the sweep crosses the paths the fixed cases take one at a time
(pre-split pass on or off, key chunks, sliding windows, IEEE-half and E4M3 caches, split-KV
decode with the fused new-token step) at shapes none of them uses. The oracle is the reference's
CPU attention restated in oracle/oracle.c (testutil.rs:130-218) with the chunk/window
extension (attn_chunk); outputs are held to the FP32 bar of tests/_gpu.py on the rows
each case samples.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload

pytestmark = pytest.mark.gpu

HDS = (4, 8, 16, 32, 64, 128, 256)


def cache_kind(narrow, seed):
    """The cache element type of a case: f32, or (narrow) IEEE half, or E4M3 for every
    third seed (drawn without the case's generator, so its other draws stay put)."""
    if not narrow:
        return "f32"
    return "f8" if seed % 3 == 0 else "f16"


def rounded(a, kind):
    """The values a cache of this kind holds for the f32 rows a."""
    if kind == "f16":
        return oracle.f16_values(oracle.f16_bits(a)).reshape(a.shape)
    if kind == "f8":
        return oracle.f8_values(oracle.f8_bits(a)).reshape(a.shape)
    return a


DTYPE = {"f32": eb.DType.F32, "f16": eb.DType.F16, "f8": eb.DType.F8E4M3}


def draw(seed):
    r = np.random.default_rng(1000 + seed)
    hd = int(r.choice(HDS))
    hkv = int(r.choice((1, 2, 4, 8)))
    g = int(r.choice((1, 2, 3, 4, 8)))
    scale = float(r.choice((0.0, 1.0, 0.05, 0.3))) if seed % 4 == 0 else float(oracle.default_scale(hd))
    return r, hd, hkv * g, hkv, scale


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill(dev, seed):
    r, hd, h, hkv, sc = draw(seed)
    s = int(r.integers(1, 700))
    note(f"random prefill seed={seed} h={h} hkv={hkv} hd={hd} s={s} scale={sc}")
    q = oracle.randn((s, h, hd), 3 * seed)
    k, v = oracle.randn((s, hkv, hd), 3 * seed + 1), oracle.randn((s, hkv, hd), 3 * seed + 2)
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    ot = eb.Tensor.empty(dev, (s, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill(rec, qt, kt, vt, ot, h, hkv, s, hd, sc)
    rec.submit()
    got = ot.to_f32().reshape(s, h, hd)
    for r0 in sorted({0, max(0, s // 2 - 8), max(0, s - 16)}):
        n = min(16, s - r0)
        want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=(r0, n), threads=16)
        assert_close(got[r0:r0 + n], want[r0:r0 + n], what=f"rows {r0}+{n}")


@pytest.mark.parametrize("seed", range(24))
def test_random_chunk(dev, seed):
    r, hd, h, hkv, sc = draw(100 + seed)
    pos0 = int(r.integers(0, 1500))
    rows = int(r.integers(1, 400))
    window = int(r.choice((0, 0, 1, 17, 200, 5000)))
    kind = cache_kind(hd >= 8 and bool(r.integers(0, 2)), seed)
    max_seq = pos0 + rows + int(r.integers(0, 9))
    note(f"random chunk seed={seed} h={h} hkv={hkv} hd={hd} pos0={pos0} rows={rows} "
         f"window={window} cache={kind}")
    q = oracle.randn((rows, h, hd), 7 * seed + 1)
    kc, vc = oracle.randn((max_seq, hkv, hd), 7 * seed + 2), oracle.randn((max_seq, hkv, hd), 7 * seed + 3)
    if kind != "f32":
        kt = eb.Tensor.empty(dev, kc.shape, DTYPE[kind])
        vt = eb.Tensor.empty(dev, vc.shape, DTYPE[kind])
        rec = eb.Recorder(dev)
        eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
        eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
        rec.submit()
        kc, vc = rounded(kc, kind), rounded(vc, kind)
    else:
        kt, vt = upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, upload(dev, q), kt, vt, ot, h, hkv, pos0, rows, hd, max_seq, sc,
                          window)
    rec.submit()
    got = ot.to_f32().reshape(rows, h, hd)
    for rr in sorted({0, rows // 2, rows - 1}):
        want = oracle.attn_chunk(q[rr:rr + 1], kc, vc, h, hkv, pos0 + rr, 1, hd, sc, window,
                                 threads=16)
        assert_close(got[rr:rr + 1], want, what=f"row {rr}")


@pytest.mark.parametrize("seed", range(20))
def test_random_decode_step(dev, seed):
    """The fused step (new row written at pos, attention over 0..=pos, optional window)
    against kv_write + the oracle; the cache row must be the new row's bits (f32) or its
    rounding (IEEE half, E4M3)."""
    r, hd, h, hkv, sc = draw(200 + seed)
    max_seq = int(r.integers(2, 20000))
    pos = int(r.integers(0, max_seq))
    window = int(r.choice((0, 0, 1, 33, 4096)))
    kind = cache_kind(hd >= 8 and bool(r.integers(0, 2)), seed)
    note(f"random decode seed={seed} h={h} hkv={hkv} hd={hd} pos={pos} max_seq={max_seq} "
         f"window={window} cache={kind}")
    kc, vc = oracle.randn((max_seq, hkv, hd), 11 * seed + 1), oracle.randn((max_seq, hkv, hd), 11 * seed + 2)
    q = oracle.randn((h, hd), 11 * seed + 3)
    kn, vn = oracle.randn((hkv, hd), 11 * seed + 4), oracle.randn((hkv, hd), 11 * seed + 5)
    dt = DTYPE[kind]
    kt, vt = eb.Tensor.empty(dev, kc.shape, dt), eb.Tensor.empty(dev, vc.shape, dt)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
    eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
    ot = eb.Tensor.empty(dev, (h, hd))
    eb.attn_decode_step_window(rec, upload(dev, q), upload(dev, kn), upload(dev, vn), kt, vt, ot,
                               h, hkv, pos, hd, max_seq, sc, window)
    rec.submit()
    kc[pos], vc[pos] = kn, vn
    if kind == "f16":
        row = np.frombuffer(kt.read_bytes(), np.uint16).reshape(max_seq, hkv, hd)[pos]
        assert np.array_equal(row, oracle.f16_bits(kn).reshape(hkv, hd))
    elif kind == "f8":
        row = np.frombuffer(kt.read_bytes(), np.uint8).reshape(max_seq, hkv, hd)[pos]
        assert np.array_equal(row, oracle.f8_bits(kn).reshape(hkv, hd))
    if kind != "f32":
        kc, vc = rounded(kc, kind), rounded(vc, kind)
    else:
        assert_bitwise(kt.to_f32().reshape(max_seq, hkv, hd)[pos], kn, "new K row")
    want = oracle.attn_chunk(q.reshape(1, h, hd), kc, vc, h, hkv, pos, 1, hd, sc, window,
                             threads=16)
    assert_close(ot.to_f32().reshape(1, h, hd), want, what="decode step")


def _caches(dev, max_seq, hkv, hd, kind, seed):
    """Seeded K/V caches on the device (f32, or IEEE-half / E4M3 written by kv_write) and
    the values they hold, as f32 for the oracle."""
    kc = oracle.randn((max_seq, hkv, hd), seed)
    vc = oracle.randn((max_seq, hkv, hd), seed + 1)
    if kind == "f32":
        return upload(dev, kc), upload(dev, vc), kc, vc
    kt = eb.Tensor.empty(dev, kc.shape, DTYPE[kind])
    vt = eb.Tensor.empty(dev, vc.shape, DTYPE[kind])
    rec = eb.Recorder(dev)
    eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
    eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
    rec.submit()
    return kt, vt, rounded(kc, kind), rounded(vc, kind)


@pytest.mark.parametrize("seed", range(24))
def test_random_raw_decode(dev, seed):
    """Stream-level decode on a caller workspace of exactly the size the public sizing
    function returns, for CU counts other than the device's (other split plans), f32,
    IEEE-half and E4M3 caches, with and without a window. The workspace starts as NaN so a partial
    the launch forgets to write shows up in the output."""
    r, hd, h, hkv, sc = draw(300 + seed)
    max_seq = int(r.integers(2, 20000))
    pos = int(r.integers(0, max_seq))
    window = int(r.choice((0, 0, 1, 77, 3000)))
    kind = cache_kind(hd >= 8 and bool(r.integers(0, 2)), seed)
    cus = int(r.choice((dev.cu_count, 1, 40, 304, 1000)))
    note(f"random raw decode seed={seed} h={h} hkv={hkv} hd={hd} pos={pos} max_seq={max_seq} "
         f"window={window} cache={kind} cus={cus}")
    kt, vt, kc, vc = _caches(dev, max_seq, hkv, hd, kind, 13 * seed + 1)
    q = oracle.randn((h, hd), 13 * seed + 3)
    qt = upload(dev, q)
    ot = eb.Tensor.empty(dev, (h, hd))
    need = eb.attn_decode_workspace_floats(h, hkv, pos, hd, cus)
    ws = upload(dev, np.full(max(need, 1), np.nan, np.float32))
    args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
            vt.numel(), ot.data_ptr, ot.numel(), h, hkv, pos, hd, max_seq, sc)
    if kind == "f16":
        eb.launch_attn_decode_f16(*args, window, ws.data_ptr, need, cus)
    elif kind == "f8":
        eb.launch_attn_decode_f8(*args, window, ws.data_ptr, need, cus)
    else:
        eb.launch_attn_decode_window(*args, window, ws.data_ptr, need, cus)
    dev.synchronize()
    want = oracle.attn_chunk(q.reshape(1, h, hd), kc, vc, h, hkv, pos, 1, hd, sc, window,
                             threads=16)
    assert_close(ot.to_f32().reshape(1, h, hd), want, what="raw decode")


@pytest.mark.parametrize("seed", range(20))
def test_random_raw_prefill_ws(dev, seed):
    """Stream-level chunked prefill on a caller workspace of exactly the size
    eb_attn_prefill_workspace_floats returns (pre-split records and, for launches with few
    query blocks, key-chunk partials), NaN-filled beforehand."""
    r, hd, h, hkv, sc = draw(400 + seed)
    pos0 = int(r.integers(0, 3000))
    rows = int(r.integers(1, 300))
    window = int(r.choice((0, 0, 1, 40, 1000)))
    kind = cache_kind(hd >= 8 and bool(r.integers(0, 2)), seed)
    max_seq = pos0 + rows + int(r.integers(0, 5))
    note(f"random raw prefill_ws seed={seed} h={h} hkv={hkv} hd={hd} pos0={pos0} rows={rows} "
         f"window={window} cache={kind}")
    kt, vt, kc, vc = _caches(dev, max_seq, hkv, hd, kind, 17 * seed + 1)
    q = oracle.randn((rows, h, hd), 17 * seed + 3)
    qt = upload(dev, q)
    ot = eb.Tensor.empty(dev, (rows, h, hd))
    need = eb.attn_prefill_workspace_floats(h, hkv, hd, pos0, rows, window)
    ws = upload(dev, np.full(max(need, 1), np.nan, np.float32))
    eb.launch_attn_prefill_chunk_ws(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr,
                                    kt.numel(), vt.data_ptr, vt.numel(), ot.data_ptr,
                                    ot.numel(), h, hkv, pos0, rows, hd, max_seq, sc, window,
                                    ws.data_ptr, need, f16=kind == "f16", f8=kind == "f8")
    dev.synchronize()
    got = ot.to_f32().reshape(rows, h, hd)
    for rr in sorted({0, rows // 3, rows - 1}):
        want = oracle.attn_chunk(q[rr:rr + 1], kc, vc, h, hkv, pos0 + rr, 1, hd, sc, window,
                                 threads=16)
        assert_close(got[rr:rr + 1], want, what=f"row {rr}")


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill_pv16(dev, seed):
    """The scores-accurate mode at random shapes (head dims 24-256, odd multiples of 8
    included, GQA 1-8, lengths 1-900, scales up to 1.0) and random launch forms (recorder,
    raw with and without a workspace), against the oracle at the mode's bound: max-abs
    <= 2^-11 x max|V| + 2e-5 and rel-L2 <= 4e-4 on the sampled rows."""
    r = np.random.default_rng(5000 + seed)
    hd = int(r.choice((24, 32, 40, 64, 72, 96, 120, 128, 160, 256)))
    hkv = int(r.choice((1, 2, 4, 8)))
    g = int(r.choice((1, 2, 3, 4, 8)))
    h = hkv * g
    s = int(r.integers(1, 900))
    sc = float(r.choice((1.0, 0.3))) if seed % 3 == 0 else float(oracle.default_scale(hd))
    form = ("recorder", "raw", "raw_ws")[seed % 3]
    note(f"random pv16 seed={seed} h={h} hkv={hkv} hd={hd} s={s} scale={sc} {form}")
    q = oracle.randn((s, h, hd), 7 * seed)
    k, v = oracle.randn((s, hkv, hd), 7 * seed + 1), oracle.randn((s, hkv, hd), 7 * seed + 2)
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    ot = eb.Tensor.empty(dev, (s, h, hd))
    if form == "recorder":
        rec = eb.Recorder(dev)
        eb.attn_prefill_pv16(rec, qt, kt, vt, ot, h, hkv, s, hd, sc)
        rec.submit()
    else:
        args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
                vt.numel(), ot.data_ptr, ot.numel(), h, hkv, s, hd, sc)
        if form == "raw":
            eb.launch_attn_prefill_pv16(*args)
        else:
            need = eb.attn_prefill_workspace_floats(h, hkv, hd, 0, s)
            ws = eb.Tensor.empty(dev, (max(need, 1),))
            eb.launch_attn_prefill_pv16_ws(*args, ws.data_ptr, need)
        dev.synchronize()
    got = ot.to_f32().reshape(s, h, hd)
    assert np.isfinite(got).all()
    bound = 2.0 ** -11 * float(np.abs(v).max()) + 2e-5
    for r0 in sorted({0, max(0, s // 2 - 8), max(0, s - 16)}):
        n = min(16, s - r0)
        want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=(r0, n), threads=16)
        d = got[r0:r0 + n].astype(np.float64) - want[r0:r0 + n].astype(np.float64)
        assert float(np.abs(d).max()) <= bound, (r0, float(np.abs(d).max()), bound)
        den = float(np.linalg.norm(want[r0:r0 + n].astype(np.float64)))
        assert float(np.linalg.norm(d)) <= 4e-4 * den + 1e-12, (r0, float(np.linalg.norm(d)) / den)
