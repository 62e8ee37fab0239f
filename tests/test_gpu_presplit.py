"""The prefill's pre-split pass on the GPU.

A prefill launched through a recorder with at least 256 query rows and head_dim 32..128
first splits every key in range once (pre-split records in the device workspace) and then
only copies records into LDS; a raw launch (no workspace) splits while staging. Both hold
the same values in LDS, so their outputs must be equal bit for bit; the recorder path is
also checked against the oracle (attention.rs:94-120 / testutil.rs:130-172 restated in
oracle/oracle.c) at the FP32 bar of tests/_gpu.py.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload

pytestmark = pytest.mark.gpu


def recorder_and_raw_prefill(dev, q, k, v, h, hkv, s, hd, sc):
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    a = eb.Tensor.empty(dev, (s, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill(rec, qt, kt, vt, a, h, hkv, s, hd, sc)
    rec.submit()
    b = eb.Tensor.empty(dev, (s, h, hd))
    eb.launch_attn_prefill(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                           vt.data_ptr, vt.numel(), b.data_ptr, b.numel(), h, hkv, s, hd, sc)
    dev.synchronize()
    return a.to_f32().reshape(s, h, hd), b.to_f32().reshape(s, h, hd)


@pytest.mark.parametrize("h,hkv,s,hd", [
    (16, 8, 300, 128),   # Qwen3 heads: 2 heads x 2 blocks x 2 key splits per workgroup
    (32, 8, 257, 128),   # Mistral heads: 4 heads per workgroup, one record per step
    (24, 8, 290, 128),   # GQA 3: 1 head x 4 blocks x 2 key splits
    (8, 8, 297, 64),
    (4, 2, 300, 32),
    (16, 8, 256, 128),   # exactly the threshold, whole tiles
    (16, 8, 300, 256),   # head_dim 256: image records copied memory-to-LDS, 2 heads x 2 blocks
    (32, 8, 257, 256),   # head_dim 256, 4 heads per workgroup
    (8, 8, 290, 256),    # head_dim 256, MHA: 4 query blocks per workgroup
])
def test_prefill_presplit_equals_staged_split(dev, h, hkv, s, hd):
    note(f"presplit prefill h={h} hkv={hkv} s={s} hd={hd}")
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 31), oracle.randn((s, hkv, hd), 32), oracle.randn((s, hkv, hd), 33)
    a, b = recorder_and_raw_prefill(dev, q, k, v, h, hkv, s, hd, sc)
    assert_bitwise(a, b, "pre-split vs staged split")
    rows = (0, 40) if s <= 260 else (s - 60, 60)
    want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=rows, threads=16)
    assert_close(a[rows[0]:rows[0] + rows[1]], want[rows[0]:rows[0] + rows[1]], what="pre-split")


@pytest.mark.parametrize("hd", [128, 256])
def test_prefill_presplit_special_rows(dev, hd):
    """Zero K/V rows (kept below every real exponent), rows of very different magnitudes,
    and an inf in one V row at key 224 (the first key of a tile, so no earlier query's wave
    reads it)."""
    note(f"presplit special rows hd={hd}")
    h, hkv, s = 16, 8, 320
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 41), oracle.randn((s, hkv, hd), 42), oracle.randn((s, hkv, hd), 43)
    k[5], v[7] = 0.0, 0.0
    k[100:110] *= np.float32(1e-20)
    v[120:130] *= np.float32(1e20)
    v[224, 3, 17] = np.inf
    a, b = recorder_and_raw_prefill(dev, q, k, v, h, hkv, s, hd, sc)
    assert_bitwise(a, b, "special rows")
    want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=(0, 224), threads=16)
    assert_close(a[:120], want[:120], what="rows before the large V rows")
    scale = np.abs(want[130:224]).max()
    assert_close(a[130:224] / scale, want[130:224] / scale, what="rows after the large V rows")
    assert not np.isfinite(a[224:, 6:8]).all()  # the heads of KV head 3 see the inf
    assert np.isfinite(a[224:, :6]).all() and np.isfinite(a[224:, 8:]).all()


def chunk_pair(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16):
    qt = upload(dev, q)
    if f16:
        kt = eb.Tensor.empty(dev, kc.shape, eb.DType.F16)
        vt = eb.Tensor.empty(dev, vc.shape, eb.DType.F16)
        rec = eb.Recorder(dev)
        eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
        eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
        rec.submit()
        raw = eb.launch_attn_prefill_chunk_f16
    else:
        kt, vt = upload(dev, kc), upload(dev, vc)
        raw = eb.launch_attn_prefill_chunk
    a = eb.Tensor.empty(dev, (rows, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill_chunk(rec, qt, kt, vt, a, h, hkv, pos0, rows, hd, max_seq, sc, window)
    rec.submit()
    b = eb.Tensor.empty(dev, (rows, h, hd))
    raw(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr, vt.numel(),
        b.data_ptr, b.numel(), h, hkv, pos0, rows, hd, max_seq, sc, window)
    dev.synchronize()
    return a.to_f32().reshape(rows, h, hd), b.to_f32().reshape(rows, h, hd)


@pytest.mark.parametrize("h,hkv,hd,pos0,rows,window,f16", [
    (16, 8, 128, 100, 300, 0, False),    # continuation, unaligned start
    (32, 8, 128, 0, 256, 0, False),      # from position 0 through the chunk entry point
    (8, 1, 64, 0, 300, 50, False),       # windowed prompt
    (16, 8, 128, 300, 260, 100, False),  # windowed continuation: records start past tile 0
    (16, 8, 128, 70, 280, 0, True),      # f16 cache
    (24, 8, 128, 500, 300, 77, True),    # f16 cache, GQA 3, window
    (16, 8, 256, 100, 300, 0, False),    # head_dim 256 continuation
    (16, 8, 256, 300, 260, 100, True),   # head_dim 256, f16 cache, window
])
def test_chunk_presplit_equals_staged_split(dev, h, hkv, hd, pos0, rows, window, f16):
    note(f"presplit chunk h={h} hd={hd} pos0={pos0} rows={rows} window={window} f16={f16}")
    max_seq = pos0 + rows + 9
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 51)
    kc, vc = oracle.randn((max_seq, hkv, hd), 52), oracle.randn((max_seq, hkv, hd), 53)
    a, b = chunk_pair(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16)
    assert_bitwise(a, b, "pre-split vs staged split")
    if f16:
        kc = oracle.f16_values(oracle.f16_bits(kc)).reshape(kc.shape)
        vc = oracle.f16_values(oracle.f16_bits(vc)).reshape(vc.shape)
    for r in (0, 1, rows // 2, rows - 1):
        want = oracle.attn_chunk(q[r:r + 1], kc, vc, h, hkv, pos0 + r, 1, hd, sc, window,
                                 threads=16)
        assert_close(a[r:r + 1], want, what=f"row {r}")


def test_raw_ws_launches(dev):
    """The _ws raw launches on a caller workspace give the recorder's bits; a workspace
    smaller than eb_attn_prefill_workspace_floats is refused; shapes that need none take a
    null workspace."""
    note("presplit raw _ws launches")
    h, hkv, hd, s = 16, 8, 128, 300
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 61), oracle.randn((s, hkv, hd), 62), oracle.randn((s, hkv, hd), 63)
    a, _ = recorder_and_raw_prefill(dev, q, k, v, h, hkv, s, hd, sc)
    need = eb.attn_prefill_workspace_floats(hkv, hd, 0, s)
    assert need == hkv * ((s + 31) // 32) * (16 * hd + 16) * 4
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    ws = upload(dev, np.full(need, np.nan, np.float32))  # contents need no initialisation
    ot = eb.Tensor.empty(dev, (s, h, hd))
    args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
            vt.numel(), ot.data_ptr, ot.numel(), h, hkv, s, hd, sc)
    eb.launch_attn_prefill_ws(*args, ws.data_ptr, need)
    dev.synchronize()
    assert_bitwise(ot.to_f32().reshape(s, h, hd), a, "raw _ws vs recorder")
    with pytest.raises(eb.ShapeMismatch):
        eb.launch_attn_prefill_ws(*args, ws.data_ptr, need - 1)
    # below the row threshold no workspace is needed
    assert eb.attn_prefill_workspace_floats(hkv, hd, 0, 100) == 0
    o2 = eb.Tensor.empty(dev, (100, h, hd))
    q2 = upload(dev, q[:100].copy())
    eb.launch_attn_prefill_ws(dev.stream, q2.data_ptr, q2.numel(), kt.data_ptr,
                              100 * hkv * hd, vt.data_ptr, 100 * hkv * hd, o2.data_ptr,
                              o2.numel(), h, hkv, 100, hd, sc, 0, 0)
    dev.synchronize()
    assert_bitwise(o2.to_f32().reshape(100, h, hd), a[:100], "no workspace needed")

    # chunk over f32 and f16 caches, windowed
    pos0, rows, window, max_seq = 300, 260, 100, 600
    kc, vc = oracle.randn((max_seq, hkv, hd), 64), oracle.randn((max_seq, hkv, hd), 65)
    qc = oracle.randn((rows, h, hd), 66)
    for f16 in (False, True):
        want, _ = chunk_pair(dev, qc, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16)
        need = eb.attn_prefill_workspace_floats(hkv, hd, pos0, rows, window)
        assert need == hkv * ((pos0 + rows + 31) // 32 - (pos0 - window + 1) // 32) * (16 * hd + 16) * 4
        if f16:
            kt = eb.Tensor.empty(dev, kc.shape, eb.DType.F16)
            vt = eb.Tensor.empty(dev, vc.shape, eb.DType.F16)
            rec = eb.Recorder(dev)
            eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
            eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
            rec.submit()
        else:
            kt, vt = upload(dev, kc), upload(dev, vc)
        qt = upload(dev, qc)
        ws = eb.Tensor.empty(dev, (need,))
        ot = eb.Tensor.empty(dev, (rows, h, hd))
        eb.launch_attn_prefill_chunk_ws(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr,
                                        kt.numel(), vt.data_ptr, vt.numel(), ot.data_ptr,
                                        ot.numel(), h, hkv, pos0, rows, hd, max_seq, sc, window,
                                        ws.data_ptr, need, f16=f16)
        dev.synchronize()
        assert_bitwise(ot.to_f32().reshape(rows, h, hd), want, f"chunk _ws f16={f16}")
