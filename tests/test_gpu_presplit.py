"""The prefill's workspace paths on the GPU: the pre-split pass and key chunks.

A prefill given a workspace (recorder launches use the device's; raw callers pass one to
the _ws launches) may
  - run the pre-split pass (head_dim 32..256, at least 3 query blocks, 2 at head_dim 256,
    share the keys): every key in range
    is split once into records that the attention kernel copies into LDS, where a plain
    raw launch (no workspace) splits while staging. Both hold the same values in LDS, so
    on shapes that are not cut into key chunks the outputs are equal bit for bit;
  - cut the key tiles of each query block into chunks, one workgroup each, merged by a
    second launch, when the query blocks alone give fewer than 128 workgroups. That
    changes the order of the sums, so chunked launches are checked against the oracle
    (attention.rs:94-120 / testutil.rs:130-172 restated in oracle/oracle.c) at the FP32 bar
    of tests/_gpu.py, and recorder and _ws launches (the same chunks) bit for bit.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload

pytestmark = pytest.mark.gpu


def run_prefill(dev, q, k, v, h, hkv, s, hd, sc, how):
    """how: "rec" (device workspace), "raw" (no workspace), "ws" (caller workspace)."""
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    o = eb.Tensor.empty(dev, (s, h, hd))
    args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
            vt.numel(), o.data_ptr, o.numel(), h, hkv, s, hd, sc)
    if how == "rec":
        rec = eb.Recorder(dev)
        eb.attn_prefill(rec, qt, kt, vt, o, h, hkv, s, hd, sc)
        rec.submit()
    elif how == "raw":
        eb.launch_attn_prefill(*args)
    else:
        need = eb.attn_prefill_workspace_floats(h, hkv, hd, 0, s)
        ws = upload(dev, np.full(max(need, 1), np.nan, np.float32))  # no initialisation needed
        eb.launch_attn_prefill_ws(*args, ws.data_ptr, need)
    dev.synchronize()
    return o.to_f32().reshape(s, h, hd)


def rows_check(got, q, k, v, h, hkv, s, hd, sc, starts=None):
    for r0 in starts or (0, s // 2, s - 40):
        n = min(40, s - r0)
        want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=(r0, n), threads=16)
        assert_close(got[r0:r0 + n], want[r0:r0 + n], what=f"rows {r0}+{n}")


# ------------------------------------------------------------- pre-split ------------

@pytest.mark.parametrize("h,hkv,s,hd", [
    (64, 32, 1024, 128),   # 2 heads x 2 blocks x 2 key splits per workgroup
    (128, 32, 1024, 128),  # 4 heads per workgroup, one record per step
    (64, 16, 1024, 128),   # 4 heads x 2 key splits (GQA 4 grid of one 4-wave round)
    (96, 32, 1024, 128),   # GQA 3: 1 head x 4 blocks x 2 key splits
    (128, 128, 512, 64),
    (128, 128, 512, 32),
    (64, 32, 1024, 256),   # head_dim 256: image records copied memory-to-LDS
    (128, 32, 512, 256),   # head_dim 256, 4 heads per workgroup
    (128, 128, 512, 256),  # head_dim 256, MHA: 4 query blocks per workgroup
])
def test_presplit_equals_staged_split(dev, h, hkv, s, hd):
    """Shapes with enough workgroups for no key chunks: the pre-split path gives the bits
    of the plain raw launch, which splits while staging."""
    note(f"presplit h={h} hkv={hkv} s={s} hd={hd}")
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 31), oracle.randn((s, hkv, hd), 32), oracle.randn((s, hkv, hd), 33)
    a = run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "rec")
    assert_bitwise(a, run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "raw"), "pre-split vs staged split")
    assert_bitwise(a, run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "ws"), "recorder vs _ws")
    rows_check(a, q, k, v, h, hkv, s, hd, sc, starts=(s - 40,))


@pytest.mark.parametrize("hd", [128, 256])
def test_special_rows(dev, hd):
    """Zero K/V rows (kept below every real exponent), rows of very different magnitudes,
    and an inf in one V row at key 224 (the first key of a tile, so no earlier query's wave
    reads it), through the pre-split path with key chunks (320 rows: 40 workgroups of
    blocks) and through the plain raw launch."""
    note(f"special rows hd={hd}")
    h, hkv, s = 16, 8, 320
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 41), oracle.randn((s, hkv, hd), 42), oracle.randn((s, hkv, hd), 43)
    k[5], v[7] = 0.0, 0.0
    k[100:110] *= np.float32(1e-20)
    v[120:130] *= np.float32(1e20)
    v[224, 3, 17] = np.inf
    want = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc, rows=(0, 224), threads=16)
    scale = np.abs(want[130:224]).max()
    for how in ("rec", "raw"):
        a = run_prefill(dev, q, k, v, h, hkv, s, hd, sc, how)
        assert_close(a[:120], want[:120], what=f"{how}: rows before the large V rows")
        assert_close(a[130:224] / scale, want[130:224] / scale, what=f"{how}: rows after them")
        assert not np.isfinite(a[224:, 6:8]).all()  # the heads of KV head 3 see the inf
        assert np.isfinite(a[224:, :6]).all() and np.isfinite(a[224:, 8:]).all()


# ------------------------------------------------------------- key chunks -----------

@pytest.mark.parametrize("h,hkv,s,hd,scale", [
    (16, 8, 512, 128, None),   # BASELINE config 3, T=512: 64 workgroups of blocks
    (8, 4, 1536, 128, None),   # fewer KV heads: 96 workgroups of blocks
    (32, 8, 400, 128, None),   # 4 heads per workgroup, ragged
    (16, 8, 512, 256, 1.0),    # head_dim 256
    (24, 8, 600, 64, None),    # GQA 3
    (4, 2, 300, 16, None),     # head_dim 16 (no f16 split), chunks without the pre-split pass
    (16, 8, 200, 128, None),   # below the pre-split threshold: chunks only
])
def test_chunked_prefill_matches_oracle(dev, h, hkv, s, hd, scale):
    note(f"chunked prefill h={h} hkv={hkv} s={s} hd={hd}")
    sc = float(oracle.default_scale(hd)) if scale is None else scale
    q, k, v = oracle.randn((s, h, hd), 51), oracle.randn((s, hkv, hd), 52), oracle.randn((s, hkv, hd), 53)
    assert eb.attn_prefill_workspace_floats(h, hkv, hd, 0, s) > 0
    a = run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "rec")
    assert np.isfinite(a).all()
    rows_check(a, q, k, v, h, hkv, s, hd, sc)
    assert_bitwise(a, run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "ws"), "recorder vs _ws")
    assert_bitwise(a, run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "rec"), "repeat")
    # the plain raw launch (no chunks, split while staging) agrees to the FP32 bar
    assert_close(a, run_prefill(dev, q, k, v, h, hkv, s, hd, sc, "raw"), what="raw vs chunked")


def chunk_run(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16, how):
    qt = upload(dev, q)
    if f16:
        kt = eb.Tensor.empty(dev, kc.shape, eb.DType.F16)
        vt = eb.Tensor.empty(dev, vc.shape, eb.DType.F16)
        rec = eb.Recorder(dev)
        eb.kv_write(rec, kt, upload(dev, kc), hkv, max_seq, hd, max_seq, 0)
        eb.kv_write(rec, vt, upload(dev, vc), hkv, max_seq, hd, max_seq, 0)
        rec.submit()
    else:
        kt, vt = upload(dev, kc), upload(dev, vc)
    o = eb.Tensor.empty(dev, (rows, h, hd))
    args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
            vt.numel(), o.data_ptr, o.numel(), h, hkv, pos0, rows, hd, max_seq, sc, window)
    if how == "rec":
        rec = eb.Recorder(dev)
        eb.attn_prefill_chunk(rec, qt, kt, vt, o, h, hkv, pos0, rows, hd, max_seq, sc, window)
        rec.submit()
    elif how == "raw":
        (eb.launch_attn_prefill_chunk_f16 if f16 else eb.launch_attn_prefill_chunk)(*args)
    else:
        need = eb.attn_prefill_workspace_floats(h, hkv, hd, pos0, rows, window)
        ws = eb.Tensor.empty(dev, (max(need, 1),))
        eb.launch_attn_prefill_chunk_ws(*args, ws.data_ptr, need, f16=f16)
    dev.synchronize()
    return o.to_f32().reshape(rows, h, hd)


@pytest.mark.parametrize("h,hkv,hd,pos0,rows,window,f16", [
    (16, 8, 128, 100, 300, 0, False),    # continuation, unaligned start
    (16, 8, 128, 4000, 128, 0, False),   # a short chunk over a long cache: many key chunks
    (32, 8, 128, 0, 256, 0, False),      # from position 0 through the chunk entry point
    (8, 1, 64, 0, 300, 50, False),       # windowed prompt
    (16, 8, 128, 300, 260, 100, False),  # windowed continuation: records start past tile 0
    (16, 8, 128, 70, 280, 0, True),      # f16 cache
    (24, 8, 128, 500, 300, 77, True),    # f16 cache, GQA 3, window
    (16, 8, 256, 100, 300, 0, False),    # head_dim 256 continuation
    (16, 8, 256, 3000, 64, 0, True),     # head_dim 256, f16 cache, short chunk, long cache
])
def test_chunk_entry_points(dev, h, hkv, hd, pos0, rows, window, f16):
    note(f"chunk h={h} hd={hd} pos0={pos0} rows={rows} window={window} f16={f16}")
    max_seq = pos0 + rows + 9
    sc = float(oracle.default_scale(hd))
    q = oracle.randn((rows, h, hd), 61)
    kc, vc = oracle.randn((max_seq, hkv, hd), 62), oracle.randn((max_seq, hkv, hd), 63)
    a = chunk_run(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16, "rec")
    assert_bitwise(a, chunk_run(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16,
                                "ws"), "recorder vs _ws")
    b = chunk_run(dev, q, kc, vc, h, hkv, pos0, rows, hd, max_seq, sc, window, f16, "raw")
    assert_close(a, b, what="raw vs workspace path")
    if f16:
        kc = oracle.f16_values(oracle.f16_bits(kc)).reshape(kc.shape)
        vc = oracle.f16_values(oracle.f16_bits(vc)).reshape(vc.shape)
    for r in (0, 1, rows // 2, rows - 1):
        want = oracle.attn_chunk(q[r:r + 1], kc, vc, h, hkv, pos0 + r, 1, hd, sc, window,
                                 threads=16)
        assert_close(a[r:r + 1], want, what=f"row {r}")


def test_workspace_sizes_and_refusal(dev):
    """Records plus chunk partials; a smaller workspace is refused; a shape that needs none
    (enough workgroups, too few rows for the pre-split pass) takes a null one."""
    note("workspace sizes")
    h, hkv, hd, s = 16, 8, 128, 300
    records = hkv * ((s + 31) // 32) * 4 * (16 * hd + 16)  # one record per (KV head, tile)
    need = eb.attn_prefill_workspace_floats(h, hkv, hd, 0, s)
    assert need > records  # 300 rows: 40 workgroups of blocks, so key chunks too
    sc = float(oracle.default_scale(hd))
    q, k, v = oracle.randn((s, h, hd), 71), oracle.randn((s, hkv, hd), 72), oracle.randn((s, hkv, hd), 73)
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    ot = eb.Tensor.empty(dev, (s, h, hd))
    ws = eb.Tensor.empty(dev, (need,))
    args = (dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(), vt.data_ptr,
            vt.numel(), ot.data_ptr, ot.numel(), h, hkv, s, hd, sc)
    with pytest.raises(eb.ShapeMismatch):
        eb.launch_attn_prefill_ws(*args, ws.data_ptr, need - 1)
    # 512 workgroups of 64-row blocks, two blocks only (too few to share a pre-split pass
    # at head_dim 128): no workspace at all
    h2, hkv2, s2 = 512, 256, 100
    assert eb.attn_prefill_workspace_floats(h2, hkv2, hd, 0, s2) == 0
    q2 = upload(dev, oracle.randn((s2, h2, hd), 74))
    k2, v2 = upload(dev, oracle.randn((s2, hkv2, hd), 75)), upload(dev, oracle.randn((s2, hkv2, hd), 76))
    o2, o3 = eb.Tensor.empty(dev, (s2, h2, hd)), eb.Tensor.empty(dev, (s2, h2, hd))
    a2 = (dev.stream, q2.data_ptr, q2.numel(), k2.data_ptr, k2.numel(), v2.data_ptr, v2.numel())
    eb.launch_attn_prefill_ws(*a2, o2.data_ptr, o2.numel(), h2, hkv2, s2, hd, sc, 0, 0)
    eb.launch_attn_prefill(*a2, o3.data_ptr, o3.numel(), h2, hkv2, s2, hd, sc)
    dev.synchronize()
    assert_bitwise(o2.to_f32(), o3.to_f32(), "no workspace needed")
