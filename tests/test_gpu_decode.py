"""attn_decode on the GPU against the oracle (crates/eyebrowse-kernels/src/testutil.rs:
177-218 restated in oracle/oracle.c), at the reference's own test case and at every
BASELINE decode config (kv-write of the new token included)."""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, decode, note, upload
from tests._textbook import ramp, rel_l2_f64

pytestmark = pytest.mark.gpu


def test_reference_ramp_case(dev):
    """attention.rs:205-233: h=4, hkv=2, hd=8, max_seq=16, pos=5, ramp inputs; the
    reference asserts rel_l2 < 1e-4 against the CPU oracle."""
    note("decode reference ramp case")
    h, hkv, hd, max_seq, pos = 4, 2, 8, 16, 5
    q = ramp(h * hd, -0.4, 0.02)
    kc = ramp(hkv * max_seq * hd, -0.2, 0.005)
    vc = ramp(hkv * max_seq * hd, 0.1, 0.009)
    got = decode(dev, q.reshape(h, hd), kc.reshape(max_seq, hkv, hd), vc.reshape(max_seq, hkv, hd),
                 h, hkv, pos, hd, max_seq, 1 / np.sqrt(np.float32(hd)))
    want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, max_seq)
    assert oracle.rel_l2(got, want) < 1e-4
    assert_close(got, want, what="ramp")


def test_golden_fixture(dev):
    g = np.load("tests/golden/qwen_decode_small.npz", allow_pickle=False)
    H, Hkv, hd, ms, pos = (int(g[x]) for x in ("H", "Hkv", "hd", "max_seq", "pos"))
    note(f"decode golden H={H} pos={pos}")
    got = decode(dev, oracle.randn((H, hd), 1), oracle.randn((ms, Hkv, hd), 2),
                 oracle.randn((ms, Hkv, hd), 3), H, Hkv, pos, hd, ms, float(g["scale"]))
    assert_close(got, g["o"], what="golden decode")


def _decode_step(dev, h, hkv, hd, max_seq, pos, scale, seed=1):
    """Cache rows 0..pos-1 random, the new token's K/V written at pos by kv_write, then
    decode over pos+1 keys (one decode step of attention.rs:149-183)."""
    kc = oracle.randn((max_seq, hkv, hd), seed + 1)
    vc = oracle.randn((max_seq, hkv, hd), seed + 2)
    knew = oracle.randn((1, hkv, hd), seed + 3)
    vnew = oracle.randn((1, hkv, hd), seed + 4)
    q = oracle.randn((h, hd), seed)
    kt, vt = upload(dev, kc), upload(dev, vc)
    knt, vnt, qt = upload(dev, knew), upload(dev, vnew), upload(dev, q)
    ot = eb.Tensor.empty(dev, (1, h * hd))
    rec = eb.Recorder(dev)
    eb.kv_write(rec, kt, knt, hkv, 1, hd, max_seq, pos)
    eb.kv_write(rec, vt, vnt, hkv, 1, hd, max_seq, pos)
    eb.attn_decode(rec, qt, kt, vt, ot, h, hkv, pos, hd, max_seq, scale)
    rec.submit()
    kc2 = oracle.kv_write(kc, knew, hkv, 1, hd, pos)
    vc2 = oracle.kv_write(vc, vnew, hkv, 1, hd, pos)
    assert_bitwise(kt.to_f32(), kc2, "cache after kv_write")
    want = oracle.attn_decode(q, kc2, vc2, h, hkv, pos, hd, max_seq, scale, threads=8)
    return ot.to_f32().reshape(h, hd), want


@pytest.mark.parametrize("L", [512, 2048, 4096, 8191])
def test_qwen_decode_config(dev, L):
    """Qwen3 16/8 heads, hd 128, max_seq 8192, new token at pos L."""
    note(f"decode qwen L={L}")
    got, want = _decode_step(dev, 16, 8, 128, 8192, L, float(oracle.default_scale(128)))
    assert_close(got, want, what=f"qwen L={L}")


@pytest.mark.parametrize("pos", [8192, 32767])
def test_mistral_decode_config(dev, pos):
    """Mistral 32/8 heads, max_seq 32768, 8193 and 32768 keys."""
    note(f"decode mistral pos={pos}")
    got, want = _decode_step(dev, 32, 8, 128, 32768, pos, float(oracle.default_scale(128)))
    assert_close(got, want, what=f"mistral pos={pos}")


@pytest.mark.parametrize("h,hkv,hd,max_seq,pos,scale", [
    (4, 2, 8, 16, 0, 0.35),         # one key: o = v[0]
    (16, 8, 128, 100, 63, None),
    (16, 16, 64, 1000, 999, None),  # MHA
    (24, 8, 128, 700, 650, None),   # g = 3 (three single-head workgroups per KV head)
    (64, 4, 128, 3000, 2999, None), # g = 16 (four 4-head workgroups per KV head)
    (8, 1, 256, 5000, 4321, 1.0),   # scale 1.0, hd 256
    (8, 8, 32, 300, 255, 0.0),      # scale 0: mean of V
    (2, 1, 4, 70, 69, None),
    (2, 2, 16, 130, 128, None),
])
def test_shapes(dev, h, hkv, hd, max_seq, pos, scale):
    note(f"decode h={h} hkv={hkv} hd={hd} max_seq={max_seq} pos={pos} scale={scale}")
    sc = float(oracle.default_scale(hd)) if scale is None else scale
    q = oracle.randn((h, hd), 1)
    kc = oracle.randn((max_seq, hkv, hd), 2)
    vc = oracle.randn((max_seq, hkv, hd), 3)
    got = decode(dev, q, kc, vc, h, hkv, pos, hd, max_seq, sc)
    want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, max_seq, sc)
    assert_close(got, want, what="shape")
    if pos == 0:
        g = h // hkv
        np.testing.assert_array_equal(got, np.repeat(vc[0], g, axis=0))


def test_raw_launch_with_caller_workspace(dev):
    """eb_launch_attn_decode on caller memory with the workspace size the ABI reports."""
    note("decode raw launch")
    h, hkv, hd, ms, pos = 32, 8, 128, 20000, 19999
    q = oracle.randn((h, hd), 4)
    kc = oracle.randn((ms, hkv, hd), 5)
    vc = oracle.randn((ms, hkv, hd), 6)
    qt, kt, vt = upload(dev, q), upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    cus = dev.cu_count
    wsn = eb.attn_decode_workspace_floats(h, hkv, pos, hd, cus)
    assert wsn > 0
    # the workspace needs no initialisation: fill it with NaN first
    ws = upload(dev, np.full(wsn, np.nan, np.float32))
    want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, ms, threads=8)
    for _ in range(2):
        eb.launch_attn_decode(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                              vt.data_ptr, vt.numel(), ot.data_ptr, ot.numel(), h, hkv, pos, hd,
                              ms, float(oracle.default_scale(hd)), ws.data_ptr, wsn, cus)
        dev.synchronize()
        assert_close(ot.to_f32().reshape(h, hd), want, what="raw")


def test_shrinking_shapes_share_the_device_workspace(dev):
    """Decode calls of decreasing size on one device reuse its grow-only workspace: a
    smaller shape must not pick up a larger shape's leftovers."""
    note("decode shrinking shapes")
    for h, hkv, hd, ms, pos in [(32, 8, 128, 32768, 32767), (16, 8, 256, 9000, 8999),
                                (16, 8, 128, 4096, 4095), (8, 8, 64, 3000, 2999),
                                (24, 8, 128, 700, 650), (4, 2, 8, 600, 599)]:
        q, kc, vc = oracle.randn((h, hd), 1), oracle.randn((ms, hkv, hd), 2), oracle.randn((ms, hkv, hd), 3)
        got = decode(dev, q, kc, vc, h, hkv, pos, hd, ms, 0.1)
        want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, ms, 0.1, threads=8)
        assert_close(got, want, what=f"h={h} hd={hd} pos={pos}")


@pytest.mark.parametrize("h,hkv,hd,max_seq,pos", [
    (16, 8, 128, 8192, 8191),
    (32, 8, 128, 32768, 20000),
    (16, 8, 256, 16384, 16383),
    (4, 2, 8, 16, 5),
    (4, 2, 8, 16, 0),
])
def test_fused_step_equals_kv_write_then_decode(dev, h, hkv, hd, max_seq, pos):
    """eb_attn_decode_step == kv_write(K), kv_write(V), attn_decode (attention.rs:149-183):
    same cache bytes; the same output up to f32 rounding (the fused step folds key `pos`
    in after the cached keys, the separate calls fold it in with its chunk)."""
    note(f"decode step h={h} hd={hd} pos={pos}")
    sc = float(oracle.default_scale(hd))
    kc = oracle.randn((max_seq, hkv, hd), 2)
    vc = oracle.randn((max_seq, hkv, hd), 3)
    knew, vnew = oracle.randn((1, hkv, hd), 4), oracle.randn((1, hkv, hd), 5)
    q = oracle.randn((h, hd), 1)
    qt, knt, vnt = upload(dev, q), upload(dev, knew), upload(dev, vnew)
    k1, v1, k2, v2 = upload(dev, kc), upload(dev, vc), upload(dev, kc), upload(dev, vc)
    o1, o2 = eb.Tensor.empty(dev, (h, hd)), eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.kv_write(rec, k1, knt, hkv, 1, hd, max_seq, pos)
    eb.kv_write(rec, v1, vnt, hkv, 1, hd, max_seq, pos)
    eb.attn_decode(rec, qt, k1, v1, o1, h, hkv, pos, hd, max_seq, sc)
    eb.attn_decode_step(rec, qt, knt, vnt, k2, v2, o2, h, hkv, pos, hd, max_seq, sc)
    rec.submit()
    assert_bitwise(k2.to_f32(), k1.to_f32(), "K cache")
    assert_bitwise(v2.to_f32(), v1.to_f32(), "V cache")
    assert_close(o2.to_f32(), o1.to_f32(), what="step vs separate calls")
    want = oracle.attn_decode(q, oracle.kv_write(kc, knew, hkv, 1, hd, pos),
                              oracle.kv_write(vc, vnew, hkv, 1, hd, pos), h, hkv, pos, hd,
                              max_seq, sc, threads=8)
    assert_close(o2.to_f32().reshape(h, hd), want, what="step")


@pytest.mark.parametrize("h,hkv,hd", [(32, 8, 128), (16, 8, 128), (16, 8, 256)])
@pytest.mark.parametrize("pos", [1023, 1024, 1025, 1039, 1040, 1551])
def test_fused_step_at_split_dealing_edges(dev, h, hkv, hd, pos):
    """The split pass deals keys to the splits in superblocks of one step of each wave (16
    rows at these shapes). The fused step at positions on and around superblock edges
    (the last superblock partial or empty, the split that folds key `pos` changing) against
    the oracle, with cache rows 0..=pos bit-exact."""
    max_seq = 2048
    note(f"decode step edges h={h} hkv={hkv} hd={hd} pos={pos}")
    sc = float(oracle.default_scale(hd))
    kc = oracle.randn((max_seq, hkv, hd), 12)
    vc = oracle.randn((max_seq, hkv, hd), 13)
    knew, vnew = oracle.randn((1, hkv, hd), 14), oracle.randn((1, hkv, hd), 15)
    q = oracle.randn((h, hd), 11)
    qt, knt, vnt = upload(dev, q), upload(dev, knew), upload(dev, vnew)
    kt, vt = upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode_step(rec, qt, knt, vnt, kt, vt, ot, h, hkv, pos, hd, max_seq, sc)
    rec.submit()
    kw = oracle.kv_write(kc, knew, hkv, 1, hd, pos)
    vw = oracle.kv_write(vc, vnew, hkv, 1, hd, pos)
    n = (pos + 1) * hkv * hd
    assert_bitwise(kt.to_f32()[:n], kw.reshape(-1)[:n], "K cache rows 0..=pos")
    assert_bitwise(vt.to_f32()[:n], vw.reshape(-1)[:n], "V cache rows 0..=pos")
    want = oracle.attn_decode(q, kw, vw, h, hkv, pos, hd, max_seq, sc, threads=8)
    assert_close(ot.to_f32().reshape(h, hd), want, what=f"step at pos {pos}")


def test_sequence_of_steps_reuses_the_workspace(dev):
    """A decode loop (positions 0..N-1 through the fused step) on one device workspace;
    each step matches the oracle, so the split counters reset correctly every launch."""
    note("decode loop")
    h, hkv, hd, max_seq = 16, 8, 128, 4096
    kc = eb.Tensor.empty(dev, (max_seq, hkv, hd))
    vc = eb.Tensor.empty(dev, (max_seq, hkv, hd))
    kall = oracle.randn((max_seq, hkv, hd), 7)
    vall = oracle.randn((max_seq, hkv, hd), 8)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, kc, upload(dev, kall), hkv, 3000, hd, max_seq, 0)
    eb.kv_write(rec, vc, upload(dev, vall), hkv, 3000, hd, max_seq, 0)
    rec.submit()
    for pos in (3000, 3001, 3002, 3500, 4095):
        q = oracle.randn((h, hd), pos)
        o = eb.Tensor.empty(dev, (h, hd))
        rec = eb.Recorder(dev)
        eb.attn_decode_step(rec, upload(dev, q), upload(dev, kall[pos:pos + 1]),
                            upload(dev, vall[pos:pos + 1]), kc, vc, o, h, hkv, pos, hd, max_seq, 0.09)
        rec.submit()
        # decode at pos reads rows 0..pos only, all of which the cache holds by now
        want = oracle.attn_decode(q, kall, vall, h, hkv, pos, hd, max_seq, 0.09, threads=8)
        assert_close(o.to_f32().reshape(h, hd), want, what=f"pos {pos}")
        gap = {3002: (3003, 3500), 3500: (3501, 4095)}.get(pos)
        if gap:  # fill the rows the loop skips
            a, b = gap
            rec = eb.Recorder(dev)
            eb.kv_write(rec, kc, upload(dev, kall[a:b]), hkv, b - a, hd, max_seq, a)
            eb.kv_write(rec, vc, upload(dev, vall[a:b]), hkv, b - a, hd, max_seq, a)
            rec.submit()


def test_repeated_calls_are_deterministic(dev):
    note("decode determinism")
    h, hkv, hd, ms, pos = 16, 8, 128, 9000, 8999
    q, kc, vc = oracle.randn((h, hd), 1), oracle.randn((ms, hkv, hd), 2), oracle.randn((ms, hkv, hd), 3)
    a = decode(dev, q, kc, vc, h, hkv, pos, hd, ms, 0.1)
    b = decode(dev, q, kc, vc, h, hkv, pos, hd, ms, 0.1)
    assert_bitwise(a, b, "repeat")
    assert rel_l2_f64(a, oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, ms, 0.1)) < 2e-5
