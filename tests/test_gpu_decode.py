"""attn_decode on the GPU against the oracle (crates/eyebrowse-kernels/src/testutil.rs:
177-218 restated in oracle/oracle.c), at the reference's own test case and at every
BASELINE decode config (kv-write of the new token included)."""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_close, decode, note, upload
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
    assert kt.to_f32().tobytes() == kc2.tobytes()
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
    (64, 4, 128, 3000, 2999, None), # g = 16 (two 8-head workgroups per KV head)
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
    ws = eb.Tensor.empty(dev, (wsn,))
    eb.launch_attn_decode(dev.stream, qt.data_ptr, qt.numel(), kt.data_ptr, kt.numel(),
                          vt.data_ptr, vt.numel(), ot.data_ptr, ot.numel(), h, hkv, pos, hd, ms,
                          float(oracle.default_scale(hd)), ws.data_ptr, wsn, cus)
    dev.synchronize()
    want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, ms, threads=8)
    assert_close(ot.to_f32().reshape(h, hd), want, what="raw")


def test_repeated_calls_are_deterministic(dev):
    note("decode determinism")
    h, hkv, hd, ms, pos = 16, 8, 128, 9000, 8999
    q, kc, vc = oracle.randn((h, hd), 1), oracle.randn((ms, hkv, hd), 2), oracle.randn((ms, hkv, hd), 3)
    a = decode(dev, q, kc, vc, h, hkv, pos, hd, ms, 0.1)
    b = decode(dev, q, kc, vc, h, hkv, pos, hd, ms, 0.1)
    assert a.tobytes() == b.tobytes()
    assert rel_l2_f64(a, oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, ms, 0.1)) < 2e-5
