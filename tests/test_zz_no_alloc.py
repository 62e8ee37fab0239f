"""The no-allocation decode step (eb_launch_attn_decode_step_noalloc) on the GPU.

It runs the kernels of eb_launch_attn_decode_step with the split partials in the library's
static device scratch instead of a caller workspace. Same kernels, same split plan, so the
output and the new cache row must equal the workspace entry point's bit for bit. Two
calls run in a row, the second with a smaller shape (fewer keys and heads): the scratch
still holds the first call's partials when the second starts, and needs no clearing.
Each output is also held to the oracle (rel-L2 / max-abs bars of tests/_gpu.py).
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload

pytestmark = pytest.mark.gpu


def test_noalloc_decode_step_under_graph_capture(dev):
    """Graph capture is what the entry point is for: the no-allocation step captured into a
    HIP graph (first in this file, so that in a fresh process the capture holds the first
    decode launch) and replayed; every replay, with eager work and an eager no-allocation
    call of another shape between replays (which overwrites the scratch), must give the
    workspace entry point's output and cache row bit for bit."""
    H, Hkv, hd, max_seq, pos, seed = 16, 8, 128, 4096, 1500, 31
    scale = float(oracle.default_scale(hd))
    note(f"no-alloc decode step under capture H={H} Hkv={Hkv} hd={hd} pos={pos}")
    q = oracle.randn((H, hd), seed)
    kn = oracle.randn((1, Hkv, hd), seed + 1)
    vn = oracle.randn((1, Hkv, hd), seed + 2)
    fill_k = oracle.randn((max_seq, Hkv, hd), seed + 3)
    fill_v = oracle.randn((max_seq, Hkv, hd), seed + 4)
    qt, knt, vnt = upload(dev, q), upload(dev, kn), upload(dev, vn)
    kc_a, vc_a = upload(dev, fill_k), upload(dev, fill_v)
    kc_b, vc_b = upload(dev, fill_k), upload(dev, fill_v)
    o_a = eb.Tensor.empty(dev, (H, hd))
    o_b = eb.Tensor.empty(dev, (H, hd))
    cus = dev.cu_count
    args_b = (qt.data_ptr, qt.numel(), knt.data_ptr, vnt.data_ptr, knt.numel(), kc_b.data_ptr,
              kc_b.numel(), vc_b.data_ptr, vc_b.numel(), o_b.data_ptr, o_b.numel(), H, Hkv, pos,
              hd, max_seq, scale, cus)
    dev.begin_capture()
    try:
        eb.launch_attn_decode_step_noalloc(dev.stream, *args_b)
    finally:
        graph = dev.end_capture()
    need = eb.attn_decode_workspace_floats(H, Hkv, pos, hd, cus)
    ws = eb.Tensor.empty(dev, (max(need, 1),))
    eb.launch_attn_decode_step(dev.stream, qt.data_ptr, qt.numel(), knt.data_ptr, vnt.data_ptr,
                               knt.numel(), kc_a.data_ptr, kc_a.numel(), vc_a.data_ptr,
                               vc_a.numel(), o_a.data_ptr, o_a.numel(), H, Hkv, pos, hd, max_seq,
                               scale, ws.data_ptr, need, cus)
    dev.synchronize()
    want_o = o_a.to_f32()
    n = (pos + 1) * Hkv * hd
    want_k, want_v = kc_a.to_f32()[:n], vc_a.to_f32()[:n]
    for rep in range(3):
        graph.launch()
        dev.synchronize()
        assert_bitwise(o_b.to_f32(), want_o, f"replay {rep}: output")
        assert_bitwise(kc_b.to_f32()[:n], want_k, f"replay {rep}: K cache rows 0..=pos")
        assert_bitwise(vc_b.to_f32()[:n], want_v, f"replay {rep}: V cache rows 0..=pos")
        _step_both(dev, 32, 8, 128, 8192, 5000 + 1000 * rep, scale, 40 + rep)
    graph.release()
    kc_w = oracle.kv_write(fill_k, kn, Hkv, 1, hd, pos)
    vc_w = oracle.kv_write(fill_v, vn, Hkv, 1, hd, pos)
    want = oracle.attn_decode(q, kc_w, vc_w, H, Hkv, pos, hd, max_seq, scale, threads=16)
    assert_close(want_o.reshape(H, hd), want.reshape(H, hd), what="captured no-alloc vs oracle")


def _step_both(dev, H, Hkv, hd, max_seq, pos, scale, seed):
    """One decode step at `pos` through both entry points on two copies of the same
    caches; returns the workspace size the shape needs (floats)."""
    note(f"no-alloc decode step H={H} Hkv={Hkv} hd={hd} pos={pos}")
    q = oracle.randn((H, hd), seed)
    kn = oracle.randn((1, Hkv, hd), seed + 1)
    vn = oracle.randn((1, Hkv, hd), seed + 2)
    fill_k = oracle.randn((max_seq, Hkv, hd), seed + 3)
    fill_v = oracle.randn((max_seq, Hkv, hd), seed + 4)
    qt, knt, vnt = upload(dev, q), upload(dev, kn), upload(dev, vn)
    kc_a, vc_a = upload(dev, fill_k), upload(dev, fill_v)
    kc_b, vc_b = upload(dev, fill_k), upload(dev, fill_v)
    o_a = eb.Tensor.empty(dev, (H, hd))
    o_b = eb.Tensor.empty(dev, (H, hd))
    cus = dev.cu_count
    need = eb.attn_decode_workspace_floats(H, Hkv, pos, hd, cus)
    ws = eb.Tensor.empty(dev, (max(need, 1),))
    eb.launch_attn_decode_step(dev.stream, qt.data_ptr, qt.numel(), knt.data_ptr, vnt.data_ptr,
                               knt.numel(), kc_a.data_ptr, kc_a.numel(), vc_a.data_ptr,
                               vc_a.numel(), o_a.data_ptr, o_a.numel(), H, Hkv, pos, hd, max_seq,
                               scale, ws.data_ptr, need, cus)
    eb.launch_attn_decode_step_noalloc(dev.stream, qt.data_ptr, qt.numel(), knt.data_ptr,
                                       vnt.data_ptr, knt.numel(), kc_b.data_ptr, kc_b.numel(),
                                       vc_b.data_ptr, vc_b.numel(), o_b.data_ptr, o_b.numel(), H,
                                       Hkv, pos, hd, max_seq, scale, cus)
    dev.synchronize()
    assert_bitwise(o_b.to_f32(), o_a.to_f32(), "no-alloc vs workspace output")
    n = (pos + 1) * Hkv * hd
    assert_bitwise(kc_b.to_f32()[:n], kc_a.to_f32()[:n], "K cache rows 0..=pos")
    assert_bitwise(vc_b.to_f32()[:n], vc_a.to_f32()[:n], "V cache rows 0..=pos")
    kc_w = oracle.kv_write(fill_k, kn, Hkv, 1, hd, pos)
    vc_w = oracle.kv_write(fill_v, vn, Hkv, 1, hd, pos)
    want = oracle.attn_decode(q, kc_w, vc_w, H, Hkv, pos, hd, max_seq, scale, threads=16)
    assert_close(o_b.to_f32().reshape(H, hd), want.reshape(H, hd), what="no-alloc vs oracle")
    return need


def test_noalloc_decode_step_matches_the_workspace_entry_point(dev):
    """Mistral decode at 32768 keys, then a smaller Qwen-shaped step at pos 1000, then a
    Gemma-4 head_dim 256 step at scale 1.0."""
    limit = eb.attn_decode_noalloc_max_floats()
    need1 = _step_both(dev, 32, 8, 128, 32768, 32767, float(oracle.default_scale(128)), 1)
    need2 = _step_both(dev, 16, 8, 128, 4096, 1000, float(oracle.default_scale(128)), 11)
    assert 0 < need2 < need1 <= limit
    need3 = _step_both(dev, 16, 8, 256, 16384, 16383, 1.0, 21)
    assert 0 < need3 <= limit


def test_noalloc_refuses_shapes_beyond_the_scratch(dev):
    """A shape whose split partials exceed the static scratch is refused before any launch
    (64 query heads over one KV head, head_dim 256, 20001 keys planned for 4096 CUs)."""
    H, Hkv, hd, pos, cus = 64, 1, 256, 20000, 4096
    need = eb.attn_decode_workspace_floats(H, Hkv, pos, hd, cus)
    assert need > eb.attn_decode_noalloc_max_floats()
    with pytest.raises(eb.UnsupportedConfig):
        eb.launch_attn_decode_step_noalloc(dev.stream, 0, H * hd, 0, 0, Hkv * hd, 0,
                                           (pos + 1) * Hkv * hd, 0, (pos + 1) * Hkv * hd, 0,
                                           H * hd, H, Hkv, pos, hd, pos + 1, 1.0, cus)
    np.testing.assert_equal(eb.attn_decode_noalloc_max_floats(), 1 << 20)
