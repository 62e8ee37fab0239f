"""Greedy argmax and the whole-step HIP graph on the GPU.

argmax against the oracle's step-by-step restatement of the reference's 256-lane scan and
tree (crates/eyebrowse-kernels/src/sampling.rs:6-53), pinned in tests/test_oracle.py by
its closed form (tie order) and numpy on tie-free vectors; indices must be equal.

Graphs: an attention layer's decode step (projections, norms, RoPE, fused kv_write +
attention, o_proj, LM-head projection, argmax) captured once and replayed. Every replay
must give the bits the same step gives eagerly, with eager work between replays; an
update to the next position must give that position's eager bits.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, note, upload
from tests.test_oracle import signed_zero_cases

pytestmark = pytest.mark.gpu


def gpu_argmax(dev, x):
    x = np.ascontiguousarray(x, np.float32)
    lt = upload(dev, x) if x.size else eb.Tensor.empty(dev, (1,))
    out = eb.Tensor.from_u32(dev, (1,), [0xDEADBEEF])
    rec = eb.Recorder(dev)
    eb.argmax(rec, lt, out, x.size)
    rec.submit()
    return int(np.frombuffer(out.read_bytes(), np.uint32)[0])


def test_argmax_reference_case(dev):
    """sampling.rs:62-80."""
    note("argmax reference case")
    v = np.sin(np.arange(1000, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    v[731] = 5.0
    assert gpu_argmax(dev, v) == 731


def test_argmax_ties_and_specials(dev):
    note("argmax ties / specials")
    t = np.zeros(600, np.float32)
    t[1] = t[256] = t[513] = 2.0
    assert gpu_argmax(dev, t) == oracle.argmax(t) == 256
    t = np.zeros(300, np.float32)
    t[44] = t[116] = 1.0
    assert gpu_argmax(dev, t) == oracle.argmax(t) == 116
    for x in (np.array([np.nan, 2, np.nan, 1], np.float32), np.full(5, -np.inf, np.float32),
              np.array([-3.1e38, -3.3e38, np.nan], np.float32), np.array([7.0], np.float32),
              np.zeros(0, np.float32), np.array([-np.inf, np.inf, 1.0], np.float32)):
        assert gpu_argmax(dev, x) == oracle.argmax(x), x


def test_argmax_signed_zero_ties(dev):
    """-0.0 and +0.0 tie under the reference's strict `>` (sampling.rs:21,29): lane order
    decides. Pairs, a short all-nonpositive vector, and vocabularies of one slice (the
    one-launch path) and of several (two passes) with the zeros of both signs spread over
    lanes and slices."""
    note("argmax signed-zero ties")
    assert gpu_argmax(dev, np.array([-0.0, 0.0], np.float32)) == 0
    assert gpu_argmax(dev, np.array([0.0, -0.0], np.float32)) == 0
    for case in signed_zero_cases():
        assert gpu_argmax(dev, case) == oracle.argmax(case), case.size
    raw = np.full(10000, -2.0, np.float32)
    raw[4099], raw[5000], raw[9998] = -0.0, 0.0, -0.0  # winners in different slices
    assert gpu_argmax(dev, raw) == oracle.argmax(raw)


@pytest.mark.parametrize("vocab,seed", [(151936, 1), (262144, 2), (1001, 3), (4099, 4),
                                        (32000, 5), (5, 6), (4096, 7)])
def test_argmax_matches_oracle(dev, vocab, seed):
    """Qwen3 and Gemma vocab sizes, ragged sizes, one full slice (4096: the one-launch
    path), and heavy ties (values rounded to 0.5)."""
    note(f"argmax vocab={vocab}")
    x = oracle.randn((vocab,), seed)
    assert gpu_argmax(dev, x) == oracle.argmax(x)
    r = np.round(x * 2) / 2
    r[seed::11] = np.nan
    assert gpu_argmax(dev, r) == oracle.argmax(r)


def test_argmax_raw_launch(dev):
    note("argmax raw")
    x = oracle.randn((70000,), 9)
    lt = upload(dev, x)
    out = eb.Tensor.from_u32(dev, (1,), [0])
    need = eb.argmax_workspace_floats(x.size)
    ws = eb.Tensor.empty(dev, (need,))
    eb.launch_argmax(dev.stream, lt.data_ptr, lt.numel(), out.data_ptr, x.size, ws.data_ptr, need)
    dev.synchronize()
    assert int(np.frombuffer(out.read_bytes(), np.uint32)[0]) == oracle.argmax(x)
    with pytest.raises(eb.ShapeMismatch):
        eb.launch_argmax(dev.stream, lt.data_ptr, lt.numel(), out.data_ptr, x.size, ws.data_ptr,
                         need - 1)


# ---------------------------------------------------------------- graphs ---------------

H, HKV, HD, HIDDEN, VOCAB, MAX_SEQ = 16, 8, 128, 1024, 4096, 256


def _layer(dev):
    rnd = lambda shape, seed, s: oracle.randn(shape, seed) * np.float32(s)  # noqa: E731
    w = {n: eb.Tensor.from_f16_packed(dev, sh, rnd(sh, sd, 0.03))
         for n, sh, sd in (("q", (H * HD, HIDDEN), 1), ("k", (HKV * HD, HIDDEN), 2),
                           ("v", (HKV * HD, HIDDEN), 3), ("o", (HIDDEN, H * HD), 4),
                           ("lm", (VOCAB, HIDDEN), 5))}
    gq = upload(dev, (1 + 0.1 * oracle.randn((HD,), 6)).astype(np.float32))
    gk = upload(dev, (1 + 0.1 * oracle.randn((HD,), 7)).astype(np.float32))
    attn = eb.Attention(H, HKV, HD, float(oracle.default_scale(HD)), q_norm=gq, k_norm=gk,
                        q_proj=w["q"], k_proj=w["k"], v_proj=w["v"], o_proj=w["o"],
                        hidden=HIDDEN)
    return attn, w, (gq, gk)


def _step(dev, attn, lm, rope, kv, x, pos):
    """One decode step: attention layer, LM head, argmax. Returns (y, logits, idx)."""
    rec = eb.Recorder(dev)
    y = attn.forward(rec, x, rope, kv, 0, 1, pos)
    logits = eb.Tensor.empty(dev, (1, VOCAB))
    eb.linear_f16w(rec, y, lm, logits, 1, HIDDEN, VOCAB)
    idx = eb.Tensor.empty(dev, (1,), eb.DType.U32)
    eb.argmax(rec, logits, idx, VOCAB)
    rec.submit()
    return y, logits, idx


def _prompt(dev, attn, rope, kv, n):
    rec = eb.Recorder(dev)
    attn.forward(rec, upload(dev, oracle.randn((n, HIDDEN), 40)), rope, kv, 0, n, 0)
    rec.submit()


def test_decode_step_graph_replays_and_updates(dev):
    note("graph: capture decode step")
    attn, w, _keep = _layer(dev)
    rope = eb.Rope.build(dev, MAX_SEQ, HD, 1e6)
    kv_e = eb.KvCache.new(dev, 1, MAX_SEQ, HKV, HD)
    kv_g = eb.KvCache.new(dev, 1, MAX_SEQ, HKV, HD)
    _prompt(dev, attn, rope, kv_e, 100)
    _prompt(dev, attn, rope, kv_g, 100)
    x1 = oracle.randn((1, HIDDEN), 50)
    # eager reference (also sizes the device workspace and fills the pool)
    ye, le, ie = _step(dev, attn, w["lm"], rope, kv_e, upload(dev, x1), 100)
    ye, le, ie = ye.to_f32(), le.to_f32(), int(np.frombuffer(ie.read_bytes(), np.uint32)[0])
    assert ie == oracle.argmax(le)

    xg = upload(dev, x1)
    dev.begin_capture()
    try:
        yg, lg, ig = _step(dev, attn, w["lm"], rope, kv_g, xg, 100)
    finally:
        graph = dev.end_capture()
    for rep in range(3):
        graph.launch()
        assert_bitwise(yg.to_f32(), ye, f"replay {rep}: layer output")
        assert_bitwise(lg.to_f32(), le, f"replay {rep}: logits")
        assert int(np.frombuffer(ig.read_bytes(), np.uint32)[0]) == ie
        n = 101 * HKV * HD  # rows 0..=100; later rows are uninitialised in both caches
        assert_bitwise(kv_g.k[0].to_f32()[:n], kv_e.k[0].to_f32()[:n], f"replay {rep}: K cache")
        # eager work between replays, on the other cache
        _prompt(dev, attn, rope, eb.KvCache.new(dev, 1, MAX_SEQ, HKV, HD), 17)

    note("graph: update to the next position")
    x2 = oracle.randn((1, HIDDEN), 51)
    ye2, le2, ie2 = _step(dev, attn, w["lm"], rope, kv_e, upload(dev, x2), 101)
    xg.write(x2)
    dev.begin_capture()
    try:
        yg2, lg2, ig2 = _step(dev, attn, w["lm"], rope, kv_g, xg, 101)
    finally:
        graph = dev.end_capture(graph)
    for rep in range(2):
        graph.launch()
        assert_bitwise(yg2.to_f32(), ye2.to_f32(), f"updated replay {rep}: layer output")
        assert int(np.frombuffer(ig2.read_bytes(), np.uint32)[0]) == \
            int(np.frombuffer(ie2.read_bytes(), np.uint32)[0])
    n = 102 * HKV * HD
    assert_bitwise(kv_g.v[0].to_f32()[:n], kv_e.v[0].to_f32()[:n], "V cache after update")
    graph.release()


def test_capture_rules(dev):
    note("graph: capture rules")
    with pytest.raises(eb.EyebrowseError):
        dev.end_capture()  # nothing to end
    dev.begin_capture()
    try:
        with pytest.raises(eb.EyebrowseError):
            eb.Tensor.from_f32(dev, (4,), np.zeros(4, np.float32))  # host copy while capturing
        with pytest.raises(eb.EyebrowseError):
            dev.begin_capture()  # already capturing
    finally:
        g = dev.end_capture()
    g.launch()  # an empty graph runs
    dev.synchronize()
    g.release()


def test_graph_keeps_its_workspace_when_the_device_workspace_grows():
    """A captured step keeps the workspace buffer its kernels were captured with: eager work
    that grows the device workspace afterwards must neither free it (the replays would then
    write freed memory) nor change what the replays compute. Its own device, so that the
    workspace starts small (the session device's may already be large)."""
    note("graph: workspace growth between replays")
    d2 = eb.Device.new(0)
    attn, w, _keep = _layer(d2)
    rope = eb.Rope.build(d2, MAX_SEQ, HD, 1e6)
    kv_e = eb.KvCache.new(d2, 1, MAX_SEQ, HKV, HD)
    kv_g = eb.KvCache.new(d2, 1, MAX_SEQ, HKV, HD)
    _prompt(d2, attn, rope, kv_e, 100)
    _prompt(d2, attn, rope, kv_g, 100)
    x1 = oracle.randn((1, HIDDEN), 52)
    ye, le, ie = _step(d2, attn, w["lm"], rope, kv_e, upload(d2, x1), 100)
    ye, le = ye.to_f32(), le.to_f32()
    ie = int(np.frombuffer(ie.read_bytes(), np.uint32)[0])
    xg = upload(d2, x1)
    d2.begin_capture()
    try:
        yg, lg, ig = _step(d2, attn, w["lm"], rope, kv_g, xg, 100)
    finally:
        graph = d2.end_capture()
    graph.launch()
    assert_bitwise(lg.to_f32(), le, "replay before growth: logits")
    # A 1024-row prefill needs far more workspace (pre-split records, key-chunk partials)
    # than the decode step: the device workspace grows while the graph is alive.
    T = 1024
    q = oracle.randn((T, H, HD), 60)
    k = oracle.randn((T, HKV, HD), 61)
    v = oracle.randn((T, HKV, HD), 62)
    qt, kt, vt = upload(d2, q), upload(d2, k), upload(d2, v)
    ot = eb.Tensor.empty(d2, (T, H, HD))
    rec = eb.Recorder(d2)
    eb.attn_prefill(rec, qt, kt, vt, ot, H, HKV, T, HD, float(oracle.default_scale(HD)))
    rec.submit()
    o_first = ot.to_f32()
    # Fresh buffers allocated after the growth, NaN-filled: the replays must not touch them.
    sizes = (1024, 4096, 16384, 65536, 262144, 1 << 20)
    poison = [eb.Tensor.from_f32(d2, (n,), np.full(n, np.nan, np.float32)) for n in sizes]
    pbits = [p.read_bytes() for p in poison]
    for rep in range(3):
        graph.launch()
        assert_bitwise(yg.to_f32(), ye, f"replay {rep} after growth: layer output")
        assert_bitwise(lg.to_f32(), le, f"replay {rep} after growth: logits")
        assert int(np.frombuffer(ig.read_bytes(), np.uint32)[0]) == ie
        for p, b in zip(poison, pbits):
            assert p.read_bytes() == b, f"replay {rep} wrote a buffer allocated after the growth"
        # eager work on the grown workspace between replays still gives its own bits
        rec = eb.Recorder(d2)
        eb.attn_prefill(rec, qt, kt, vt, ot, H, HKV, T, HD, float(oracle.default_scale(HD)))
        rec.submit()
        assert_bitwise(ot.to_f32(), o_first, f"eager prefill after replay {rep}")
    graph.release()
    d2.synchronize()
