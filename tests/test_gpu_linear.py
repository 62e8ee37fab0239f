"""linear_f16w (the projections either side of attention) on the GPU against the oracle.

The oracle's linear_f16w follows the reference's CPU linear on f16-rounded weights
(crates/eyebrowse-kernels/src/testutil.rs:68-80, matmul.rs:255-272) and is pinned in
tests/test_oracle.py (float64, identity and one-hot closed forms, a planted transposed
weight). Outputs are held to the FP32 bar of tests/_gpu.py: the few-row kernel multiplies
in f32 on the halves, and the many-row kernel runs the matrix cores on an exact f16 split
of x, so only the summation order differs from the oracle.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, assert_close, note, upload

pytestmark = pytest.mark.gpu


def weight(dev, w, as_f16=False):
    """The reference's packed-u32 weight (Tensor::from_f16_packed), or an F16 tensor with
    the same bits (written by kv_write's f16 rounding, which is bit-exact; in_f % 4 == 0)."""
    if not as_f16:
        return eb.Tensor.from_f16_packed(dev, w.shape, w)
    out_f, in_f = w.shape
    t = eb.Tensor.empty(dev, (out_f, 1, in_f), eb.DType.F16)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, t, upload(dev, w), 1, out_f, in_f, out_f, 0)
    rec.submit()
    assert np.array_equal(np.frombuffer(t.read_bytes(), np.uint16), oracle.f16_bits(w).ravel())
    return t


def run(dev, x, w, m, in_f, out_f, as_f16=False):
    xt = upload(dev, x)
    wt = weight(dev, w, as_f16)
    ct = eb.Tensor.empty(dev, (m, out_f))
    rec = eb.Recorder(dev)
    eb.linear_f16w(rec, xt, wt, ct, m, in_f, out_f)
    rec.submit()
    return ct.to_f32().reshape(m, out_f)


def want_of(x, w, m, in_f, out_f):
    return oracle.linear_f16w(x, oracle.f16_bits(w), m, in_f, out_f, threads=16)


def test_reference_ramp_case(dev):
    """matmul.rs:255-272: m=5, in=33 (not a multiple of 8: the scalar kernel), out=7."""
    note("linear ramp")
    m, in_f, out_f = 5, 33, 7
    x = (np.arange(m * in_f) * 0.01 - 0.2).astype(np.float32).reshape(m, in_f)
    w = (np.arange(out_f * in_f) * 0.005 - 0.3).astype(np.float32).reshape(out_f, in_f)
    assert_close(run(dev, x, w, m, in_f, out_f), want_of(x, w, m, in_f, out_f), what="ramp")


@pytest.mark.parametrize("m,in_f,out_f", [
    (1, 1024, 2048),   # Qwen3 q_proj, decode
    (1, 2048, 1024),   # Qwen3 o_proj, decode
    (1, 4096, 1024),   # Mistral k_proj, decode
    (2, 1024, 1024),
    (3, 1024, 130),    # ragged feature count
    (5, 2560, 512),
    (8, 1024, 1024),   # largest few-row batch
    (1, 8, 5),         # one chunk per row
    (1, 1032, 7),      # contraction not a multiple of the lane stride
])
def test_few_rows_match_oracle(dev, m, in_f, out_f):
    note(f"linear gemv m={m} in={in_f} out={out_f}")
    x = oracle.randn((m, in_f), 1)
    w = oracle.randn((out_f, in_f), 2) * 0.05
    assert_close(run(dev, x, w, m, in_f, out_f), want_of(x, w, m, in_f, out_f),
                 what="gemv")


@pytest.mark.parametrize("m,in_f,out_f", [
    (9, 1024, 256),     # smallest matrix-core batch
    (64, 1024, 2048),   # Qwen3 q_proj, T=64
    (300, 1024, 1024),  # ragged rows
    (130, 4096, 136),   # ragged features, Mistral hidden
    (77, 2048, 1024),   # Qwen3 o_proj
    (33, 40, 48),       # contraction shorter than a stage
    (129, 264, 130),    # contraction not a multiple of the stage
])
def test_many_rows_match_oracle(dev, m, in_f, out_f):
    note(f"linear gemm m={m} in={in_f} out={out_f}")
    x = oracle.randn((m, in_f), 3)
    w = oracle.randn((out_f, in_f), 4) * 0.05
    assert_close(run(dev, x, w, m, in_f, out_f), want_of(x, w, m, in_f, out_f),
                 what="gemm")


def test_qwen_prompt_projection_sampled_rows(dev):
    """Qwen3 T=4096 q_proj (4096 x 1024 -> 2048), checked on sampled rows."""
    note("linear gemm qwen T=4096")
    m, in_f, out_f = 4096, 1024, 2048
    x = oracle.randn((m, in_f), 5)
    w = oracle.randn((out_f, in_f), 6) * 0.03
    got = run(dev, x, w, m, in_f, out_f)
    rows = [0, 1, 127, 128, 2049, 4094, 4095]
    want = want_of(x[rows], w, len(rows), in_f, out_f)
    assert_close(got[rows], want, what="qwen q_proj rows")


def test_qwen_o_proj_split_contraction(dev):
    """Qwen3 o_proj at T=4096 (4096 x 2048 -> 1024): one 128 x 128 tile per CU, so the
    contraction is cut in two halves whose partials add into the zeroed output. Sampled
    rows against the oracle, and a second launch bit-identical (two addends onto zero give
    the same bits in either order)."""
    note("linear gemm qwen o_proj T=4096 (split contraction)")
    m, in_f, out_f = 4096, 2048, 1024
    x = oracle.randn((m, in_f), 7)
    w = oracle.randn((out_f, in_f), 8) * 0.03
    got = run(dev, x, w, m, in_f, out_f)
    again = run(dev, x, w, m, in_f, out_f)
    assert_bitwise(again, got, "second launch")
    rows = [0, 1, 127, 128, 1000, 2049, 4094, 4095]
    want = want_of(x[rows], w, len(rows), in_f, out_f)
    assert_close(got[rows], want, what="qwen o_proj rows")


def test_row_scaling_extremes(dev):
    """Rows of very different magnitudes (1e-30 .. 1e30), a zero row, and rows holding inf
    or NaN: the split path scales each row by a power of two, so every finite row keeps
    f32 accuracy and a non-finite row stays non-finite without touching the others."""
    note("linear row scaling")
    m, in_f, out_f = 16, 256, 64
    x = oracle.randn((m, in_f), 7)
    mags = [1e-30, 1e-20, 1e-8, 1e-3, 1.0, 1e3, 1e8, 1e20, 1e30, 3e4, 7e4, 1e-38 * 16]
    for i, s in enumerate(mags):
        x[i] *= np.float32(s)
    x[12] = 0.0
    x[13, 5] = np.inf
    x[14, 9] = np.nan
    w = oracle.randn((out_f, in_f), 8) * 0.05
    got = run(dev, x, w, m, in_f, out_f)
    want = want_of(x, w, m, in_f, out_f)
    for i in list(range(12)) + [15]:
        scale = float(np.max(np.abs(want[i]))) or 1.0
        assert_close(got[i] / scale, want[i] / scale, what=f"row {i} (|x| ~ {mags[i] if i < 12 else 1})")
    assert np.array_equal(got[12], np.zeros(out_f, np.float32))
    assert not np.isfinite(got[13]).any() and not np.isfinite(got[14]).any()


def test_f16_tensor_weight_equals_packed_words(dev):
    note("linear f16 tensor weight")
    for m in (1, 40):
        x = oracle.randn((m, 512), 9)
        w = oracle.randn((96, 512), 10) * 0.05
        assert_bitwise(run(dev, x, w, m, 512, 96, as_f16=True), run(dev, x, w, m, 512, 96),
                       f"F16 vs U32 weight m={m}")


@pytest.mark.parametrize("m", [1, 4, 200])
def test_fused_qkv_equals_separate_projections(dev, m):
    """One launch for q/k/v (Qwen3 widths) gives the bits of three linear_f16w calls."""
    note(f"linear multi m={m}")
    in_f, outs = 1024, (2048, 1024, 1024)
    x = oracle.randn((m, in_f), 11)
    ws = [oracle.randn((o, in_f), 12 + i) * 0.05 for i, o in enumerate(outs)]
    xt = upload(dev, x)
    wts = [eb.Tensor.from_f16_packed(dev, w.shape, w) for w in ws]
    cs = [eb.Tensor.empty(dev, (m, o)) for o in outs]
    rec = eb.Recorder(dev)
    eb.linear_f16w_multi(rec, xt, wts, cs, outs, m, in_f)
    rec.submit()
    for i, o in enumerate(outs):
        sep = eb.Tensor.empty(dev, (m, o))
        rec = eb.Recorder(dev)
        eb.linear_f16w(rec, xt, wts[i], sep, m, in_f, o)
        rec.submit()
        assert_bitwise(cs[i].to_f32(), sep.to_f32(), f"projection {i}")
        assert_close(cs[i].to_f32().reshape(m, o), want_of(x, ws[i], m, in_f, o),
                     what=f"projection {i}")


@pytest.mark.parametrize("m", [1, 3])
def test_gemv_features_per_wave_same_bits(dev, m):
    """Outputs of 16384 features and more run four features per wave, shorter ones one:
    the first 1000 features of a 16384-feature launch equal, bit for bit, a launch of
    those 1000 rows alone (the same lanes, chunks and reduction per feature)."""
    note(f"linear gemv features per wave m={m}")
    in_f, big, small = 1024, 16384, 1000
    x = oracle.randn((m, in_f), 31)
    w = oracle.randn((big, in_f), 32) * 0.05
    got_big = run(dev, x, w, m, in_f, big)
    got_small = run(dev, x, np.ascontiguousarray(w[:small]), m, in_f, small)
    assert_bitwise(got_small, got_big[:, :small], "1000 features alone vs in a 16384 launch")
    assert_close(got_small, want_of(x, w[:small], m, in_f, small), what="gemv one per wave")


def test_raw_launch_with_workspace(dev):
    note("linear raw launch")
    m, in_f, out_f = 50, 1024, 320
    x = oracle.randn((m, in_f), 20)
    w = oracle.randn((out_f, in_f), 21) * 0.05
    xt = upload(dev, x)
    wt = eb.Tensor.from_f16_packed(dev, w.shape, w)
    ct = eb.Tensor.empty(dev, (m, out_f))
    need = eb.linear_workspace_floats(m, in_f)
    assert need > 0 and eb.linear_workspace_floats(1, in_f) == 0
    ws = upload(dev, np.full(need, np.nan, np.float32))
    eb.launch_linear_f16w(dev.stream, xt.data_ptr, xt.numel(), wt.data_ptr, 2 * wt.numel(),
                          ct.data_ptr, ct.numel(), m, in_f, out_f, ws.data_ptr, need)
    dev.synchronize()
    assert_close(ct.to_f32().reshape(m, out_f), want_of(x, w, m, in_f, out_f), what="raw")
    with pytest.raises(eb.ShapeMismatch):
        eb.launch_linear_f16w(dev.stream, xt.data_ptr, xt.numel(), wt.data_ptr,
                              2 * wt.numel(), ct.data_ptr, ct.numel(), m, in_f, out_f,
                              ws.data_ptr, need - 1)


def test_empty_and_invalid(dev):
    note("linear empty / invalid")
    x = upload(dev, oracle.randn((4, 16), 30))
    w = eb.Tensor.from_f16_packed(dev, (8, 16), oracle.randn((8, 16), 31))
    c = eb.Tensor.empty(dev, (4, 8))
    rec = eb.Recorder(dev)
    eb.linear_f16w(rec, x, w, c, 0, 16, 8)  # no rows: no-op
    with pytest.raises(eb.ShapeMismatch):
        eb.linear_f16w(rec, x, w, c, 4, 16, 9)  # weight too small
    with pytest.raises(eb.ShapeMismatch):
        eb.linear_f16w(rec, x, x, c, 4, 16, 8)  # f32 weight
    rec.submit()
    # in_f = 0: empty sums are zeros
    c2 = upload(dev, np.full((3, 5), 7.0, np.float32))
    w0 = eb.Tensor.empty(dev, (1,), eb.DType.F16)
    rec = eb.Recorder(dev)
    eb.linear_f16w(rec, x, w0, c2, 3, 0, 5)
    rec.submit()
    assert np.array_equal(c2.to_f32(), np.zeros(15, np.float32))


@pytest.mark.parametrize("m,outs", [
    (4096, (2048, 1024, 1024)),  # Qwen3 q/k/v at T=4096: wide 128 x 256 tiles
    (2000, (4096, 2000, 4000)),  # ragged rows and features on the wide tiles
])
def test_wide_tile_gemm_sampled_rows(dev, m, outs):
    """Grids with at least two wide tiles per CU take the 64 x 128-per-wave kernel; rows
    sampled across the tiles (first, last, tile edges) against the oracle."""
    note(f"linear wide gemm m={m} outs={outs}")
    in_f = 1024
    x = oracle.randn((m, in_f), 60)
    ws = [oracle.randn((o, in_f), 61 + i) * 0.03 for i, o in enumerate(outs)]
    xt = upload(dev, x)
    wts = [eb.Tensor.from_f16_packed(dev, w.shape, w) for w in ws]
    cs = [eb.Tensor.empty(dev, (m, o)) for o in outs]
    rec = eb.Recorder(dev)
    eb.linear_f16w_multi(rec, xt, wts, cs, outs, m, in_f)
    rec.submit()
    rows = sorted({0, 1, 127, 128, 129, m // 2, m - 129, m - 2, m - 1})
    for i, o in enumerate(outs):
        got = cs[i].to_f32().reshape(m, o)[rows]
        want = oracle.linear_f16w(x[rows], oracle.f16_bits(ws[i]), len(rows), in_f, o, threads=16)
        assert_close(got, want, what=f"projection {i}")
